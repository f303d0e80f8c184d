// Router of the sparse-MoE block on gfx950: fp32 logits, softmax, top-k,
// renormalised weights.
//
// Replaces, from Qwen35MoeBlock::forward
// (crates/mlxr-lm/src/qwen3_5/text/moe.rs:117-138):
//   gate.forward(x)            Linear::forward, layers/linear.rs:91-95
//   shared_expert_gate(x)      same, one extra output row (moe.rs:118)
//   softmax_axis(.., precise)  ops/arithmetic.rs:1298-1311
//   argpartition_axis(-K)      ops/sort.rs:211-226 (+ slice, moe.rs:128-132)
//   take_along_axis/sum/divide moe.rs:136-138
//
// Logits are computed with a fixed summation order (per lane: fmaf over
// elements j = 4l + 256i + c in (i, c) order; across lanes: butterfly
// v += v[l^m], m = 32..1; then + bias[e] when the router has one) so the
// selected expert sets reproduce bit for bit on the CPU.  Selection is on logits (softmax is monotone), descending,
// ties to the lower expert id.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {
namespace {

// One wave computes EB logit columns for up to TB tokens of a token block.
// Router weights stream as float4 (16 B per lane), x as 4 bf16 (8 B).
template <int EB, int TB>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, int T, int d, const float* __restrict__ w,
    const float* __restrict__ bias, int E, const float* __restrict__ w_extra,
    float* __restrict__ logits, int64_t ld) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int e_tot = E + (w_extra ? 1 : 0);
  const int e0 = (blockIdx.x * 4 + wave) * EB;
  if (e0 >= e_tot) return;
  const int t0 = blockIdx.y * TB;
  const int nt = min(TB, T - t0);

  const float* wrow[EB];
#pragma unroll
  for (int q = 0; q < EB; ++q) {
    const int e = e0 + q;
    wrow[q] = e < E ? w + (int64_t)e * d : (e == E ? w_extra : nullptr);
  }
  float acc[EB][TB];
#pragma unroll
  for (int q = 0; q < EB; ++q)
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) acc[q][tt] = 0.0f;

  for (int j = 4 * lane; j < d; j += 256) {
    float4 wv[EB];
#pragma unroll
    for (int q = 0; q < EB; ++q)
      wv[q] = wrow[q] ? *reinterpret_cast<const float4*>(wrow[q] + j)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      if (tt < nt) {
        const uint2 xv = *reinterpret_cast<const uint2*>(
            x + (int64_t)(t0 + tt) * d + j);
        const float x0 = __uint_as_float(xv.x << 16);
        const float x1 = __uint_as_float(xv.x & 0xffff0000u);
        const float x2 = __uint_as_float(xv.y << 16);
        const float x3 = __uint_as_float(xv.y & 0xffff0000u);
#pragma unroll
        for (int q = 0; q < EB; ++q) {
          float a = acc[q][tt];
          a = __builtin_fmaf(x0, wv[q].x, a);
          a = __builtin_fmaf(x1, wv[q].y, a);
          a = __builtin_fmaf(x2, wv[q].z, a);
          a = __builtin_fmaf(x3, wv[q].w, a);
          acc[q][tt] = a;
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < EB; ++q) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      if (tt < nt) {
        float v = wave_sum_butterfly(acc[q][tt]);
        if (bias && e0 + q < E) v += bias[e0 + q];
        if (lane == 0 && e0 + q < e_tot)
          logits[(int64_t)(t0 + tt) * ld + e0 + q] = v;
      }
    }
  }
}

// One wave per token.  Lane l holds experts l + 64s.  Result k lives in
// lane k until it is written.
template <int SLOTS>
__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, int64_t ld, int T, int E, int K,
    int32_t* __restrict__ idx, float* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float v[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const int e = lane + 64 * s;
    v[s] = e < E ? logits[(int64_t)t * ld + e] : -INFINITY;
  }
  uint32_t taken = 0;
  int my_idx = 0;
  float my_val = 0.0f, m = 0.0f;
  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int e = lane + 64 * s;
      if (e < E && !((taken >> s) & 1u)) {
        if (v[s] > bv || (v[s] == bv && e < bi)) {
          bv = v[s];
          bi = e;
        }
      }
    }
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) {
      const float ov = __shfl_xor(bv, msk, 64);
      const int oi = __shfl_xor(bi, msk, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    if (lane == k) {
      my_idx = bi;
      my_val = bv;
    }
    if (k == 0) m = bv;
  }
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s)
    if (lane + 64 * s < E) acc += expf(v[s] - m);
  const float S = wave_sum_butterfly(acc);
  const float p = lane < K ? expf(my_val - m) / S : 0.0f;
  float psum = 0.0f;
  for (int k = 0; k < K; ++k) psum += __shfl(p, k, 64);
  if (lane < K) {
    idx[(int64_t)t * K + lane] = my_idx;
    wts[(int64_t)t * K + lane] = p / psum;
  }
}

// Full ascending sort of each row (value, then index): a valid
// argpartition for every kth.  Bitonic network in LDS, P = pow2 >= n.
__global__ __launch_bounds__(1024) void argsort_rows_kernel(
    const float* __restrict__ a, int n, int P, uint32_t* __restrict__ out) {
  extern __shared__ char smem[];
  float* kv = reinterpret_cast<float*>(smem);
  int* ki = reinterpret_cast<int*>(kv + P);
  const int64_t row = blockIdx.x;
  for (int i = threadIdx.x; i < P; i += blockDim.x) {
    kv[i] = i < n ? a[row * n + i] : INFINITY;
    ki[i] = i;
  }
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const bool asc = (i & k) == 0;
          const float a0 = kv[i], a1 = kv[ixj];
          const int i0 = ki[i], i1 = ki[ixj];
          const bool gt = a0 > a1 || (a0 == a1 && i0 > i1);
          if (gt == asc) {
            kv[i] = a1;
            kv[ixj] = a0;
            ki[i] = i1;
            ki[ixj] = i0;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x)
    out[row * n + i] = (uint32_t)ki[i];
}

__global__ __launch_bounds__(256) void softmax_rows_kernel(
    const float* __restrict__ a, int n, float* __restrict__ out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float* r = a + row * n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, r[i]);
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1)
    mx = fmaxf(mx, __shfl_xor(mx, msk, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) sum += expf(r[i] - mx);
  sum = wave_sum_butterfly(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = (red[0] + red[1]) + (red[2] + red[3]);
  for (int i = threadIdx.x; i < n; i += 256)
    out[row * n + i] = expf(r[i] - mx) / sum;
}

}  // namespace

hipError_t launch_router_logits(const uint16_t* x, int64_t T, int64_t d,
                                const float* w, const float* bias, int64_t E,
                                const float* w_extra, float* logits,
                                int64_t ld, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const int64_t e_tot = E + (w_extra ? 1 : 0);
  // Few tokens: one logit column per wave so the 4*d*E bytes of router
  // weights spread over E/4 workgroups.  Many tokens: 4 columns x 16
  // tokens per wave for register reuse of both operands.
  ProfileScope prof("router_logits", s);
  if (T <= 16) {
    const dim3 grid((unsigned)((e_tot + 3) / 4), 1);
    router_logits_kernel<1, 16><<<grid, 256, 0, s>>>(
        x, (int)T, (int)d, w, bias, (int)E, w_extra, logits, ld);
  } else {
    const dim3 grid((unsigned)((e_tot + 15) / 16), (unsigned)((T + 15) / 16));
    router_logits_kernel<4, 16><<<grid, 256, 0, s>>>(
        x, (int)T, (int)d, w, bias, (int)E, w_extra, logits, ld);
  }
  return hipGetLastError();
}

hipError_t launch_router_topk(const float* logits, int64_t ld, int64_t T,
                              int64_t E, int64_t K, int32_t* idx, float* wts,
                              hipStream_t s) {
  if (T == 0) return hipSuccess;
  ProfileScope prof("router_topk", s);
  const dim3 grid((unsigned)((T + 3) / 4));
  const int slots = (int)((E + 63) / 64);
#define MLXR_TOPK(S)                                                     \
  router_topk_kernel<S><<<grid, 256, 0, s>>>(logits, ld, (int)T, (int)E, \
                                             (int)K, idx, wts)
  if (slots <= 1)
    MLXR_TOPK(1);
  else if (slots <= 2)
    MLXR_TOPK(2);
  else if (slots <= 4)
    MLXR_TOPK(4);
  else if (slots <= 8)
    MLXR_TOPK(8);
  else
    MLXR_TOPK(16);
#undef MLXR_TOPK
  return hipGetLastError();
}

hipError_t launch_argsort_rows(const float* a, int64_t rows, int64_t n,
                               uint32_t* out, hipStream_t s) {
  if (rows == 0 || n == 0) return hipSuccess;
  int P = 1;
  while (P < n) P <<= 1;
  argsort_rows_kernel<<<(unsigned)rows, 1024, (size_t)P * 8, s>>>(a, (int)n,
                                                                   P, out);
  return hipGetLastError();
}

hipError_t launch_softmax_rows(const float* a, int64_t rows, int64_t n,
                               float* out, hipStream_t s) {
  if (rows == 0 || n == 0) return hipSuccess;
  softmax_rows_kernel<<<(unsigned)rows, 256, 0, s>>>(a, (int)n, out);
  return hipGetLastError();
}

}  // namespace mlxr_moe
