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
// selected expert sets reproduce bit for bit on the CPU.  Selection is on
// logits (softmax is monotone), descending, ties to the lower expert id.
//
// The router may also be a QuantizedLinear (QuantizedLinear::forward,
// crates/mlxr/src/layers/quantized.rs:356-373; the shipped Qwen3.6
// checkpoints quantise mlp.gate and mlp.shared_expert_gate at 8 bits, group
// 64, qwen3_5/text/moe.rs:255-284).  Then element j's weight is the f32
// fmaf(code_j, scale, bias) of its group, the same lane order applies, and
// the logit is rounded to bf16 (the reference's result dtype with bf16 x
// and scales); the selection is then on the bf16 probabilities
// (wave_topk).
#include "common.hpp"
#include "kernels.hpp"
#include "route.hpp"

namespace mlxr_moe {
namespace {

// One router weight row: f32 values, or packed codes with their group
// scales and biases.  w == nullptr: no row (zeros).
struct WRow {
  const void* w;
  const uint16_t* s;
  const uint16_t* b;
};

template <int BITS>
__device__ __forceinline__ WRow router_row(const RouterWeights& rw, int e,
                                           int E, int d) {
  if (e < E) {
    if (BITS == 0)
      return {static_cast<const float*>(rw.w) + (int64_t)e * d, nullptr, nullptr};
    if (BITS == 16)
      return {static_cast<const uint16_t*>(rw.w) + (int64_t)e * d, nullptr, nullptr};
    return {static_cast<const uint8_t*>(rw.w) + (int64_t)e * d * BITS / 8,
            rw.scales + (int64_t)e * (d / 64), rw.biases + (int64_t)e * (d / 64)};
  }
  if (e == E && rw.w_extra) return {rw.w_extra, rw.scales_extra, rw.biases_extra};
  return {nullptr, nullptr, nullptr};
}

// Weights j..j+3 of a row (j % 4 == 0): four f32, four bf16 (BITS 16: a
// dense bf16 Linear), or four codes (one word at 8 bits, half a word at 4,
// little end first) dequantised in f32 as fmaf(code, scale, bias) with the
// scale and bias of group j / 64.  In two steps: router_raw4 only loads
// (the words as stored, and for codes the group's scale and bias bits),
// router_cvt4 only computes.  The kernels hold the raw words while the
// loads are in flight and convert them where they use them (a conversion
// next to its load would wait for the load there).  All-zero words convert
// to four zeros.
struct WRaw4 {
  uint32_t a, b, c, d;
};
template <int BITS>
__device__ __forceinline__ WRaw4 router_raw4(const WRow& r, int j) {
  if constexpr (BITS == 0) {
    const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const float*>(r.w) + j);
    return WRaw4{u.x, u.y, u.z, u.w};
  } else if constexpr (BITS == 16) {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(r.w) + j);
    return WRaw4{u.x, u.y, 0u, 0u};
  } else {
    const uint8_t* p = static_cast<const uint8_t*>(r.w);
    const uint32_t c = BITS == 8
                           ? *reinterpret_cast<const uint32_t*>(p + j)
                           : (uint32_t)*reinterpret_cast<const uint16_t*>(p + j / 2);
    return WRaw4{c, (uint32_t)r.s[j >> 6], (uint32_t)r.b[j >> 6], 0u};
  }
}
template <int BITS>
__device__ __forceinline__ float4 router_cvt4(const WRaw4& w) {
  if constexpr (BITS == 0) {
    return make_float4(__uint_as_float(w.a), __uint_as_float(w.b), __uint_as_float(w.c),
                       __uint_as_float(w.d));
  } else if constexpr (BITS == 16) {
    return make_float4(__uint_as_float(w.a << 16), __uint_as_float(w.a & 0xffff0000u),
                       __uint_as_float(w.b << 16), __uint_as_float(w.b & 0xffff0000u));
  } else {
    const uint32_t c = w.a;
    const float sc = __uint_as_float(w.b << 16), bi = __uint_as_float(w.c << 16);
    constexpr uint32_t m = (1u << BITS) - 1u;
    return make_float4(__builtin_fmaf((float)(c & m), sc, bi),
                       __builtin_fmaf((float)((c >> BITS) & m), sc, bi),
                       __builtin_fmaf((float)((c >> (2 * BITS)) & m), sc, bi),
                       __builtin_fmaf((float)((c >> (3 * BITS)) & m), sc, bi));
  }
}

// The finished dot product of logit column e: + bias for an f32 Linear
// that has one, one bf16 rounding for a bf16 or quantised router.
template <int BITS>
__device__ __forceinline__ float router_finish(float v, const float* bias,
                                               int e, int E) {
  if (BITS) return bf16_round(v);
  return (bias && e < E) ? v + bias[e] : v;
}

// One wave computes EB logit columns for up to TB tokens of a token block.
// Router weights stream as float4 (16 B per lane), x as 4 bf16 (8 B); the
// loads of U consecutive 256-wide steps are issued before their FMAs.
// NORM: the logits of fast::rms_norm(x) instead (the norm in front of the
// router folded in): each wave first takes the sum of squares of its tokens'
// rows in rms_norm_kernel's lane order, then normalises every x element as
// rms_norm_kernel does before its FMA, so the logits and the normalised rows
// are bit-identical to the two-kernel sequence; the first wave of the first
// expert block also writes the normalised rows (nm.out) for the experts.
// router_logits_wave is one wave's share: columns e0 .. e0 + EB - 1 for
// tokens t0 .. t0 + TB - 1 (those below T; t0 < T); `writer`: this wave
// also writes the normalised rows.
template <int EB, int TB, int U, int BITS, bool NORM>
__device__ __forceinline__ void router_logits_wave(
    const uint16_t* __restrict__ x, int T, int d, const RouterWeights& rw,
    const float* __restrict__ bias, int E, float* __restrict__ logits,
    int64_t ld, const RouterNorm& nm, int e0, int t0, bool writer) {
  const int lane = threadIdx.x & 63;
  const int e_tot = E + (rw.w_extra ? 1 : 0);
  const int nt = min(TB, T - t0);

  WRow wrow[EB];
#pragma unroll
  for (int q = 0; q < EB; ++q) wrow[q] = router_row<BITS>(rw, e0 + q, E, d);
  const uint16_t* xrow[TB];
#pragma unroll
  for (int tt = 0; tt < TB; ++tt)
    xrow[tt] = x + (int64_t)(t0 + (tt < nt ? tt : 0)) * d;
  float acc[EB][TB];
#pragma unroll
  for (int q = 0; q < EB; ++q)
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) acc[q][tt] = 0.0f;
  float rs[TB];
  if constexpr (NORM) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      float a = 0.0f;
      for (int j0 = 4 * lane; j0 < d; j0 += 256) {
        const uint2 u = *reinterpret_cast<const uint2*>(xrow[tt] + j0);
        const float v[4] = {__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                            __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u)};
#pragma unroll
        for (int c = 0; c < 4; ++c) a = __builtin_fmaf(v[c], v[c], a);
      }
      const float ss = wave_sum_butterfly(a);
      rs[tt] = 1.0f / sqrtf(ss / (float)d + nm.eps);
    }
  }

  const int steps = (d + 255) / 256;
  for (int i0 = 0; i0 < steps; i0 += U) {
    WRaw4 wv[U][EB];
    uint2 xv[U][TB];
    uint2 nwv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = 4 * lane + 256 * (i0 + u);
      const bool in = j < d;
#pragma unroll
      for (int q = 0; q < EB; ++q)
        wv[u][q] = (in && wrow[q].w) ? router_raw4<BITS>(wrow[q], j) : WRaw4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int tt = 0; tt < TB; ++tt)
        xv[u][tt] = in ? *reinterpret_cast<const uint2*>(xrow[tt] + j)
                       : make_uint2(0u, 0u);
      nwv[u] = make_uint2(0u, 0u);
      if constexpr (NORM)
        nwv[u] = in ? *reinterpret_cast<const uint2*>(nm.w + j) : make_uint2(0u, 0u);
    }
    // elements past d contribute fmaf(0, 0, acc) = acc exactly
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float4 wf[EB];
#pragma unroll
      for (int q = 0; q < EB; ++q) wf[q] = router_cvt4<BITS>(wv[u][q]);
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) {
        if constexpr (NORM) {
          // out_j = bf16(w_j * bf16(x_j * r)), as rms_norm_kernel
          const uint2 xw = xv[u][tt], nw = nwv[u];
          const uint32_t o0 = f32_to_bf16(__uint_as_float(nw.x << 16) *
                                          bf16_round(__uint_as_float(xw.x << 16) * rs[tt]));
          const uint32_t o1 = f32_to_bf16(__uint_as_float(nw.x & 0xffff0000u) *
                                          bf16_round(__uint_as_float(xw.x & 0xffff0000u) * rs[tt]));
          const uint32_t o2 = f32_to_bf16(__uint_as_float(nw.y << 16) *
                                          bf16_round(__uint_as_float(xw.y << 16) * rs[tt]));
          const uint32_t o3 = f32_to_bf16(__uint_as_float(nw.y & 0xffff0000u) *
                                          bf16_round(__uint_as_float(xw.y & 0xffff0000u) * rs[tt]));
          xv[u][tt] = make_uint2(o0 | (o1 << 16), o2 | (o3 << 16));
          const int j = 4 * lane + 256 * (i0 + u);
          if (writer && tt < nt && j < d)
            *reinterpret_cast<uint2*>(nm.out + (int64_t)(t0 + tt) * d + j) = xv[u][tt];
        }
        const float x0 = __uint_as_float(xv[u][tt].x << 16);
        const float x1 = __uint_as_float(xv[u][tt].x & 0xffff0000u);
        const float x2 = __uint_as_float(xv[u][tt].y << 16);
        const float x3 = __uint_as_float(xv[u][tt].y & 0xffff0000u);
#pragma unroll
        for (int q = 0; q < EB; ++q) {
          float a = acc[q][tt];
          a = __builtin_fmaf(x0, wf[q].x, a);
          a = __builtin_fmaf(x1, wf[q].y, a);
          a = __builtin_fmaf(x2, wf[q].z, a);
          a = __builtin_fmaf(x3, wf[q].w, a);
          acc[q][tt] = a;
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < EB; ++q) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      const float v =
          router_finish<BITS>(wave_sum_butterfly(acc[q][tt]), bias, e0 + q, E);
      if (lane == 0 && e0 + q < e_tot && tt < nt)
        logits[(int64_t)(t0 + tt) * ld + e0 + q] = v;
    }
  }
}

template <int EB, int TB, int U, int BITS, bool NORM>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, int T, int d, const RouterWeights rw,
    const float* __restrict__ bias, int E, float* __restrict__ logits,
    int64_t ld, const RouterNorm nm, int32_t* __restrict__ clear) {
  const int wave = threadIdx.x >> 6;
  if (clear && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *clear = 0;
  const int e0 = (blockIdx.x * 4 + wave) * EB;
  if (e0 >= E + (rw.w_extra ? 1 : 0)) return;
  router_logits_wave<EB, TB, U, BITS, NORM>(x, T, d, rw, bias, E, logits, ld, nm, e0,
                                            blockIdx.y * TB,
                                            NORM && nm.out && blockIdx.x == 0 && wave == 0);
}

// Many tokens: one workgroup computes 32 tokens x 16 logit columns.  Each
// 256-wide step of d is staged in LDS (x as bf16, the weights as f32; the
// next step's loads are in flight in registers meanwhile) and every wave
// multiplies 8 tokens x 16 columns from it, so each value loaded from memory
// feeds 8 or 16 dot products.  A lane accumulates exactly the elements
// j = 4l + 256i + c in (i, c) order, like router_logits_kernel, and the 64
// lane sums of a logit are added in the butterfly's pairwise tree (lanes
// l and l^32 first, ... l and l^1 last) -- by one lane reading them from
// LDS rather than by six shuffles on every lane.  Same bits.
// kRtCol experts x 4 * WT tokens per workgroup (WT tokens per wave: 8, or
// 4 where 8 would leave CUs idle)
constexpr int kRtCol = 16;
// With `extra` the grid's last column of workgroups computes one more logit
// column (weights rx, written at lx): the lone extra column (the shared
// expert's gate beside 16k experts) in router_logits_wave's lane order, WT
// tokens per wave, instead of a round of 16-column blocks or a launch of
// its own.
template <int BITS, int WT>
__global__ __launch_bounds__(256) void router_logits_tiled_kernel(
    const uint16_t* __restrict__ x, int T, int d, const RouterWeights rw,
    const float* __restrict__ bias, int E, float* __restrict__ logits,
    int64_t ld, bool extra, const RouterWeights rx, float* __restrict__ lx,
    int32_t* __restrict__ clear) {
  constexpr int kRtTok = 4 * WT, kRtWaveTok = WT;
  if (clear && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *clear = 0;
  if (extra && blockIdx.x == gridDim.x - 1) {
    const int t0 = (int)blockIdx.y * kRtTok + (int)(threadIdx.x >> 6) * WT;
    if (t0 < T)
      router_logits_wave<1, WT, 2, BITS, false>(x, T, d, rx, nullptr, 1, lx, ld,
                                                RouterNorm{nullptr, 0.0f, nullptr}, 0, t0,
                                                false);
    return;
  }
  constexpr int XK = kRtTok / 8;  // 16-byte x chunks per thread per step
  constexpr int CPR = 32 / WT;    // columns per round of the final sums
  static_assert(WT == 4 || WT == 8, "tokens per wave");
  // the step's x [kRtTok][256] bf16 and w [16][256] f32; afterwards the
  // lane sums [wave][32 logits][64 lanes] f32 (32 KB), 32 logits at a time
  constexpr int kStageBytes = kRtTok * 256 * 2 + kRtCol * 256 * 4;
  __shared__ __attribute__((aligned(16))) char lds[kStageBytes > 32768 ? kStageBytes : 32768];
  uint16_t (*xs)[256] = reinterpret_cast<uint16_t (*)[256]>(lds);
  float (*ws)[256] = reinterpret_cast<float (*)[256]>(lds + kRtTok * 256 * 2);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e_tot = E + (rw.w_extra ? 1 : 0);
  const int e0 = blockIdx.x * kRtCol, t0 = blockIdx.y * kRtTok;
  float acc[kRtCol][kRtWaveTok];
#pragma unroll
  for (int q = 0; q < kRtCol; ++q)
#pragma unroll
    for (int tt = 0; tt < kRtWaveTok; ++tt) acc[q][tt] = 0.0f;
  // this thread's staging chunks: x rows id/32 (8 bf16 at (id%32)*8), w rows
  // id/64 (4 weights at (id%64)*4, dequantised to f32 on the way to LDS),
  // id = tid + 256k; zeros past d / T / e_tot
  const uint16_t* xp[XK];
  WRow wp[4];
#pragma unroll
  for (int k = 0; k < XK; ++k) {
    const int id = tid + 256 * k;
    const int t = t0 + (id >> 5);
    xp[k] = t < T ? x + (int64_t)t * d + (id & 31) * 8 : nullptr;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) wp[k] = router_row<BITS>(rw, e0 + ((tid + 256 * k) >> 6), E, d);
  u32x4_t xr[XK];
  WRaw4 wr[4];  // raw: converted when staged, so the loads stay in flight
  auto fetch = [&](int i) {
    const int j0 = 256 * i;
#pragma unroll
    for (int k = 0; k < XK; ++k) {
      const int id = tid + 256 * k;
      xr[k] = (xp[k] && j0 + (id & 31) * 8 < d)
                  ? *reinterpret_cast<const u32x4_t*>(xp[k] + j0)
                  : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int id = tid + 256 * k;
      wr[k] = (wp[k].w && j0 + (id & 63) * 4 < d)
                  ? router_raw4<BITS>(wp[k], j0 + (id & 63) * 4)
                  : WRaw4{0u, 0u, 0u, 0u};
    }
  };
  const int steps = (d + 255) / 256;
  fetch(0);
  for (int i = 0; i < steps; ++i) {
#pragma unroll
    for (int k = 0; k < XK; ++k) {
      const int id = tid + 256 * k;
      *reinterpret_cast<u32x4_t*>(&xs[id >> 5][(id & 31) * 8]) = xr[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int id = tid + 256 * k;
      *reinterpret_cast<float4*>(&ws[id >> 6][(id & 63) * 4]) = router_cvt4<BITS>(wr[k]);
    }
    __syncthreads();
    if (i + 1 < steps) fetch(i + 1);
    float xv[kRtWaveTok][4];
#pragma unroll
    for (int tt = 0; tt < kRtWaveTok; ++tt) {
      const uint2 u = *reinterpret_cast<const uint2*>(&xs[wave * kRtWaveTok + tt][4 * lane]);
      xv[tt][0] = __uint_as_float(u.x << 16);
      xv[tt][1] = __uint_as_float(u.x & 0xffff0000u);
      xv[tt][2] = __uint_as_float(u.y << 16);
      xv[tt][3] = __uint_as_float(u.y & 0xffff0000u);
    }
#pragma unroll
    for (int q = 0; q < kRtCol; ++q) {
      const float4 wv = *reinterpret_cast<const float4*>(&ws[q][4 * lane]);
#pragma unroll
      for (int tt = 0; tt < kRtWaveTok; ++tt) {
        float a = acc[q][tt];
        a = __builtin_fmaf(xv[tt][0], wv.x, a);
        a = __builtin_fmaf(xv[tt][1], wv.y, a);
        a = __builtin_fmaf(xv[tt][2], wv.z, a);
        a = __builtin_fmaf(xv[tt][3], wv.w, a);
        acc[q][tt] = a;
      }
    }
    __syncthreads();
  }
  // lane sums -> logits, 32 logits (CPR columns x WT tokens) per round;
  // each wave uses its own quarter of the LDS, logit i's row swizzled by i
  float* red = reinterpret_cast<float*>(lds) + wave * 32 * 64;
#pragma unroll
  for (int q0 = 0; q0 < kRtCol; q0 += CPR) {
#pragma unroll
    for (int qq = 0; qq < CPR; ++qq)
#pragma unroll
      for (int tt = 0; tt < kRtWaveTok; ++tt)
        red[(qq * kRtWaveTok + tt) * 64 + (lane ^ (qq * kRtWaveTok + tt))] =
            acc[q0 + qq][tt];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 32) {
      // lane j's sum of logit `lane` sits at [lane][j ^ lane] (the swizzle
      // keeps the 32 readers on distinct banks)
      const float* v = red + lane * 64;
      float s[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) s[j] = v[j ^ lane] + v[(j + 32) ^ lane];
#pragma unroll
      for (int h = 16; h >= 1; h >>= 1)
#pragma unroll
        for (int j = 0; j < h; ++j) s[j] = s[j] + s[j + h];
      const int qq = lane / kRtWaveTok, tt = lane % kRtWaveTok;
      const int e = e0 + q0 + qq, t = t0 + wave * kRtWaveTok + tt;
      const float r = router_finish<BITS>(s[0], bias, e, E);
      if (e < e_tot && t < T) logits[(int64_t)t * ld + e] = r;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// One wave per token: top-K, softmax and renormalised weights (wave_topk).
// Workgroup 0 also clears the workspace status word when given.
template <int SLOTS, bool BF16>
__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, int64_t ld, int T, int E, int K,
    int32_t* __restrict__ idx, float* __restrict__ wts, int32_t* status) {
  __shared__ TopkScratch sc[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (status && blockIdx.x == 0 && threadIdx.x == 0) *status = 0;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  int id;
  float wt;
  wave_topk<SLOTS, BF16>(logits + (int64_t)t * ld, E, K, &sc[wave], &id, &wt);
  if (lane < K) {
    idx[(int64_t)t * K + lane] = id;
    wts[(int64_t)t * K + lane] = wt;
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

// rows the norm holds in registers (up to kMaxRmsDims values): 4 values
// per lane per 256-wide piece
constexpr int kRmsPieces = 16;
constexpr int kMaxRmsDims = 256 * kRmsPieces;
// fast::rms_norm as gemma4's router applies it (Router::forward,
// crates/mlxr-lm/src/gemma4/text/text.rs:640) and as RmsNorm::forward does
// (crates/mlxr/src/layers/normalization.rs:272-276): out_j = bf16(w_j *
// bf16(x_j * r)), r = 1 / sqrt(sum_j x_j^2 / d + eps) -- MLX's rounding
// points (the normalised value in the input dtype, then the weight
// product) -- with the sum of squares in the router's lane order (fmaf over
// j = 4l + 256i + c, then the butterfly).  One wave per row.
__global__ __launch_bounds__(256) void rms_norm_kernel(
    const uint16_t* __restrict__ x, int T, int d,
    const uint16_t* __restrict__ w, float eps, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const uint16_t* xr = x + (int64_t)t * d;
  uint16_t* orow = out + (int64_t)t * d;
  const auto piece = [](uint2 u, float (&v)[4]) {
    v[0] = __uint_as_float(u.x << 16);
    v[1] = __uint_as_float(u.x & 0xffff0000u);
    v[2] = __uint_as_float(u.y << 16);
    v[3] = __uint_as_float(u.y & 0xffff0000u);
  };
  if (d <= kMaxRmsDims && (reinterpret_cast<uintptr_t>(w) & 7) == 0) {
    // the row's 4-element pieces stay in registers between the two passes,
    // and the weight's load with them (8-byte pieces)
    uint2 xv[kRmsPieces], wv[kRmsPieces];
#pragma unroll
    for (int i = 0; i < kRmsPieces; ++i) {
      const int j0 = 4 * lane + 256 * i;
      xv[i] = j0 < d ? *reinterpret_cast<const uint2*>(xr + j0) : make_uint2(0u, 0u);
      wv[i] = j0 < d ? *reinterpret_cast<const uint2*>(w + j0) : make_uint2(0u, 0u);
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kRmsPieces; ++i) {
      float v[4];
      piece(xv[i], v);
      // (pieces past d are zeros: adding 0*0 leaves the sum as it is)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc = __builtin_fmaf(v[c], v[c], acc);
    }
    const float ss = wave_sum_butterfly(acc);
    const float r = 1.0f / sqrtf(ss / (float)d + eps);
#pragma unroll
    for (int i = 0; i < kRmsPieces; ++i) {
      const int j0 = 4 * lane + 256 * i;
      float v[4], g[4];
      piece(xv[i], v);
      piece(wv[i], g);
      uint32_t o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = f32_to_bf16(g[c] * bf16_round(v[c] * r));
      if (j0 < d)
        *reinterpret_cast<uint2*>(orow + j0) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
    }
    return;
  }
  // wider rows (or a weight not 8-byte aligned): x read twice, w by element
  float acc = 0.0f;
  for (int j0 = 4 * lane; j0 < d; j0 += 256) {
    float v[4];
    piece(*reinterpret_cast<const uint2*>(xr + j0), v);
#pragma unroll
    for (int c = 0; c < 4; ++c) acc = __builtin_fmaf(v[c], v[c], acc);
  }
  const float ss = wave_sum_butterfly(acc);
  const float r = 1.0f / sqrtf(ss / (float)d + eps);
  for (int j0 = 4 * lane; j0 < d; j0 += 256) {
    float v[4];
    piece(*reinterpret_cast<const uint2*>(xr + j0), v);
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      o[c] = f32_to_bf16(bf16_to_f32(w[j0 + c]) * bf16_round(v[c] * r));
    *reinterpret_cast<uint2*>(orow + j0) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
  }
}

// gemma4's router top-k (wave_topk GEMMA): one wave per token; bf16 weights.
template <int SLOTS>
__global__ __launch_bounds__(256) void gemma_topk_kernel(
    const float* __restrict__ scores, int64_t ld, int T, int E, int K,
    const uint16_t* __restrict__ pes, int32_t* __restrict__ idx,
    uint16_t* __restrict__ wts) {
  __shared__ TopkScratch sc[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  int id;
  float wt;
  wave_topk<SLOTS, false, true>(scores + (int64_t)t * ld, E, K, &sc[wave], &id,
                                &wt, pes);
  if (lane < K) {
    idx[(int64_t)t * K + lane] = id;
    wts[(int64_t)t * K + lane] = f32_to_bf16(wt);
  }
}

// Launch shape for 16 < T <= MLXR_RL_TILED_T (experts and tokens per wave,
// 256-wide steps of loads in flight); the LDS-tiled kernel above that.
#ifndef MLXR_RL_MID_EB
#define MLXR_RL_MID_EB 2
#endif
#ifndef MLXR_RL_MID_TB
#define MLXR_RL_MID_TB 4
#endif
#ifndef MLXR_RL_MID_U
#define MLXR_RL_MID_U 4
#endif
// ... and with one expert per wave (4 steps in flight: c2 T=32 logits
// 9.1 to 8.4 us, T=64 9.6 to 9.2, c6 T=64 12.9 to 12.6 against 2; 8 slower
// at c6)
#ifndef MLXR_RL_MID_U1
#define MLXR_RL_MID_U1 4
#endif
#ifndef MLXR_RL_TILED_T
#define MLXR_RL_TILED_T 256
#endif
// most tokens for which the norm in front of the router is folded into it
// The matrix-core router (router_logits_mfma_kernel) for f32 routers above
// MLXR_RL_TILED_T tokens, and its chunks of loads in flight per lane.
#ifndef MLXR_RL_MFMA
#define MLXR_RL_MFMA 1
#endif
#ifndef MLXR_RL_MFMA_MIN_T
#define MLXR_RL_MFMA_MIN_T 512
#endif
// ... and from this many 32 x 32 tiles (workgroups): below it the grid
// leaves too many SIMDs without a wave (measured at T = 1024: c3, 128
// tiles, 17.7 to 19.0-20.1 us; c4, 544, 53.6 to 36.2; c6, 288, 33.5 to
// 29.9; c8, 256, 32.3 to 27.0; c3 T = 1536, 192, 22.1 to 20.5)
#ifndef MLXR_RL_MFMA_MIN_WG
#define MLXR_RL_MFMA_MIN_WG 192
#endif
#ifndef MLXR_RL_MFMA_PARTS
#define MLXR_RL_MFMA_PARTS 4
#endif
#ifndef MLXR_RL_NORM_MAX_T
#define MLXR_RL_NORM_MAX_T 2
#endif
// Many tokens: the matrix cores (any router format: f32, bf16 or 4/8-bit
// weights, converted to f32 as they are staged).  One workgroup = P
// waves = one tile of 32 tokens x 32 logit columns; wave q takes the q-th
// of P equal parts of d, in chunks of 16 elements.  Per chunk each lane
// holds 8 consecutive x values of its token row (lanes 32-63 the chunk's
// upper half) and the same 8 weights of its column, and 8
// v_mfma_f32_32x32x2_f32 add them: MFMA s computes
// fmaf(x[j+8+s] w[j+8+s], fmaf(x[j+s] w[j+s], acc)) for every (token,
// column) of the tile (an in-bounds probe of the instruction on this GPU
// matched that pair of fmaf bit for bit on 20480 outputs).  The parts meet
// in LDS and wave 0 adds them in order, ((q0 + q1) + q2) + ..., then the
// bias.  Each wave stages 64 elements (4 chunks) of its 32 x rows and 32
// weight rows at a time through its own LDS region, loaded as whole cache
// lines (a direct load per fragment touched 32 lines per instruction), the
// next 64 in flight in registers meanwhile; rows padded by 16 bytes so the
// fragment reads of 16 rows fall on distinct banks.  Rows past T read the
// last row and columns past the router read zeros; neither is stored.  A
// quantised or bf16 router's logit is the sum rounded to bf16 (its weights
// the f32 values router_cvt4 gives: fmaf(code, scale, bias), or exact).
// Needs d % (64 P) == 0 and 16-byte aligned rows.
// elements of d per staging step (64 or 32: 4 or 2 chunks of 16; 32 halves
// the LDS, which measured no faster)
#ifndef MLXR_RL_MFMA_STAGE
#define MLXR_RL_MFMA_STAGE 64
#endif
constexpr int kRmStage = MLXR_RL_MFMA_STAGE;
constexpr int kRmXp = kRmStage / 8, kRmWp = kRmStage / 4;  // 16-byte pieces of a row
constexpr int kRmXs = 2 * kRmStage + 16, kRmWs = 4 * kRmStage + 16;  // LDS row strides
constexpr int kRmWave = 32 * kRmXs + 32 * kRmWs;                     // LDS per wave
template <int BITS, int P>
__global__ __launch_bounds__(64 * P) void router_logits_mfma_kernel(
    const uint16_t* __restrict__ x, int T, int d, const RouterWeights rw,
    const float* __restrict__ bias, int E, float* __restrict__ logits, int64_t ld,
    int32_t* __restrict__ clear) {
  static_assert((P - 1) * 64 * 64 <= P * kRmWave, "partial sums fit the staging LDS");
  constexpr int XI = 32 * kRmXp / 64, WI = 32 * kRmWp / 64;  // pieces per lane
  __shared__ __attribute__((aligned(16))) char lds[P * kRmWave];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6, h = lane >> 5, r = lane & 31;
  if (clear && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *clear = 0;
  const int t0 = (int)blockIdx.y * 32, e0 = (int)blockIdx.x * 32;
  const int e_tot = E + (rw.w_extra ? 1 : 0);
  char* xs = lds + q * kRmWave;
  char* ws = xs + 32 * kRmXs;
  // staging: x piece id = lane + 64 i (i < XI): row id / kRmXp, 16 bytes
  // id % kRmXp; weight piece id = lane + 64 i (i < WI): column id / kRmWp,
  // 16 bytes id % kRmWp
  const uint16_t* xsrc[XI];
  int wcol[WI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int id = lane + 64 * i;
    xsrc[i] = x + (int64_t)min(t0 + id / kRmXp, T - 1) * d + 8 * (id % kRmXp);
  }
#pragma unroll
  for (int i = 0; i < WI; ++i) wcol[i] = e0 + (lane + 64 * i) / kRmWp;
  const int dq = d / P, nsc = dq / kRmStage;  // staging steps per part
  const int kq = q * dq;
  u32x4_t xg[XI];
  WRaw4 wg[WI];
  auto load = [&](int sc) {
    const int k = kq + kRmStage * sc;
#pragma unroll
    for (int i = 0; i < XI; ++i) xg[i] = *reinterpret_cast<const u32x4_t*>(xsrc[i] + k);
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      // (columns past the router: a row of zeros from the first one)
      const WRow row = router_row<BITS>(rw, wcol[i] < e_tot ? wcol[i] : 0, E, d);
      wg[i] = router_raw4<BITS>(row, k + 4 * ((lane + 64 * i) % kRmWp));
    }
  };
  load(0);
  f32x16_t acc = {};
  for (int sc = 0; sc < nsc; ++sc) {
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int id = lane + 64 * i;
      *reinterpret_cast<u32x4_t*>(xs + id / kRmXp * kRmXs + 16 * (id % kRmXp)) = xg[i];
    }
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const int id = lane + 64 * i;
      const float4 v = router_cvt4<BITS>(wg[i]);
      *reinterpret_cast<f32x4_t*>(ws + id / kRmWp * kRmWs + 16 * (id % kRmWp)) =
          wcol[i] < e_tot ? f32x4_t{v.x, v.y, v.z, v.w} : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    load(min(sc + 1, nsc - 1));
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < kRmStage / 16; ++c) {
      const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xs + r * kRmXs + 32 * c + 16 * h);
      const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(ws + r * kRmWs + 64 * c + 32 * h);
      const f32x4_t w1 =
          *reinterpret_cast<const f32x4_t*>(ws + r * kRmWs + 64 * c + 32 * h + 16);
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const uint32_t u = xv[s >> 1];
        const float a = __uint_as_float((s & 1) ? (u & 0xffff0000u) : (u << 16));
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, s < 4 ? w0[s] : w1[s - 4], acc, 0, 0, 0);
      }
    }
  __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();  // the staging regions are free: partial sums in their place
  f32x16_t* part = reinterpret_cast<f32x16_t*>(lds);
  if (q > 0) part[(q - 1) * 64 + lane] = acc;
  __syncthreads();
  if (q != 0) return;
#pragma unroll
  for (int jq = 0; jq < P - 1; ++jq) {
    const f32x16_t pj = part[jq * 64 + lane];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = acc[i] + pj[i];
  }
  const int ec = e0 + r;
  if (ec >= e_tot) return;
  const float bv = BITS == 0 && bias && ec < E ? bias[ec] : 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = t0 + 8 * (i >> 2) + 4 * h + (i & 3);
    if (t < T)
      logits[(int64_t)t * ld + ec] = BITS != 0                 ? bf16_round(acc[i])
                                     : bias && ec < E ? acc[i] + bv
                                                      : acc[i];
  }
}

template <int BITS>
void router_logits_launch(const uint16_t* x, int64_t T, int64_t d,
                          const RouterWeights& w, const float* bias, int64_t E,
                          float* logits, int64_t ld, const RouterNorm* norm,
                          hipStream_t s, int32_t* clear) {
  const int64_t e_tot = E + (w.w_extra ? 1 : 0);
  const RouterNorm nm = norm ? *norm : RouterNorm{nullptr, 0.0f, nullptr};
  // Enough waves to have every CU pulling router weights at small T, and
  // register reuse of both operands (EB experts x TB tokens) at large T.
#define MLXR_RL_N(EB, TB, U, N)                                              \
  router_logits_kernel<EB, TB, U, BITS, N>                                   \
      <<<dim3((unsigned)((e_tot + 4 * EB - 1) / (4 * EB)),                   \
              (unsigned)((T + TB - 1) / TB)),                                \
         256, 0, s>>>(x, (int)T, (int)d, w, bias, (int)E, logits, ld, nm, clear)
#define MLXR_RL(EB, TB, U)           \
  if (norm)                          \
    MLXR_RL_N(EB, TB, U, true);      \
  else                               \
    MLXR_RL_N(EB, TB, U, false)
  // The folded norm pays only while the launch it saves outweighs its
  // repetition (every expert block of a token block normalises the same
  // rows).  Measured on the c6 layer tail against the separate norm pass:
  // T = 1 3 us and T = 2 1.3 us faster, T = 8 2 us and T = 16 8 us
  // slower (c7's router: T = 1 2 us faster).  Above MLXR_RL_NORM_MAX_T
  // tokens the norm is its own pass.
  if (norm && T > MLXR_RL_NORM_MAX_T) {
    // (a failed launch stays the runtime's last error, which the caller
    // returns after the logits launch)
    (void)launch_rms_norm(x, T, d, norm->w, norm->eps, norm->out, s);
    x = norm->out;
    norm = nullptr;
  }
  {
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (router_matrix_order(T, d, e_tot) && !norm && al16(x) && al16(w.w) &&
        (!w.w_extra || al16(w.w_extra))) {
      constexpr int P = MLXR_RL_MFMA_PARTS;
      router_logits_mfma_kernel<BITS, P>
          <<<dim3((unsigned)((e_tot + 31) / 32), (unsigned)((T + 31) / 32)), 64 * P, 0, s>>>(
              x, (int)T, (int)d, w, bias, (int)E, logits, ld, clear);
      return;
    }
  }
  if (T <= 2) {
    MLXR_RL(1, 1, 8);
  } else if (T <= 16) {
    MLXR_RL(1, 2, 8);
  } else if (T <= MLXR_RL_TILED_T || d % 8 ||
             (reinterpret_cast<uintptr_t>(x) & 15)) {
    // (the tiled kernel stages x in 16-byte chunks of 8 values: whole
    // chunks only, so rows of a multiple of 8 values, 16-byte aligned)
    // (up to 256 logit columns one expert per wave, which measured faster
    // there: c2 T=64 10.0 -> 9.7 us, c6 15.3 -> 12.8; wider routers keep
    // two per wave)
    if (e_tot <= 4 * 64 + 1)
      MLXR_RL_N(1, MLXR_RL_MID_TB, MLXR_RL_MID_U1, false);
    else
      MLXR_RL_N(MLXR_RL_MID_EB, MLXR_RL_MID_TB, MLXR_RL_MID_U, false);
  } else {
    // A lone extra column (the shared expert's gate beside 16k experts)
    // would add a round of whole column blocks: the tiled blocks take the
    // E expert columns and per-wave code the extra one (the same lane order
    // and butterfly, so the same bits).
    const bool split = w.w_extra && e_tot % kRtCol == 1;
    RouterWeights wm = w;
    if (split) wm.w_extra = nullptr, wm.scales_extra = nullptr, wm.biases_extra = nullptr;
    const int64_t cols = split ? E : e_tot;
    // 8 tokens per wave, or 4 where 8 would make fewer workgroups than
    // the GPU's 2 x 256 slots (c3 T=512: 128 workgroups)
    const int64_t cb = (cols + kRtCol - 1) / kRtCol;
    // The extra column, when split off: one more column of workgroups in
    // the same grid while the grid fits the GPU's workgroup slots at once
    // (two per CU at 8 tokens per wave, three at 4: the registers allow no
    // more; c6 T=512 logits 23.5 to 21.1 µs); on a larger grid those light
    // workgroups would add a round of slots (c6 T=2048 57.0 to 63.1 µs), so
    // there they run as a launch of their own after it.
    const RouterWeights we{w.bits, w.w_extra, w.scales_extra, w.biases_extra,
                           nullptr, nullptr, nullptr};
    const bool wt8 = cb * ((T + 31) / 32) >= 512;
    const int64_t rows = wt8 ? (T + 31) / 32 : (T + 15) / 16;
    const bool fold = split && (cb + 1) * rows <= (wt8 ? 512 : 768);
    const unsigned gx = (unsigned)cb + (fold ? 1u : 0u);
    if (wt8)
      router_logits_tiled_kernel<BITS, 8>
          <<<dim3(gx, (unsigned)rows), 256, 0, s>>>(
              x, (int)T, (int)d, wm, bias, (int)E, logits, ld, fold, we, logits + E,
              clear);
    else
      router_logits_tiled_kernel<BITS, 4>
          <<<dim3(gx, (unsigned)rows), 256, 0, s>>>(
              x, (int)T, (int)d, wm, bias, (int)E, logits, ld, fold, we, logits + E,
              clear);
    if (split && !fold) {
      constexpr int kTB = MLXR_RL_MID_TB;
      router_logits_kernel<1, kTB, 2, BITS, false>
          <<<dim3(1u, (unsigned)((T + kTB - 1) / kTB)), 256, 0, s>>>(
              x, (int)T, (int)d, we, nullptr, 1, logits + E, ld, nm, nullptr);
    }
  }
#undef MLXR_RL
#undef MLXR_RL_N
}

template <bool BF16>
void router_topk_launch(const float* logits, int64_t ld, int64_t T, int64_t E,
                        int64_t K, int32_t* idx, float* wts, int32_t* status,
                        hipStream_t s) {
  const dim3 grid((unsigned)((T + 3) / 4));
  const int slots = (int)((E + 63) / 64);
#define MLXR_TOPK(S)                                                           \
  router_topk_kernel<S, BF16><<<grid, 256, 0, s>>>(logits, ld, (int)T, (int)E, \
                                                   (int)K, idx, wts, status)
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
}

}  // namespace

bool router_matrix_order(int64_t T, int64_t d, int64_t cols) {
  return MLXR_RL_MFMA && T >= MLXR_RL_MFMA_MIN_T && d % (64 * MLXR_RL_MFMA_PARTS) == 0 &&
         (cols + 31) / 32 * ((T + 31) / 32) >= MLXR_RL_MFMA_MIN_WG;
}

hipError_t launch_router_logits(const uint16_t* x, int64_t T, int64_t d,
                                const RouterWeights& w, const float* bias,
                                int64_t E, float* logits, int64_t ld,
                                hipStream_t s, const RouterNorm* norm, int32_t* clear) {
  if (T == 0) return hipSuccess;
  if (w.bits != 0 && w.bits != 4 && w.bits != 8 && w.bits != 16)
    return hipErrorInvalidValue;
  if (norm && (!norm->w || !norm->out || d % 4)) return hipErrorInvalidValue;
  ProfileScope prof("router_logits", s);
  if (w.bits == 16)
    router_logits_launch<16>(x, T, d, w, bias, E, logits, ld, norm, s, clear);
  else if (w.bits == 8)
    router_logits_launch<8>(x, T, d, w, bias, E, logits, ld, norm, s, clear);
  else if (w.bits == 4)
    router_logits_launch<4>(x, T, d, w, bias, E, logits, ld, norm, s, clear);
  else
    router_logits_launch<0>(x, T, d, w, bias, E, logits, ld, norm, s, clear);
  return hipGetLastError();
}

hipError_t launch_router_topk(const float* logits, int64_t ld, int64_t T,
                              int64_t E, int64_t K, bool bf16, int32_t* idx,
                              float* wts, int32_t* status, hipStream_t s) {
  if (T == 0) return hipSuccess;
  ProfileScope prof("router_topk", s);
  if (bf16)
    router_topk_launch<true>(logits, ld, T, E, K, idx, wts, status, s);
  else
    router_topk_launch<false>(logits, ld, T, E, K, idx, wts, status, s);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const uint16_t* x, int64_t T, int64_t d,
                           const uint16_t* w, float eps, uint16_t* out,
                           hipStream_t s) {
  if (T == 0) return hipSuccess;
  ProfileScope prof("rms_norm", s);
  rms_norm_kernel<<<(unsigned)((T + 3) / 4), 256, 0, s>>>(x, (int)T, (int)d, w,
                                                          eps, out);
  return hipGetLastError();
}

hipError_t launch_gemma_topk(const float* scores, int64_t ld, int64_t T,
                             int64_t E, int64_t K, const uint16_t* pes,
                             int32_t* idx, uint16_t* wts, hipStream_t s) {
  if (T == 0) return hipSuccess;
  ProfileScope prof("router_topk", s);
  const dim3 grid((unsigned)((T + 3) / 4));
  const int slots = (int)((E + 63) / 64);
#define MLXR_GT(S)                                                        \
  gemma_topk_kernel<S><<<grid, 256, 0, s>>>(scores, ld, (int)T, (int)E,   \
                                            (int)K, pes, idx, wts)
  if (slots <= 1)
    MLXR_GT(1);
  else if (slots <= 2)
    MLXR_GT(2);
  else if (slots <= 4)
    MLXR_GT(4);
  else if (slots <= 8)
    MLXR_GT(8);
  else
    MLXR_GT(16);
#undef MLXR_GT
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
