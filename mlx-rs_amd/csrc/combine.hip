// Weighted combine of the routed expert rows, plus the sigmoid-gated shared
// expert, on gfx950.
//
// Replaces combine_with_weights (crates/mlxr-lm/src/nn/switch.rs:223-234):
// (w * y) with w f32 [T,K,1] and y bf16 [T,K,d] promotes to f32, then a sum
// over K; and, from Qwen35MoeBlock::forward (moe.rs:117-120, 145),
// shared * sigmoid(shared_gate(x)) + routed.  Each product is rounded to f32
// before the k-ordered sum, as in the reference's two-op sequence.
// With a quantised (bf16) router the weights and the shared-gate logit are
// bf16 and so is every op: w * y rounded to bf16, the sum over k in f32
// rounded to bf16, shared = bf16(y_s * bf16(sigmoid(sg))), out =
// bf16(shared + routed).
// With a residual h (bf16 [T, d]) the decoder layer's add after the block
// (DecoderLayer::forward, crates/mlxr-lm/src/qwen3_5/text/layer.rs:138)
// follows in the same pass: out = h + mlp_out, f32 (bf16 + f32 promotes) or
// bf16(h + bf16(mlp_out)) in the bf16 chain.
// HBM-bound elementwise pass: 8 outputs per thread, 16 B loads of y.
#include "common.hpp"
#include "kernels.hpp"

// threads per workgroup (64 or 256)
#ifndef MLXR_COMBINE_THREADS
#define MLXR_COMBINE_THREADS 64
#endif

namespace mlxr_moe {
namespace {

template <bool BF16, typename WT>
__global__ __launch_bounds__(256) void combine_kernel(
    const uint16_t* __restrict__ y, const WT* __restrict__ w, int T, int K,
    int d, const uint16_t* __restrict__ shared_y,
    const float* __restrict__ shared_logit, int64_t shared_ld,
    const uint16_t* __restrict__ residual, void* __restrict__ out) {
  constexpr int kBatch = 8;
  const int t = blockIdx.y;
  const int n0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (t >= T || n0 >= d) return;
  // the shared row, its gate logit and the residual row are issued first
  const u32x4_t zq = {0u, 0u, 0u, 0u};
  const u32x4_t sv = shared_y ? *reinterpret_cast<const u32x4_t*>(
                                    shared_y + (int64_t)t * d + n0)
                              : zq;
  const float slog = shared_y ? shared_logit[t * shared_ld] : 0.0f;
  const u32x4_t rv = residual ? *reinterpret_cast<const u32x4_t*>(
                                    residual + (int64_t)t * d + n0)
                              : zq;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
  // eight rows' loads in flight at once (indices clamped, so every load is
  // in bounds and none sits under a branch), then the k-ordered sum
  for (int k0 = 0; k0 < K; k0 += kBatch) {
    u32x4_t v[kBatch];
    float wk[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int64_t r = (int64_t)t * K + min(k0 + i, K - 1);
      v[i] = *reinterpret_cast<const u32x4_t*>(y + r * d + n0);
      if constexpr (sizeof(WT) == 2)
        wk[i] = bf16_to_f32(w[r]);
      else
        wk[i] = w[r];
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (k0 + i >= K) break;
      const uint32_t pk[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = combine_add<BF16>(acc[2 * j], wk[i], __uint_as_float(pk[j] << 16));
        acc[2 * j + 1] =
            combine_add<BF16>(acc[2 * j + 1], wk[i], __uint_as_float(pk[j] & 0xffff0000u));
      }
    }
  }
  if (BF16) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = bf16_round(acc[j]);
  }
  if (shared_y) {
    const float gate = combine_gate<BF16>(slog);
    const uint32_t pk[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] = combine_shared<BF16>(acc[2 * j], __uint_as_float(pk[j] << 16), gate);
      acc[2 * j + 1] =
          combine_shared<BF16>(acc[2 * j + 1], __uint_as_float(pk[j] & 0xffff0000u), gate);
    }
  }
  if (residual) {
    const uint32_t pk[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] = combine_residual<BF16>(acc[2 * j], __uint_as_float(pk[j] << 16));
      acc[2 * j + 1] = combine_residual<BF16>(acc[2 * j + 1], __uint_as_float(pk[j] & 0xffff0000u));
    }
  }
  if (BF16) {
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      pk[j] = (uint32_t)f32_to_bf16(acc[2 * j]) |
              ((uint32_t)f32_to_bf16(acc[2 * j + 1]) << 16);
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(out) + (int64_t)t * d + n0) =
        u32x4_t{pk[0], pk[1], pk[2], pk[3]};
  } else {
    float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)t * d + n0);
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

}  // namespace

hipError_t launch_combine(const uint16_t* y, const void* w, bool w_bf16,
                          int64_t T, int64_t K, int64_t d,
                          const uint16_t* shared_y, const float* shared_logit,
                          int64_t shared_ld, const uint16_t* residual,
                          void* out, bool bf16, hipStream_t s) {
  if (T == 0) return hipSuccess;
  if (w_bf16 && !bf16) return hipErrorInvalidValue;
  // one-wave workgroups: a decode batch's rows spread over every CU (with
  // 256-thread groups T = 64 rows of d = 2048 filled a quarter of them)
  constexpr int kThreads = MLXR_COMBINE_THREADS;
  const dim3 grid((unsigned)((d / 8 + kThreads - 1) / kThreads), (unsigned)T);
  ProfileScope prof("combine", s);
  const float* wf = static_cast<const float*>(w);
  const uint16_t* wh = static_cast<const uint16_t*>(w);
  if (w_bf16)
    combine_kernel<true, uint16_t><<<grid, kThreads, 0, s>>>(
        y, wh, (int)T, (int)K, (int)d, shared_y, shared_logit, shared_ld, residual, out);
  else if (bf16)
    combine_kernel<true, float><<<grid, kThreads, 0, s>>>(
        y, wf, (int)T, (int)K, (int)d, shared_y, shared_logit, shared_ld, residual, out);
  else
    combine_kernel<false, float><<<grid, kThreads, 0, s>>>(
        y, wf, (int)T, (int)K, (int)d, shared_y, shared_logit, shared_ld, residual, out);
  return hipGetLastError();
}

}  // namespace mlxr_moe
