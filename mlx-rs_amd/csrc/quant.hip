// MLX affine quantise / dequantise on gfx950.
//
// Replaces mlx_quantize / mlx_dequantize as called from
// crates/mlxr/src/ops/quantization.rs:47-70 and :118-146.  Layout
// (crates/mlxr-lm/src/attention/kernel_source.rs:30-35,96-107):
//   wq [rows, cols*bits/32] uint32, element k of a word at bits
//   [k*bits, (k+1)*bits); scales/biases [rows, cols/group] in w's dtype.
// Setup-time kernels: HBM-bound, one thread per group / per packed word.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {
namespace {

template <bool BF16>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if constexpr (BF16)
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else
    return static_cast<const float*>(p)[i];
}
template <bool BF16>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
  if constexpr (BF16)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else
    static_cast<float*>(p)[i] = v;
}

// One thread per quantisation group.  fp32 recipe of MLX's affine
// quantiser: scale = max((max-min)/n_bins, 1e-7) signed towards the edge of
// larger magnitude, snapped so that the edge is an exact code; codes use
// the unrounded scale and bias; scale and bias are stored in w's dtype.
template <bool BF16>
__global__ __launch_bounds__(256) void quantize_kernel(
    const void* __restrict__ w, int64_t rows, int64_t cols, int gs, int bits,
    uint32_t* __restrict__ wq, void* __restrict__ scales,
    void* __restrict__ biases) {
  const int64_t groups = cols / gs;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * groups) return;
  const int64_t r = gid / groups, g = gid % groups;
  const int64_t base = r * cols + g * gs;
  const float n_bins = (float)((1 << bits) - 1);
  float wmax = -INFINITY, wmin = INFINITY;
  for (int j = 0; j < gs; ++j) {
    const float v = ld<BF16>(w, base + j);
    wmax = fmaxf(wmax, v);
    wmin = fminf(wmin, v);
  }
  const bool neg_edge = fabsf(wmin) > fabsf(wmax);
  float scale = fmaxf((wmax - wmin) / n_bins, 1e-7f);
  scale = neg_edge ? scale : -scale;
  const float edge = neg_edge ? wmin : wmax;
  const float q0 = rintf(edge / scale);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  const int per_word = 32 / bits;
  uint32_t* out = wq + r * (cols / per_word) + g * gs / per_word;
  for (int wi = 0; wi < gs / per_word; ++wi) {
    uint32_t word = 0;
    for (int k = 0; k < per_word; ++k) {
      const float v = ld<BF16>(w, base + wi * per_word + k);
      float q = rintf((v - bias) / scale);
      q = fminf(fmaxf(q, 0.0f), n_bins);
      word |= (uint32_t)q << (k * bits);
    }
    out[wi] = word;
  }
  st<BF16>(scales, gid, scale);
  st<BF16>(biases, gid, bias);
}

// One thread per packed word: code * scale + bias as one fma, rounded once.
template <bool SB_BF16, bool OUT_BF16>
__global__ __launch_bounds__(256) void dequantize_kernel(
    const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, int64_t rows, int64_t cols, int gs,
    int bits, void* __restrict__ out) {
  const int per_word = 32 / bits;
  const int64_t words = rows * cols / per_word;
  const int64_t wid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (wid >= words) return;
  const int64_t col0 = (wid * per_word) % cols;
  const int64_t r = (wid * per_word) / cols;
  const int64_t sidx = r * (cols / gs) + col0 / gs;
  const float s = ld<SB_BF16>(scales, sidx);
  const float b = ld<SB_BF16>(biases, sidx);
  const uint32_t word = wq[wid];
  const uint32_t mask = (1u << bits) - 1u;
  for (int k = 0; k < per_word; ++k) {
    const float code = (float)((word >> (k * bits)) & mask);
    st<OUT_BF16>(out, r * cols + col0 + k, __builtin_fmaf(code, s, b));
  }
}

}  // namespace

hipError_t launch_quantize(const void* w, bool w_bf16, int64_t rows,
                           int64_t cols, int group_size, int bits, uint32_t* wq,
                           void* scales, void* biases, hipStream_t s) {
  const int64_t n = rows * (cols / group_size);
  if (n == 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (w_bf16)
    quantize_kernel<true><<<grid, 256, 0, s>>>(w, rows, cols, group_size, bits,
                                               wq, scales, biases);
  else
    quantize_kernel<false><<<grid, 256, 0, s>>>(w, rows, cols, group_size,
                                                bits, wq, scales, biases);
  return hipGetLastError();
}

hipError_t launch_dequantize(const uint32_t* wq, const void* scales,
                             const void* biases, bool sb_bf16, int64_t rows,
                             int64_t cols, int group_size, int bits, void* out,
                             bool out_bf16, hipStream_t s) {
  const int64_t words = rows * cols / (32 / bits);
  if (words == 0) return hipSuccess;
  const dim3 grid((unsigned)((words + 255) / 256));
#define MLXR_DQ(SB, OB)                                                     \
  dequantize_kernel<SB, OB><<<grid, 256, 0, s>>>(wq, scales, biases, rows, \
                                                 cols, group_size, bits, out)
  if (sb_bf16 && out_bf16)
    MLXR_DQ(true, true);
  else if (sb_bf16)
    MLXR_DQ(true, false);
  else if (out_bf16)
    MLXR_DQ(false, true);
  else
    MLXR_DQ(false, false);
#undef MLXR_DQ
  return hipGetLastError();
}

}  // namespace mlxr_moe
