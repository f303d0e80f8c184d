// Shared device helpers for the MI355X (gfx950) MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlxr_moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// bf16 <-> f32.  Round-to-nearest-even, NaN -> 0x7FC0; bit-identical to the
// conversion every CPU-side check uses.
__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float((uint32_t)h << 16);
}
__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_round(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// D = A(16x32) * B(32x16) + C.  Lane l supplies A[l%16][8(l/16)+j] and
// B[8(l/16)+j][l%16]; it receives D[4(l/16)+r][l%16], r = 0..3.
__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b,
                                                f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// D = A(32x16) * B(16x32) + C.  Lane l supplies A[l%32][8(l/32)+j] and
// B[8(l/32)+j][l%32]; it receives D[8(r/4)+4(l/32)+r%4][l%32], r = 0..15.
__device__ __forceinline__ f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b,
                                                 f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// silu(g) * u with the reference's per-op bf16 rounding
// (crates/mlxr-lm/src/activations.rs:187-200; activation.rs:869-873).
// g and u are already bf16 values held in f32.
__device__ __forceinline__ uint16_t swiglu_bf16(float g, float u) {
  const float sg = bf16_round(1.0f / (1.0f + expf(-g)));
  const float h = bf16_round(g * sg);
  return f32_to_bf16(h * u);
}

// gelu_approx(g) * u with the reference's bf16 rounding points
// (gelu_approximate_in_dtype, crates/mlxr-lm/src/activations.rs:246-259:
// every op in the input dtype, the constants cast to bf16 first):
// 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).  g and u are bf16 values
// held in f32.
__device__ __forceinline__ uint16_t geglu_bf16(float g, float u) {
  const float k = 0.044677734375f;  // bf16(0.044715)
  const float c = 0.796875f;        // bf16(sqrt(2 / pi))
  const float x3 = bf16_round(bf16_round(g * g) * g);
  const float inner = bf16_round(g + bf16_round(k * x3));
  const float t = bf16_round(tanhf(bf16_round(c * inner)));
  const float gl = bf16_round(bf16_round(0.5f * g) * bf16_round(1.0f + t));
  return f32_to_bf16(gl * u);
}

// The gated GEMMs' activation: act(g, u) for g and u bf16 values in f32.
__device__ __forceinline__ uint16_t gated_act_bf16(int act, float g, float u) {
  return act == 1 ? geglu_bf16(g, u) : swiglu_bf16(g, u);
}

// The combine's arithmetic for one output element
// (combine_with_weights, crates/mlxr-lm/src/nn/switch.rs:223-234: w * y
// promoted to f32, summed over k in order; the block's shared branch,
// qwen3_5/text/moe.rs:117-120,145; the decoder layer's residual add,
// layer.rs:138).  BF16: the quantised router's bf16 chain, every op rounded
// to bf16.  A sum is combine_add over k = 0..K-1 from 0, bf16-rounded (BF16),
// then combine_shared, then combine_residual.  Every kernel that combines
// uses these, so they agree bit for bit.
template <bool BF16>
__device__ __forceinline__ float combine_add(float acc, float w, float y) {
  float p = __fmul_rn(w, y);
  if (BF16) p = bf16_round(p);
  return __fadd_rn(acc, p);
}
template <bool BF16>
__device__ __forceinline__ float combine_gate(float logit) {
  float g = 1.0f / (1.0f + expf(-logit));
  if (BF16) g = bf16_round(g);
  return g;
}
template <bool BF16>
__device__ __forceinline__ float combine_shared(float acc, float sy, float gate) {
  float p = __fmul_rn(sy, gate);
  if (BF16) p = bf16_round(p);
  return __fadd_rn(p, acc);
}
template <bool BF16>
__device__ __forceinline__ float combine_residual(float acc, float h) {
  // h + mlp_out, with mlp_out in its own dtype first
  const float m = BF16 ? bf16_round(acc) : acc;
  return __fadd_rn(h, m);
}

__device__ __forceinline__ float wave_sum_butterfly(float v) {
  // v += v[l ^ m] for m = 32, 16, 8, 4, 2, 1: every lane ends with the
  // same bits, and the CPU restatement reproduces the association.
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

}  // namespace mlxr_moe
