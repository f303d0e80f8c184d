// Grouped quantised expert GEMM (gather_qmm) on gfx950.
//
// Replaces mlx_gather_qmm as called by QuantizedSwitchLinear::apply
// (crates/mlxr-lm/src/nn/switch.rs:148-167 -> crates/mlxr/src/ops/
// quantization.rs:171-221) with transpose = true:
//   out[p, n] = sum_k x[row(p), k] * (code[e, n, k] * scale + bias)
// for every sorted slot p of expert e.  Rows arrive grouped by expert from
// the dispatch, so each expert's packed weights stream from HBM once per
// workgroup tile, however many tokens chose it.
//
// Decode kernel (few rows per expert): HBM-bound.  Weights are never
// dequantised to memory.  Each lane loads its packed words (8 B per group
// for 4-bit, 16 B for 8-bit), expands codes into bf16 registers and feeds
// v_mfma_f32_16x16x32_bf16 with tokens as the M side and output channels
// as the N side.  Per quantisation group g the MFMA yields
//   P = sum x * c'   and   X = sum x
// where c' is the code (8-bit, converted exactly) or 1 + code/16 (4-bit: the
// code is OR-ed into the top four mantissa bits of bf16 1.0, one shift and
// one v_and_or per two codes), and the group's contribution in fp32 is
//   8-bit: scale * P + bias * X
//   4-bit: 16 * scale * P + (bias - 16 * scale) * X.
// Keeping the code in the top mantissa bits keeps P within about 2x of the
// code term it carries, so the offset cancels with little loss (with the code
// in the low bits, 128 + code, the fp32 error of P grows ~8x).
// K (the input dim) is split over 1, 2 or 4 waves when few experts are
// active, so that small T still spreads over all CUs.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {
namespace {

// Reorder 8 consecutive bf16 x values to the code order that unpack4 emits:
// element j of the fragment holds x[perm(j)], perm = 0,4,1,5,2,6,3,7.
__device__ __forceinline__ u32x4_t perm4(u32x4_t v) {
  u32x4_t r;
  r.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
  r.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
  r.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  r.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return r;
}

// 8 nibbles -> bf16 (1 + code/16): nibble k moves to mantissa bits 6..3 of
// its half; pairs (n0,n4) (n1,n5) (n2,n6) (n3,n7).
__device__ __forceinline__ u32x4_t unpack4(uint32_t w) {
  const uint32_t m = 0x00780078u, one = 0x3F803F80u;
  u32x4_t r;
  r.x = ((w << 3) & m) | one;
  r.y = ((w >> 1) & m) | one;
  r.z = ((w >> 5) & m) | one;
  r.w = ((w >> 9) & m) | one;
  return r;
}

// 8 bytes (two words) -> bf16 codes in natural order.  Integers <= 255 are
// exact in bf16, so the top half of the exact f32 is the bf16 value.
__device__ __forceinline__ uint32_t pack_hi(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo),
                               0x07060302u);
}
__device__ __forceinline__ u32x4_t unpack8(uint32_t w0, uint32_t w1) {
  u32x4_t r;
  r.x = pack_hi((float)(w0 & 0xffu), (float)((w0 >> 8) & 0xffu));
  r.y = pack_hi((float)((w0 >> 16) & 0xffu), (float)(w0 >> 24));
  r.z = pack_hi((float)(w1 & 0xffu), (float)((w1 >> 8) & 0xffu));
  r.w = pack_hi((float)((w1 >> 16) & 0xffu), (float)(w1 >> 24));
  return r;
}

template <int BITS>
struct GroupWords;
template <>
struct GroupWords<4> {
  u32x2_t v;
  __device__ __forceinline__ void load(const uint32_t* p, int g4) {
    v = *reinterpret_cast<const u32x2_t*>(p + 2 * g4);
  }
  __device__ __forceinline__ u32x4_t step(int s) const {
    return unpack4(s == 0 ? v.x : v.y);
  }
};
template <>
struct GroupWords<8> {
  u32x4_t v;
  __device__ __forceinline__ void load(const uint32_t* p, int g4) {
    v = *reinterpret_cast<const u32x4_t*>(p + 4 * g4);
  }
  __device__ __forceinline__ u32x4_t step(int s) const {
    return s == 0 ? unpack8(v.x, v.y) : unpack8(v.z, v.w);
  }
};

template <int BITS, bool GATED>
__global__ __launch_bounds__(256) void qgemm_decode_kernel(QGemmArgs a,
                                                           int ks) {
  __shared__ f32x4_t red[4][2][64];
  const int n_act = *a.num_active;
  if ((int)blockIdx.y >= n_act) return;
  const int e = a.active[blockIdx.y];
  const int row0 = a.offsets[e];
  const int rows = a.offsets[e + 1] - row0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cw = 4 / ks;
  const int ct = wave / ks, kslice = wave - ct * ks;
  const int ch = (blockIdx.x * cw + ct) * 16 + (lane & 15);
  const int g4 = lane >> 4;
  const int groups = a.K >> 6;
  const int gps = groups / ks;
  const int G0 = kslice * gps, G1 = G0 + gps;
  constexpr int WPG = 2 * BITS;  // packed words per row per group
  const int64_t wrow = (int64_t)e * a.N + ch;
  const uint32_t* wp0 = a.w0.w + wrow * groups * WPG;
  const uint16_t* sp0 = a.w0.scales + wrow * groups;
  const uint16_t* bp0 = a.w0.biases + wrow * groups;
  const uint32_t* wp1 = GATED ? a.w1.w + wrow * groups * WPG : nullptr;
  const uint16_t* sp1 = GATED ? a.w1.scales + wrow * groups : nullptr;
  const uint16_t* bp1 = GATED ? a.w1.biases + wrow * groups : nullptr;
  const u32x4_t ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};

  for (int tt = 0; tt < rows; tt += 16) {
    const int tok = tt + (lane & 15);
    const bool tv = tok < rows;
    int64_t xrow = 0;
    if (tv) {
      const int slot = row0 + tok;
      xrow = a.row_map ? a.row_map[slot] / a.row_div : slot;
    }
    const uint16_t* xr = a.x + xrow * a.x_ld + 16 * g4;
    f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f};
    f32x4_t acc1 = {0.f, 0.f, 0.f, 0.f};

    auto run = [&](auto U_tag, int G) {
      constexpr int U = decltype(U_tag)::value;
      u32x4_t xa[U][2];
      GroupWords<BITS> q0[U], q1[U];
      uint16_t s0[U], b0[U], s1[U], b1[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        q0[u].load(wp0 + (G + u) * WPG, g4);
        s0[u] = sp0[G + u];
        b0[u] = bp0[G + u];
        if constexpr (GATED) {
          q1[u].load(wp1 + (G + u) * WPG, g4);
          s1[u] = sp1[G + u];
          b1[u] = bp1[G + u];
        }
        if (tv) {
          xa[u][0] = *reinterpret_cast<const u32x4_t*>(xr + 64 * (G + u));
          xa[u][1] = *reinterpret_cast<const u32x4_t*>(xr + 64 * (G + u) + 8);
        } else {
          xa[u][0] = u32x4_t{0u, 0u, 0u, 0u};
          xa[u][1] = u32x4_t{0u, 0u, 0u, 0u};
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        bf16x8_t A0, A1;
        if constexpr (BITS == 4) {
          A0 = as_bf16x8(perm4(xa[u][0]));
          A1 = as_bf16x8(perm4(xa[u][1]));
        } else {
          A0 = as_bf16x8(xa[u][0]);
          A1 = as_bf16x8(xa[u][1]);
        }
        const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
        f32x4_t X = mfma16x16x32(A0, as_bf16x8(ones), zero);
        X = mfma16x16x32(A1, as_bf16x8(ones), X);
        f32x4_t P0 = mfma16x16x32(A0, as_bf16x8(q0[u].step(0)), zero);
        P0 = mfma16x16x32(A1, as_bf16x8(q0[u].step(1)), P0);
        const float s0f = bf16_to_f32(s0[u]);
        const float bi0 = bf16_to_f32(b0[u]);
        const float sc0 = BITS == 4 ? 16.0f * s0f : s0f;
        const float c0 = BITS == 4 ? __builtin_fmaf(-16.0f, s0f, bi0) : bi0;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc0[r] = __builtin_fmaf(sc0, P0[r], __builtin_fmaf(c0, X[r], acc0[r]));
        if constexpr (GATED) {
          f32x4_t P1 = mfma16x16x32(A0, as_bf16x8(q1[u].step(0)), zero);
          P1 = mfma16x16x32(A1, as_bf16x8(q1[u].step(1)), P1);
          const float s1f = bf16_to_f32(s1[u]);
          const float bi1 = bf16_to_f32(b1[u]);
          const float sc1 = BITS == 4 ? 16.0f * s1f : s1f;
          const float c1 = BITS == 4 ? __builtin_fmaf(-16.0f, s1f, bi1) : bi1;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc1[r] =
                __builtin_fmaf(sc1, P1[r], __builtin_fmaf(c1, X[r], acc1[r]));
        }
      }
    };
    int G = G0;
    for (; G + 4 <= G1; G += 4)
      run(std::integral_constant<int, 4>{}, G);
    for (; G < G1; ++G) run(std::integral_constant<int, 1>{}, G);

    if (ks > 1) {
      red[wave][0][lane] = acc0;
      if constexpr (GATED) red[wave][1][lane] = acc1;
      __syncthreads();
      if (kslice == 0) {
        for (int q = 1; q < ks; ++q) {
          acc0 += red[wave + q][0][lane];
          if constexpr (GATED) acc1 += red[wave + q][1][lane];
        }
      }
      __syncthreads();
    }
    if (kslice == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tt + 4 * g4 + r;
        if (t < rows) {
          const int slot = row0 + t;
          if constexpr (GATED) {
            const uint16_t v =
                swiglu_bf16(bf16_round(acc0[r]), bf16_round(acc1[r]));
            a.out[(int64_t)slot * a.out_ld + ch] = v;
          } else {
            const int64_t orow = a.out_map ? a.out_map[slot] : slot;
            a.out[orow * a.out_ld + ch] = f32_to_bf16(acc0[r]);
          }
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_qgemm(const QGemmArgs& a, int64_t total_rows,
                        int64_t max_active, bool prefill, hipStream_t s) {
  (void)prefill;
  (void)total_rows;
  if (max_active <= 0) return hipSuccess;
  const int groups = a.K / 64;
  // Workgroups at ks = 1: one per (active expert, 64 output channels).
  const int64_t wg1 = max_active * (a.N / 64);
  int ks = 1;
  if (wg1 < 1024 && groups % 2 == 0 && a.N % 32 == 0) ks = 2;
  if (wg1 * 2 < 1024 && groups % 4 == 0 && a.N % 16 == 0) ks = 4;
  const int cw = 4 / ks;
  const dim3 grid((unsigned)(a.N / (16 * cw)), (unsigned)max_active);
  ProfileScope prof(a.gated ? "qgemm_gated" : "qgemm_down", s);
#define MLXR_QG(B, G) qgemm_decode_kernel<B, G><<<grid, 256, 0, s>>>(a, ks)
  if (a.bits == 4)
    a.gated ? MLXR_QG(4, true) : MLXR_QG(4, false);
  else
    a.gated ? MLXR_QG(8, true) : MLXR_QG(8, false);
#undef MLXR_QG
  return hipGetLastError();
}

}  // namespace mlxr_moe
