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
// dequantised to memory: every lane loads 16 contiguous bytes of its row per
// step (the width that streams at full HBM rate), expands the codes into bf16
// registers and feeds v_mfma_f32_16x16x32_bf16 with tokens as the M side and
// output channels as the N side.  Per quantisation group g the MFMAs yield
//   P = sum x * c'   and   X = sum x
// where c' is the code (8-bit, converted exactly) or 1 + code/16 (4-bit: the
// code is OR-ed into the top four mantissa bits of bf16 1.0, one shift and
// one v_and_or per two codes), and the group's contribution in fp32 is
//   8-bit: scale * P + bias * X
//   4-bit: 16 * scale * P + (bias - 16 * scale) * X.
// Keeping the code in the top mantissa bits keeps P within about 2x of the
// code term it carries, so the offset cancels with little loss (with the code
// in the low bits, 128 + code, the fp32 error of P grows ~8x).
// The input dim is split over the waves of a workgroup (two groups per wave
// per pass) so each wave keeps its x slice in registers and re-reads only
// weights; the partial sums meet in LDS.
// Dense bf16 weights (gather_mm, bits 16) run the same split-K kernel with
// the weights as the MFMA operand and no group terms (P alone), or the
// M-tiled kernel for many rows per expert.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {
namespace {

// Launch shape of the streaming kernel: (experts x 16-channel blocks) from
// which it runs, waves per workgroup, super-steps of loads in flight at 4-
// and 8-bit.
// (measured at T = 1..4: the streaming kernel's time is nearly flat in the
// blocks there, ~11.8 us for c2/c4 gate/up, while the split-K kernel's
// grows with the bytes: 10.1 us at 8 experts x 512 channels (288 blocks),
// 13.7 at 10 x 512 (352) and 8 x 768 (432))
#ifndef MLXR_STREAM_MIN_BLOCKS
#define MLXR_STREAM_MIN_BLOCKS 320
#endif
#ifndef MLXR_STREAM_WAVES
#define MLXR_STREAM_WAVES 4
#endif
#ifndef MLXR_STREAM_DEPTH4
#define MLXR_STREAM_DEPTH4 1
#endif
#ifndef MLXR_STREAM_DEPTH8
#define MLXR_STREAM_DEPTH8 1
#endif
// ... of the 8-token form (half the bytes per super-step: twice the depth)
#ifndef MLXR_STREAM_DEPTH4_TT8
#define MLXR_STREAM_DEPTH4_TT8 (2 * MLXR_STREAM_DEPTH4)
#endif
#ifndef MLXR_STREAM_DEPTH8_TT8
#define MLXR_STREAM_DEPTH8_TT8 (2 * MLXR_STREAM_DEPTH8)
#endif
// ... and of the gated kernels (gate and up: two rows of loads per step).
// The 4-bit gated 8-token form keeps three super-steps in flight: a ring
// of four slots divides its 16 super-steps at K = 2048 (with three slots two
// zero steps follow the last one).  Measured (event means, c2 T=8/32/64,
// c4 T=64, c6 T=64): gate/up 0.3-1% faster; depth 3 for the 4-token form
// was 2-12% slower.
#ifndef MLXR_STREAM_DEPTH4G
#define MLXR_STREAM_DEPTH4G MLXR_STREAM_DEPTH4
#endif
#ifndef MLXR_STREAM_DEPTH4G_TT8
#define MLXR_STREAM_DEPTH4G_TT8 3
#endif
#ifndef MLXR_STREAM_DEPTH8G
#define MLXR_STREAM_DEPTH8G MLXR_STREAM_DEPTH8
#endif
#ifndef MLXR_STREAM_DEPTH8G_TT8
#define MLXR_STREAM_DEPTH8G_TT8 (2 * MLXR_STREAM_DEPTH8G)
#endif
#ifndef MLXR_SCHED_BARRIER
#define MLXR_SCHED_BARRIER() __builtin_amdgcn_sched_barrier(0)
#endif

constexpr int64_t kStreamMinBlocks = MLXR_STREAM_MIN_BLOCKS;
// 16-channel blocks per wave of the down kernel, at most (1, 2 or 4; the
// launcher halves it until the grid keeps every slot busy)
#ifndef MLXR_STREAM_MAX_NB
#define MLXR_STREAM_MAX_NB 4
#endif
// four blocks per wave only while the grid stays this many times the slots
// (many small items: c4 T=512 down 157 to 141 µs, c6 T=320 91 to 85; with
// 4x the slots c2 T=128 down went 45.8 to 50.0)
#ifndef MLXR_STREAM_NB4_GRIDS
#define MLXR_STREAM_NB4_GRIDS 8
#endif
// ... and of the gated kernel (1 or 2)
#ifndef MLXR_STREAM_GATED_NB
#define MLXR_STREAM_GATED_NB 1
#endif
#ifndef MLXR_STREAM_SLOTS
#define MLXR_STREAM_SLOTS 512
#endif
// largest grid that K-slices may make (one workgroup per slot)
#ifndef MLXR_STREAM_KS_GRID
#define MLXR_STREAM_KS_GRID 512
#endif
// workgroups resident at once (2 per CU on 256 CUs)
constexpr int64_t kStreamSlots = MLXR_STREAM_SLOTS;


// quantisation groups of the input dim per wave and pass in the split-K
// kernel (its waves split the input dim; more groups per wave, fewer waves)
#ifndef MLXR_SPLITK_GROUPS
#define MLXR_SPLITK_GROUPS 4
#endif

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
// its half; pairs (n0,n4) (n1,n5) (n2,n6) (n3,n7).  Written as one shift and
// one v_and_or_b32 per output: a VOP3 op takes one scalar operand here, so
// the mask rides in an SGPR and the bf16 1.0 pair in a VGPR (`one`).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m,
                                           uint32_t one) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(one));
  return r;
}
__device__ __forceinline__ u32x4_t unpack4(uint32_t w, uint32_t one) {
  const uint32_t m = 0x00780078u;
  u32x4_t r;
  r.x = and_or(w << 3, m, one);
  r.y = and_or(w >> 1, m, one);
  r.z = and_or(w >> 5, m, one);
  r.w = and_or(w >> 9, m, one);
  return r;
}
__device__ __forceinline__ u32x4_t unpack4(uint32_t w) {
  return unpack4(w, 0x3F803F80u);
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

// One "step" of a wave is one 16-byte load per lane per row: at 4-bit two
// adjacent quantisation groups (64 B of the row; lanes q = 0,1 hold the two
// halves of the first group, q = 2,3 of the second), at 8-bit one group
// (64 B; lane q holds bytes 16q..16q+15).  Each MFMA sum must cover a single
// group (its own scale and bias), so at 4-bit the x operand exists twice per
// step, zero on the lanes of the other group: xa feeds the first group's
// sums, xb the second's, and the weight operand is shared.
// Dense bf16 weights (BITS 16) take two 16-byte loads per lane per step:
// one group of 64 weights per row, lane q holding weights 16q..16q+15 (the
// 8-bit lane layout), and no scales or biases.
template <int NM, int SPW, int WV = 1>
struct StepBuf {
  u32x4_t w[NM][SPW][WV];
  uint32_t s[NM][SPW];  // bf16 scales: 4-bit (first | second << 16), 8-bit g
  uint32_t b[NM][SPW];  // bf16 biases, same packing
};
template <int BITS>
constexpr int kStepWords = BITS == 16 ? 2 : 1;  // 16-byte loads per step

// Scale or bias bits of one step: both groups at 4-bit (one u32 when
// 4-byte aligned), the one group at 8-bit.
__device__ __forceinline__ uint32_t load_sb(const uint16_t* p, bool pair,
                                            bool two) {
  if (pair) return *reinterpret_cast<const uint32_t*>(p);
  return (uint32_t)p[0] | (two ? (uint32_t)p[1] << 16 : 0u);
}

// Loads of one 16-channel block: row `wrow` (this lane's channel), groups
// [G0, G0 + mg) of this wave.  Nothing past the row's last group is read.
template <int BITS, int NM, int SPW>
__device__ __forceinline__ void load_steps(StepBuf<NM, SPW, kStepWords<BITS>>& bb,
                                           const QGemmArgs& a, int64_t wrow,
                                           int groups, int G0, int mg, int q,
                                           bool sb_pairs) {
  constexpr int GPS = BITS == 4 ? 2 : 1;
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const QWeights& W = m == 0 ? a.w0 : a.w1;
    const uint32_t* wr = W.w + wrow * groups * (2 * BITS);
#pragma unroll
    for (int st = 0; st < SPW; ++st) {
      const int g0 = G0 + GPS * st;  // first group of the step
#pragma unroll
      for (int v = 0; v < kStepWords<BITS>; ++v) bb.w[m][st][v] = u32x4_t{0u, 0u, 0u, 0u};
      bb.s[m][st] = 0u;
      bb.b[m][st] = 0u;
      if (GPS * st < mg) {
        if constexpr (BITS == 16) {
          // weights 16q..16q+7 and 16q+8..16q+15 of the group (32 words)
          const uint32_t* p = wr + g0 * 32 + 8 * q;
          bb.w[m][st][0] = *reinterpret_cast<const u32x4_t*>(p);
          bb.w[m][st][1] = *reinterpret_cast<const u32x4_t*>(p + 4);
        } else if constexpr (BITS == 4) {
          const uint16_t* sr = W.scales + wrow * groups;
          const uint16_t* br = W.biases + wrow * groups;
          const int gl = g0 + (q >> 1);  // this lane's group
          if (gl < G0 + mg)
            bb.w[m][st][0] = *reinterpret_cast<const u32x4_t*>(
                wr + gl * 8 + 4 * (q & 1));
          const bool two = g0 + 1 < G0 + mg;
          bb.s[m][st] = load_sb(sr + g0, sb_pairs && two, two);
          bb.b[m][st] = load_sb(br + g0, sb_pairs && two, two);
        } else {
          const uint16_t* sr = W.scales + wrow * groups;
          const uint16_t* br = W.biases + wrow * groups;
          bb.w[m][st][0] =
              *reinterpret_cast<const u32x4_t*>(wr + g0 * 16 + 4 * q);
          bb.s[m][st] = sr[g0];
          bb.b[m][st] = br[g0];
        }
      }
    }
  }
}

// sc * P + cb * X terms of one group from its bf16 scale and bias bits.
template <int BITS>
__device__ __forceinline__ void group_terms(uint32_t s16, uint32_t b16,
                                            float& sc, float& cb) {
  const float sf = __uint_as_float(s16 << 16);
  const float bf = __uint_as_float(b16 << 16);
  if constexpr (BITS == 4) {
    sc = 16.0f * sf;
    cb = __builtin_fmaf(-16.0f, sf, bf);
  } else {
    sc = sf;
    cb = bf;
  }
}

// Decode grouped GEMM.  One workgroup = kw waves = one (active expert, tile
// of CB*16 output channels).  Wave w owns SPW steps of the input dim per
// pass; passes repeat until the kw waves have covered it.  Per 16-token chunk
// of the expert's rows a wave issues the weight loads of the tile's first
// block, loads its slice of x into registers (MFMA A operand) with the
// per-group token sums X, then multiplies block i while the loads of block
// i+1 are in flight.  The kw partial sums of each block meet in LDS and one
// wave writes the block.  Lane l: token / channel l%16, quarter l/16.
template <int BITS, bool GATED, int SPW, int CB>
__device__ __forceinline__ void decode_body(const QGemmArgs& a, int tile,
                                            const int32_t* rec, int4 wk,
                                            int4 fr0, int4 fr1) {
  extern __shared__ f32x4_t red[];  // [kw][CB][NM][64]
  constexpr int NM = GATED ? 2 : 1;
  constexpr int GPS = BITS == 4 ? 2 : 1;
  constexpr int GW = SPW * GPS;          // groups per wave per pass
  constexpr int NX = BITS == 4 ? 4 : 2;  // x fragments per step
  const int kw = blockDim.x >> 6;
  const int e = wk.x, row0 = wk.y, rows = wk.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int groups = a.K >> 6;
  const int per_pass = kw * GW;
  const int passes = (groups + per_pass - 1) / per_pass;
  const bool sb_pairs = (groups & 1) == 0;  // steps start on even groups
  const u32x4_t ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const u32x4_t zq = {0u, 0u, 0u, 0u};
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  const int64_t wrow0 = (int64_t)e * a.e_rows + (int64_t)tile * CB * 16 + c;

  for (int tt = 0; tt < rows; tt += 16) {
    const int tok = tt + c;
    const bool tv = tok < rows;
    int64_t xrow = 0;
    if (tv) {
      const int slot = row0 + tok;
      // this lane's flat row from the record (tok < kWorkRows = 8)
      const int f4 = (tok & 3) == 0 ? fr0.x : (tok & 3) == 1 ? fr0.y : (tok & 3) == 2 ? fr0.z : fr0.w;
      const int f8 = (tok & 3) == 0 ? fr1.x : (tok & 3) == 1 ? fr1.y : (tok & 3) == 2 ? fr1.z : fr1.w;
      const int flat = tok < 4 ? f4 : f8;
      xrow = a.x_by_slot ? slot : (a.row_map ? a.row_map[flat] : flat / a.row_div);
    }
    f32x4_t acc[CB][NM];
#pragma unroll
    for (int bi = 0; bi < CB; ++bi)
#pragma unroll
      for (int m = 0; m < NM; ++m) acc[bi][m] = zero;

    for (int pass = 0; pass < passes; ++pass) {
      const int G0 = pass * per_pass + wave * GW;
      const int mg = max(0, min(GW, groups - G0));
      StepBuf<NM, SPW, kStepWords<BITS>> buf[CB > 1 ? 2 : 1];
      load_steps<BITS, NM, SPW>(buf[0], a, wrow0, groups, G0, mg, q,
                                sb_pairs);
      // x slice (A operand) and the per-group sums X
      bf16x8_t xa[SPW][NX], xb[SPW][NX];
      f32x4_t XA[SPW], XB[SPW];
#pragma unroll
      for (int st = 0; st < SPW; ++st) {
        const int g0 = G0 + GPS * st;
        if constexpr (BITS == 4) {
          const int gl = g0 + (q >> 1);
          const bool in = tv && GPS * st < mg && gl < G0 + mg;
          const uint16_t* xr = a.x + xrow * a.x_ld + 64 * gl + 32 * (q & 1);
#pragma unroll
          for (int i = 0; i < NX; ++i) {
            u32x4_t v = zq;
            if (in) v = *reinterpret_cast<const u32x4_t*>(xr + 8 * i);
            v = perm4(v);
            xa[st][i] = as_bf16x8((q >> 1) ? zq : v);
            xb[st][i] = as_bf16x8((q >> 1) ? v : zq);
          }
        } else {
          const bool in = tv && st < mg;
          const uint16_t* xr = a.x + xrow * a.x_ld + 64 * g0 + 16 * q;
#pragma unroll
          for (int i = 0; i < NX; ++i) {
            u32x4_t v = zq;
            if (in) v = *reinterpret_cast<const u32x4_t*>(xr + 8 * i);
            xa[st][i] = as_bf16x8(v);
          }
        }
      }
#pragma unroll
      for (int st = 0; st < SPW; ++st) {
        XA[st] = zero;
        XB[st] = zero;
        if constexpr (BITS == 16) continue;  // no bias term
#pragma unroll
        for (int i = 0; i < NX; ++i) {
          XA[st] = mfma16x16x32(xa[st][i], as_bf16x8(ones), XA[st]);
          if constexpr (BITS == 4)
            XB[st] = mfma16x16x32(xb[st][i], as_bf16x8(ones), XB[st]);
        }
      }
#pragma unroll
      for (int bi = 0; bi < CB; ++bi) {
        if (bi + 1 < CB)
          load_steps<BITS, NM, SPW>(buf[(bi + 1) & 1], a,
                                    wrow0 + (bi + 1) * 16, groups, G0, mg, q,
                                    sb_pairs);
        const StepBuf<NM, SPW, kStepWords<BITS>>& cur = buf[bi & 1];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          f32x4_t ac = acc[bi][m];
#pragma unroll
          for (int st = 0; st < SPW; ++st) {
            if (GPS * st < mg) {
              const u32x4_t wv = cur.w[m][st][0];
              if constexpr (BITS == 16) {
                // the weights are the B operand as they are
                f32x4_t P = mfma16x16x32(xa[st][0], as_bf16x8(wv), zero);
                P = mfma16x16x32(xa[st][1], as_bf16x8(cur.w[m][st][kStepWords<BITS> - 1]), P);
#pragma unroll
                for (int r = 0; r < 4; ++r) ac[r] += P[r];
              } else if constexpr (BITS == 4) {
                f32x4_t PA = zero, PB = zero;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  const bf16x8_t u = as_bf16x8(unpack4(wv[i]));
                  PA = mfma16x16x32(xa[st][i], u, PA);
                  PB = mfma16x16x32(xb[st][i], u, PB);
                }
                float sA, cA, sB, cB;
                group_terms<4>(cur.s[m][st] & 0xffffu,
                               cur.b[m][st] & 0xffffu, sA, cA);
                group_terms<4>(cur.s[m][st] >> 16, cur.b[m][st] >> 16, sB,
                               cB);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  ac[r] = __builtin_fmaf(
                      sA, PA[r], __builtin_fmaf(cA, XA[st][r], ac[r]));
                  ac[r] = __builtin_fmaf(
                      sB, PB[r], __builtin_fmaf(cB, XB[st][r], ac[r]));
                }
              } else {
                f32x4_t P = mfma16x16x32(
                    xa[st][0], as_bf16x8(unpack8(wv.x, wv.y)), zero);
                P = mfma16x16x32(xa[st][1], as_bf16x8(unpack8(wv.z, wv.w)),
                                 P);
                float sc, cb;
                group_terms<8>(cur.s[m][st], cur.b[m][st], sc, cb);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  ac[r] = __builtin_fmaf(
                      sc, P[r], __builtin_fmaf(cb, XA[st][r], ac[r]));
              }
            }
          }
          acc[bi][m] = ac;
        }
      }
    }
#pragma unroll
    for (int bi = 0; bi < CB; ++bi)
#pragma unroll
      for (int m = 0; m < NM; ++m)
        red[((wave * CB + bi) * NM + m) * 64 + lane] = acc[bi][m];
    __syncthreads();
    // block bi is summed and written by wave bi % kw
    for (int bi = wave; bi < CB; bi += kw) {
      f32x4_t s0 = zero, s1 = zero;
      for (int w = 0; w < kw; ++w) {
        s0 += red[((w * CB + bi) * NM) * 64 + lane];
        if constexpr (GATED) s1 += red[((w * CB + bi) * NM + 1) * 64 + lane];
      }
      const int ch = (tile * CB + bi) * 16 + c;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tt + 4 * q + r;
        if (t < rows) {
          const int slot = row0 + t;
          if constexpr (GATED) {
            a.out[(int64_t)slot * a.out_ld + ch] =
                gated_act_bf16(a.act, bf16_round(s0[r]), bf16_round(s1[r]));
          } else {
            const int64_t orow = a.out_by_flat ? rec[4 + t] : slot;
            a.out[orow * a.out_ld + ch] = f32_to_bf16(s0[r]);
          }
        }
      }
    }
    __syncthreads();
  }
}

// The unit of workgroup blockIdx.x: a work item of the routed problem `a`
// (its record, fetched whole: header and flat rows), or, from units1 on,
// an item of a folded second problem -- the block's shared expert, every
// token's row once: item i is rows 8i..8i+7 of `rows2` in token order, its
// record made here (expert 0, the rows' own slots, no dispatch).  Returns
// false for an idle workgroup (past the routed problem's items).
struct Unit {
  const int32_t* rec;
  int4 wk, fr0, fr1;
  int tile;
  bool shared;
};
__device__ __forceinline__ bool decode_unit(const QGemmArgs& a, int tiles_n,
                                            int units1, int items1, int rows2,
                                            Unit& u) {
  u.shared = (int)blockIdx.x >= units1;
  const int v = u.shared ? (int)blockIdx.x - units1 : (int)blockIdx.x;
  const int ai = v / tiles_n;
  u.tile = v - ai * tiles_n;
  // (the routed record is read unconditionally, item 0's for a shared
  // unit)
  u.rec = a.work + (int64_t)kWorkInts * (u.shared ? 0 : min(ai, items1 - 1));
  u.wk = *reinterpret_cast<const int4*>(u.rec);
  u.fr0 = *reinterpret_cast<const int4*>(u.rec + 4);
  u.fr1 = *reinterpret_cast<const int4*>(u.rec + 8);
  const int n_act = *a.num_work;
  if (u.shared) {
    const int r0 = kWorkRows * ai;
    u.wk = make_int4(0, r0, min(kWorkRows, rows2 - r0), rows2);
    u.fr0 = make_int4(r0, r0 + 1, r0 + 2, r0 + 3);
    u.fr1 = make_int4(r0 + 4, r0 + 5, r0 + 6, r0 + 7);
    return true;
  }
  return ai < n_act;
}

template <int BITS, bool GATED, int SPW, int CB>
__global__ __launch_bounds__(1024) void qgemm_decode_kernel(
    QGemmArgs a, int tiles_n, QGemmArgs a2, int units1, int items1, int rows2) {
  Unit u;
  if (!decode_unit(a, tiles_n, units1, items1, rows2, u)) return;
  decode_body<BITS, GATED, SPW, CB>(u.shared ? a2 : a, u.tile, u.rec, u.wk,
                                    u.fr0, u.fr1);
}

// Streaming decode GEMM for many (work item, channel tile) units.  One
// workgroup = `waves` waves = one work item (at most 8 rows of one expert)
// x one tile of waves*nb*16 output channels; wave w owns nb 16-channel
// blocks over the whole input dim, so no partial sums cross waves.  The
// workgroup stages the item's x rows (bf16, in the MFMA operand order) and
// the per-group token sums X in LDS once; each wave then streams its
// blocks' packed weights with D super-steps of loads in flight (a register
// ring) and reads x from LDS.
//
// Prologue order: the work record (one scalar load: the expert and the flat
// row of each slot, so the x rows need no further lookup), then the first D
// weight super-steps, the wave's scales and biases and the x rows are all
// issued before the first LDS store, so the weight stream starts one memory
// round trip after the workgroup does.
//
// Block-diagonal MFMA: the 16 rows of the A operand are TT tokens x GG
// groups (GG = 16 / TT).  Lane quarter q (l/16) supplies the codes of group
// q*GG/4 of the super-step, and the x operand row (group j, token t) is
// non-zero only on the lanes of group j, so one v_mfma_f32_16x16x32_bf16
// yields the partial sums of GG groups at once and every lane applies the
// scale and bias of a single group.  A super-step covers GG groups; each
// lane loads 16*GG codes of its group (16 B per load).  Lanes that feed
// zeros read a zero block in LDS.  The GG partial sums of a token meet by
// cross-lane adds at the end.
template <int BITS, bool GATED, int TT, int D, int NB, int KS>
__device__ __forceinline__ void stream_body(const QGemmArgs& a,
                                            const int32_t* rec, int4 wk,
                                            int4 fr0, int4 fr1, int tile,
                                            char* smem, int ltid, int lthreads,
                                            uint16_t* yl, int yrow_off) {
  constexpr int nb = NB;
  static_assert(kWorkRows <= 8, "an item of a >4-row expert fits TT = 8");
  constexpr int NM = GATED ? 2 : 1;
  constexpr int NA = 2 * NM;            // scale and bias arrays
  constexpr int GG = 16 / TT;           // groups per MFMA
  constexpr int LPG = 4 / GG;           // lane quarters per group
  constexpr int CPL = 64 / LPG;         // codes per lane per super-step
  constexpr int NL = CPL * BITS / 128;  // 16-byte loads per lane
  constexpr int NMF = CPL / 8;          // MFMAs per super-step
  constexpr int WPG = 2 * BITS;         // packed words per row and group
  // KS waves share each set of blocks, one K-slice each (KS > 1 for small
  // grids: more, shorter waves); their sums meet in LDS at the end
  const int waves = (lthreads >> 6) / KS;  // channel waves
  // items of experts with at most 4 rows run with TT = 4, the others with
  // TT = 8 >= kWorkRows: an item is always one pass
  const int e = wk.x, row0 = wk.y, nt = min(wk.z, TT);
  const int lane = ltid & 63, wave_id = ltid >> 6;
  const int wave = wave_id / KS, kq = wave_id % KS;  // channel wave, K-slice
  const int n = lane & 15, q = lane >> 4;
  const int gq = q / LPG, sq = q % LPG;  // this lane's group, its part
  const int K = a.K, groups = K >> 6;
  const int ssteps = groups / GG;  // the host runs this kernel when GG | groups
  const int ssk = ssteps / KS;     // ... and KS | ssteps: steps per slice
  const int s0 = kq * ssk;         // this wave's first step of each block
  const int total = nb * ssk;      // super-steps of this wave, all blocks
  // LDS: x [TT][K + 8] bf16 (rows padded 16 B), 16 B zero block,
  // X [groups][TT] f32, then per wave its scales and biases
  const int xs = K + 8;
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);
  char* zero_blk = smem + (size_t)TT * xs * 2;
  float* Xl = reinterpret_cast<float*>(zero_blk + 16);
  char* sb_base =
      smem + (((size_t)TT * xs * 2 + 16 + (size_t)groups * TT * 4 + 15) & ~size_t(15));
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  const u32x4_t zq = {0u, 0u, 0u, 0u};
  // this wave's blocks: nb consecutive 16-channel blocks from ch0
  const int ch0 = ((tile * waves + wave) * nb) * 16 + n;
  const int64_t wrow0 = (int64_t)e * a.e_rows + ch0;
  // A operand row of this lane: (group m / TT, token m % TT), m = l % 16
  const int arow_g = n / TT, arow_t = n % TT;

  // ring of R = D + 1 slots: global super-step gs lives in slot gs % R; the
  // load for gs + D goes into the slot that gs - 1 freed, so nothing is
  // copied, and the ring runs on across block boundaries
  constexpr int R = D + 1;
  struct Ring {
    u32x4_t w[NM][NL];
  };
  const uint32_t* wb[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const QWeights& W = m == 0 ? a.w0 : a.w1;
    wb[m] = W.w + (wrow0 * groups + gq) * WPG + sq * (CPL * BITS / 32);
  }
  const int64_t blk_rows = (int64_t)16 * groups;  // row stride of a block
  auto load = [&](Ring& r, int gs) {
    const int bi = gs / ssk, ss = s0 + gs - bi * ssk;
    const int64_t go = bi * blk_rows + ss * GG;  // group offset
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const u32x4_t* wp = reinterpret_cast<const u32x4_t*>(wb[m] + go * WPG);
#pragma unroll
      for (int i = 0; i < NL; ++i) r.w[m][i] = wp[i];
    }
  };
  // Prologue.  Loads retire in issue order, so what the staging waits for
  // is issued first: the x rows (L2 hits, shared by every tile of the
  // item), then the wave's scales and biases, then the first D weight
  // super-steps.  Staging x waits for the x loads alone, the barrier
  // follows, and the weights' memory round trip overlaps both.  Every load
  // is issued by every thread (indices clamped, the extra copies dropped):
  // a load under a branch would make the compiler's wait counts cover the
  // loads issued after it as well.

  // x rows of the item's tokens, from the record's flat rows (fetched with
  // its header; a row_map lookup issues every load before the first use)
  int64_t xr[TT];
  {
    const int fl[8] = {fr0.x, fr0.y, fr0.z, fr0.w, fr1.x, fr1.y, fr1.z, fr1.w};
    int32_t rm[TT];
    if (!a.x_by_slot && a.row_map) {
#pragma unroll
      for (int t = 0; t < TT; ++t) rm[t] = a.row_map[t < nt ? fl[t] : fl[0]];
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      int64_t r = 0;
      if (t < nt)
        r = a.x_by_slot ? row0 + t : (a.row_map ? rm[t] : fl[t] / a.row_div);
      xr[t] = r;
    }
  }
  // thread k8 holds elements 8*k8..8*k8+7 of every token; the token sums X
  // of each 64-wide group come from the 8 threads sharing it
  const int per_row = K >> 3;
  // (only the item's nt rows are read: the padding rows of the MFMA form
  // stage zeros.  The branch is uniform, and these are the first loads of
  // the workgroup, so every later wait counts only loads issued after them)
  auto load_x = [&](int k8, u32x4_t (&v)[TT]) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      v[t] = zq;
      if (t < nt) v[t] = *reinterpret_cast<const u32x4_t*>(a.x + xr[t] * a.x_ld + 8 * k8);
    }
  };
  auto stage_x = [&](int k8, const u32x4_t (&v)[TT]) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const u32x4_t vt = t < nt ? v[t] : zq;
      float sx = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sx += __uint_as_float(vt[j] << 16) + __uint_as_float(vt[j] & 0xffff0000u);
      sx += __shfl_xor(sx, 1, 64);
      sx += __shfl_xor(sx, 2, 64);
      sx += __shfl_xor(sx, 4, 64);
      if ((k8 & 7) == 0) Xl[(k8 >> 3) * TT + t] = sx;
      u32x4_t w = vt;
      if constexpr (BITS == 4) w = perm4(w);
      *reinterpret_cast<u32x4_t*>(xl + (size_t)t * xs + 8 * k8) = w;
    }
  };
  const int k8 = ltid;
  const bool x_in = k8 < per_row;
  u32x4_t xv[TT];
  load_x(min(k8, per_row - 1), xv);
  MLXR_SCHED_BARRIER();  // issue order is retire order: x first

  // Scales and biases of this wave's blocks: 16 rows x groups bf16 per
  // block and array, contiguous in memory, copied to the wave's own LDS
  // region with 16-byte loads (the hot loop then reads its two values per
  // step from LDS): a per-step 2-byte load per lane would touch 16 cache
  // lines for 128 useful bytes.
  const int sbn = nb * 16 * groups;  // bf16 per array
  const int sbv = sbn >> 3;          // 16-byte vectors per array
  uint16_t* sbl = reinterpret_cast<uint16_t*>(sb_base) + (size_t)wave_id * NA * sbn;
  const uint16_t* sbsrc[NA];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const QWeights& W = m == 0 ? a.w0 : a.w1;
    sbsrc[2 * m] = W.scales + (wrow0 - n) * groups;
    sbsrc[2 * m + 1] = W.biases + (wrow0 - n) * groups;
  }
  u32x4_t sv[NA];
  const bool s_in = lane < sbv;
  const int sl = min(lane, sbv - 1);
#pragma unroll
  for (int i = 0; i < NA; ++i)
    sv[i] = *reinterpret_cast<const u32x4_t*>(sbsrc[i] + 8 * sl);
  MLXR_SCHED_BARRIER();

  Ring ring[R];
#pragma unroll
  for (int j = 0; j < D; ++j) load(ring[j], min(j, total - 1));
  MLXR_SCHED_BARRIER();

  if (x_in) stage_x(k8, xv);  // per_row is a multiple of 8: whole octets
  // the rest of x (input dims above 64 * 8 * waves)
  for (int c8 = k8 + lthreads; c8 < per_row; c8 += lthreads) {
    u32x4_t v[TT];
    load_x(c8, v);
    stage_x(c8, v);
  }
  if (ltid == 0) *reinterpret_cast<u32x4_t*>(zero_blk) = zq;
  __syncthreads();
  // the scales (issued before the weights) -> this wave's region; only
  // this wave reads it
  if (s_in) {
#pragma unroll
    for (int i = 0; i < NA; ++i)
      *reinterpret_cast<u32x4_t*>(sbl + i * sbn + 8 * lane) = sv[i];
  }
  for (int i = lane + 64; i < sbv; i += 64) {
#pragma unroll
    for (int j = 0; j < NA; ++j)
      *reinterpret_cast<u32x4_t*>(sbl + j * sbn + 8 * i) =
          *reinterpret_cast<const u32x4_t*>(sbsrc[j] + 8 * i);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // The loop issues the same loads every super-step (past the end they
  // repeat the last step, a cache hit) and holds no stores, so the
  // compiler can wait for exactly the oldest ring slot.  Steps past the
  // end multiply zeros.  With several blocks per wave each block's sums
  // move to done[block] when its last step is done (selects, so the
  // accumulators stay in registers).
  constexpr int ND = NB > 1 ? NB - 1 : 1;
  f32x4_t acc[NM], done[ND][NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    acc[m] = zero;
#pragma unroll
    for (int b = 0; b < ND; ++b) done[b][m] = zero;
  }
  const uint32_t one_v = 0x3F803F80u;
  // x operand source of this lane: its row's token chunk in its group's
  // codes, or the zero block off the diagonal / past the tokens
  const bool diag = arow_g == gq && arow_t < nt;
  const char* xsrc = smem + ((size_t)arow_t * xs + sq * CPL) * 2;
  for (int gs0 = 0; gs0 < total; gs0 += R) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int gs = gs0 + j;
      load(ring[(j + D) % R], min(gs + D, total - 1));
      const Ring& cur = ring[j];
      const bool live = gs < total;
      const int bi = gs / ssk, ls = gs - bi * ssk, ss = s0 + ls;
      const int g = ss * GG + gq;
      const bool on = diag && live;
      const char* xp = on ? xsrc + (size_t)(64 * g) * 2 : zero_blk;
      const int xstep = on ? 16 : 0;
      // all x fragments of the step are read before the first MFMA, so
      // the MFMA chain waits on LDS once per step, not once per MFMA
      bf16x8_t xa[NMF];
#pragma unroll
      for (int i = 0; i < NMF; ++i)
        xa[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(xp + xstep * i));
      // X of this lane's output rows: group (4q+r)/TT, tokens (4q+r)%TT
      const int og = ss * GG + (4 * q) / TT;
      f32x4_t X = *reinterpret_cast<const f32x4_t*>(Xl + og * TT + (4 * q) % TT);
      if (!live) X = zero;
      MLXR_SCHED_BARRIER();
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        f32x4_t P = zero;
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
          u32x4_t u;
          if constexpr (BITS == 4) {
            u = unpack4(cur.w[m][i / 4][i % 4], one_v);
          } else {
            const u32x4_t wv = cur.w[m][i / 2];
            u = (i & 1) ? unpack8(wv.z, wv.w) : unpack8(wv.x, wv.y);
          }
          P = mfma16x16x32(xa[i], as_bf16x8(u), P);
        }
        // scale/bias of this lane's output group og (channel n)
        const int si = ((live ? bi : 0) * 16 + n) * groups + min(og, groups - 1);
        const uint32_t sc_bits = sbl[(m * 2) * sbn + si];
        const uint32_t bi_bits = sbl[(m * 2 + 1) * sbn + si];
        float sc, cb;
        group_terms<BITS>(sc_bits, bi_bits, sc, cb);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[m][r] = __builtin_fmaf(sc, P[r], __builtin_fmaf(cb, X[r], acc[m][r]));
      }
      if constexpr (NB > 1) {
        const bool last = live && ls == ssk - 1 && bi < NB - 1;
#pragma unroll
        for (int b = 0; b < NB - 1; ++b) {
          const bool fin = last && bi == b;
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) done[b][m][r] = fin ? acc[m][r] : done[b][m][r];
        }
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[m][r] = last ? 0.0f : acc[m][r];
      }
    }
  }
  // Each token's GG group partials sit on lanes 16*(TT/4) apart: a
  // butterfly over those lanes sums them, and lanes q < TT/4 write tokens
  // 4q..4q+3 of channel n.  With K-slices the KS waves' sums of a block
  // meet in LDS (after the x region is no longer read) and the slice-0
  // wave adds them in slice order.
  f32x4_t* red = reinterpret_cast<f32x4_t*>(
      sb_base + (((size_t)(lthreads >> 6) * NA * nb * 16 * groups * 2 + 15) & ~size_t(15)));
  if constexpr (KS > 1) {
#pragma unroll
    for (int bi = 0; bi < NB; ++bi)
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        f32x4_t t = acc[m];
#pragma unroll
        for (int b = 0; b < NB - 1; ++b) t = bi == b ? done[b][m] : t;
        red[((wave_id * NB + bi) * NM + m) * 64 + lane] = t;
      }
    __syncthreads();
    if (kq != 0) return;
  }
#pragma unroll
  for (int bi = 0; bi < NB; ++bi) {
    f32x4_t tot[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      tot[m] = acc[m];
#pragma unroll
      for (int b = 0; b < NB - 1; ++b) tot[m] = bi == b ? done[b][m] : tot[m];
      if constexpr (KS > 1) {
#pragma unroll
        for (int k = 1; k < KS; ++k)
          tot[m] += red[(((wave_id + k) * NB + bi) * NM + m) * 64 + lane];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (TT == 4) tot[m][r] += __shfl_xor(tot[m][r], 16, 64);
        tot[m][r] += __shfl_xor(tot[m][r], 32, 64);
      }
    }
    if (q < TT / 4) {
      const int ch = ch0 + bi * 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 4 * q + r;
        if (t < nt) {
          const int slot = row0 + t;
          if constexpr (GATED) {
            a.out[(int64_t)slot * a.out_ld + ch] =
                gated_act_bf16(a.act, bf16_round(tot[0][r]), bf16_round(tot[1][r]));
          } else {
            const int64_t orow = a.out_by_flat ? rec[4 + t] : slot;
            if (yl)  // the single-token down + combine: rows stay in LDS
              yl[(orow + yrow_off) * 16 + n] = f32_to_bf16(tot[0][r]);
            else
              a.out[orow * a.out_ld + ch] = f32_to_bf16(tot[0][r]);
          }
        }
      }
    }
  }
}

// Tokens per pass follow the expert's row count: 4 (GG = 4) for experts
// with at most kStreamTT4Rows rows, else 8 (GG = 2).  LDS is sized
// for 8.
template <int BITS, bool GATED, int D, int D8, int NB, int KS>
__global__ __launch_bounds__(64 * MLXR_STREAM_WAVES) void qgemm_stream_kernel(
    QGemmArgs a, int tiles_n, QGemmArgs a2, int units1, int items1, int rows2) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  Unit u;
  if (!decode_unit(a, tiles_n, units1, items1, rows2, u)) return;
  const QGemmArgs& A = u.shared ? a2 : a;
  // The MFMA form follows the expert's row count (not the item's), so every
  // token of an expert is summed in the same order, wherever its item
  // boundaries fall.  Ring depths: D super-steps of the 4-token form in
  // flight, D8 of the 8-token form (half the bytes per super-step).
  if (u.wk.w <= kStreamTT4Rows)
    stream_body<BITS, GATED, 4, D, NB, KS>(A, u.rec, u.wk, u.fr0, u.fr1, u.tile, smem,
                                           threadIdx.x, blockDim.x, nullptr, 0);
  else
    stream_body<BITS, GATED, 8, D8, NB, KS>(A, u.rec, u.wk, u.fr0, u.fr1, u.tile, smem,
                                            threadIdx.x, blockDim.x, nullptr, 0);
}

// q ? b : c, field by field: every field a scalar select, so the chosen
// set stays in registers (selecting the whole struct by reference or value
// copies both argument sets to private memory)
__device__ __forceinline__ QWeights pick_w(bool q, const QWeights& b, const QWeights& c) {
  return QWeights{q ? b.w : c.w, q ? b.scales : c.scales, q ? b.biases : c.biases};
}
__device__ __forceinline__ QGemmArgs pick_args(bool q, const QGemmArgs& b, const QGemmArgs& c) {
  QGemmArgs r;
  r.x = q ? b.x : c.x;
  r.x_ld = q ? b.x_ld : c.x_ld;
  r.x_rows = q ? b.x_rows : c.x_rows;
  r.row_map = q ? b.row_map : c.row_map;
  r.row_div = q ? b.row_div : c.row_div;
  r.x_by_slot = q ? b.x_by_slot : c.x_by_slot;
  r.offsets = q ? b.offsets : c.offsets;
  r.active = q ? b.active : c.active;
  r.num_active = q ? b.num_active : c.num_active;
  r.work = q ? b.work : c.work;
  r.num_work = q ? b.num_work : c.num_work;
  r.tiles = q ? b.tiles : c.tiles;
  r.num_tiles = q ? b.num_tiles : c.num_tiles;
  r.sorted = q ? b.sorted : c.sorted;
  r.w0 = pick_w(q, b.w0, c.w0);
  r.w1 = pick_w(q, b.w1, c.w1);
  r.E = q ? b.E : c.E;
  r.N = q ? b.N : c.N;
  r.K = q ? b.K : c.K;
  r.bits = q ? b.bits : c.bits;
  r.e_rows = q ? b.e_rows : c.e_rows;
  r.act = q ? b.act : c.act;
  r.out = q ? b.out : c.out;
  r.out_ld = q ? b.out_ld : c.out_ld;
  r.out_by_flat = q ? b.out_by_flat : c.out_by_flat;
  r.gated = q ? b.gated : c.gated;
  return r;
}

// The down GEMM of one token and its combine (launch_qgemm_down_combine).
// Workgroup = 16 output channels (blockIdx.x); its waves come in groups of
// KS, one group per work item: the routed items (at most K: items 0..K-1
// of the dispatch) and, from K on, the folded shared expert's row.  Each
// group runs the streaming kernel's item work (KS K-slices, the MFMA form of
// the separate launch: 4 tokens, or 8 for an expert of more than
// kStreamTT4Rows rows when LONG) in its own LDS region and leaves its bf16
// row values in LDS (flat row k at row k, the shared row at K); after a
// barrier 16 threads sum them in k order with the combine's arithmetic.
// Without LONG the caller guarantees one row per item (K distinct
// experts).  Both MFMA forms pass the same barriers.
template <int BITS, int KS, bool BF16, typename WT, bool LONG>
__global__ __launch_bounds__(1024) void qgemm_down_combine_kernel(
    QGemmArgs a, QGemmArgs a2, int K, int nsub, int sub_lds, DownCombine c) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int L = 64 * KS;
  constexpr int D = BITS == 4 ? MLXR_STREAM_DEPTH4 : MLXR_STREAM_DEPTH8;
  constexpr int D8 = BITS == 4 ? MLXR_STREAM_DEPTH4_TT8 : MLXR_STREAM_DEPTH8_TT8;
  // (the group is uniform over a wave: said so, the choice of argument
  // set stays in scalar registers)
  const int sub = __builtin_amdgcn_readfirstlane((int)threadIdx.x / L);
  const int ltid = threadIdx.x - sub * L;
  const bool sh = sub >= K;
  uint16_t* yl = reinterpret_cast<uint16_t*>(smem + (size_t)nsub * sub_lds);
  // rows no item writes read as zeros (the groups' first barrier publishes
  // these stores)
  if ((int)threadIdx.x < nsub * 2)
    reinterpret_cast<u32x4_t*>(yl)[threadIdx.x] = u32x4_t{0u, 0u, 0u, 0u};
  const int32_t* rec = a.work + (int64_t)kWorkInts * (sh ? 0 : sub);
  int4 wk = *reinterpret_cast<const int4*>(rec);
  int4 fr0 = *reinterpret_cast<const int4*>(rec + 4);
  int4 fr1 = *reinterpret_cast<const int4*>(rec + 8);
  if (sh) {
    // the shared expert's one row: slot 0, no dispatch
    wk = make_int4(0, 0, 1, 1);
    fr0 = make_int4(0, 1, 2, 3);
    fr1 = make_int4(4, 5, 6, 7);
  } else if (sub >= *a.num_work) {
    wk = make_int4(0, 0, 0, 0);  // no such item: no rows (expert 0's loads)
  }
  const QGemmArgs A = pick_args(sh, a2, a);
  if (LONG && wk.w > kStreamTT4Rows)
    stream_body<BITS, false, 8, D8, 1, KS>(A, rec, wk, fr0, fr1, (int)blockIdx.x,
                                           smem + (size_t)sub * sub_lds, ltid, L, yl,
                                           sh ? K : 0);
  else
    stream_body<BITS, false, 4, D, 1, KS>(A, rec, wk, fr0, fr1, (int)blockIdx.x,
                                          smem + (size_t)sub * sub_lds, ltid, L, yl,
                                          sh ? K : 0);
  __syncthreads();
  if (threadIdx.x < 16) {
    const int n = threadIdx.x, ch = (int)blockIdx.x * 16 + n;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) {
      float w;
      if constexpr (sizeof(WT) == 2)
        w = bf16_to_f32(static_cast<const uint16_t*>(c.w)[k]);
      else
        w = static_cast<const float*>(c.w)[k];
      acc = combine_add<BF16>(acc, w, bf16_to_f32(yl[k * 16 + n]));
    }
    if (BF16) acc = bf16_round(acc);
    if (c.shared_logit) {
      const float sy = bf16_to_f32(nsub > K ? yl[K * 16 + n] : c.shared_y[ch]);
      acc = combine_shared<BF16>(acc, sy, combine_gate<BF16>(c.shared_logit[0]));
    }
    if (c.residual) acc = combine_residual<BF16>(acc, bf16_to_f32(c.residual[ch]));
    if (BF16)
      static_cast<uint16_t*>(c.out)[ch] = f32_to_bf16(acc);
    else
      static_cast<float*>(c.out)[ch] = acc;
  }
}

}  // namespace

namespace {

// Whether the streaming kernel runs a decode launch of `all_items` work
// items (routed and folded): quantised weights, enough (item, block) units,
// whole 64-channel tiles, groups in fours, 16-byte aligned scales and biases.
bool stream_eligible(const QGemmArgs& a, const QGemmArgs& b, int64_t all_items) {
  const auto a16 = [](const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
  };
  const bool sb16 = a16(a.w0.scales) && a16(a.w0.biases) &&
                    (!a.gated || (a16(a.w1.scales) && a16(a.w1.biases))) &&
                    a16(b.w0.scales) && a16(b.w0.biases) &&
                    (!b.gated || (a16(b.w1.scales) && a16(b.w1.biases)));
  const int groups = a.K / 64;
  return a.bits != 16 && all_items * (a.N / 16) >= kStreamMinBlocks && a.N % 64 == 0 &&
         groups % 4 == 0 && sb16;
}

// Launch shape of the streaming kernel: 16-channel blocks per wave (nb),
// K-slices (ks), channel tiles per item and the LDS of one workgroup.
struct StreamShape {
  int nb, ks, tiles_n;
  size_t lds;
};
StreamShape stream_shape(const QGemmArgs& a, int64_t all_items) {
  constexpr int kWaves = MLXR_STREAM_WAVES, kMaxTT = 8;
  const int groups = a.K / 64;
  // blocks per wave: about one workgroup per slot (two per CU), so x is
  // staged as few times as the GPU allows
  const int64_t per_tile = a.N / (16 * kWaves);
  int nb = 1;
  for (int c = a.gated ? MLXR_STREAM_GATED_NB : MLXR_STREAM_MAX_NB; c > 1; c >>= 1)
    if (per_tile % c == 0 &&
        all_items * (per_tile / c) >= kStreamSlots * (c >= 4 ? MLXR_STREAM_NB4_GRIDS : 1)) {
      nb = c;
      break;
    }
  // K-slices: a small grid (few items, one block per wave) splits each
  // block's input dim over ks waves of a workgroup, so more and shorter
  // waves run at once (the super-steps of either MFMA form divide
  // evenly), as long as the grid stays within one workgroup per slot
  // (two per CU, or one where the LDS allows only one)
  const size_t sb_lds = (size_t)kWaves * (a.gated ? 2 : 1) * 2 * nb * 16 * groups * 2;
  const size_t base_lds =
      (((size_t)kMaxTT * (a.K + 8) * 2 + 16 + (size_t)groups * kMaxTT * 4 + 15) &
       ~size_t(15)) + ((sb_lds + 15) & ~size_t(15));
  const size_t red_lds = (size_t)kWaves * (a.gated ? 2 : 1) * 64 * 16;
  const int64_t slots = (kStreamSlots / 2) * (base_lds + red_lds <= 80 * 1024 ? 2 : 1);
  int ks = 1;
  if (nb == 1)
    for (int c = std::min(4, kWaves); c > 1; c >>= 1)
      if ((groups / 4) % c == 0 &&
          all_items * (a.N / (16 * (kWaves / c))) <= std::min<int64_t>(slots, MLXR_STREAM_KS_GRID)) {
        ks = c;
        break;
      }
  const int tiles_n = (int)(a.N / (16 * (kWaves / ks)) / nb);
  return StreamShape{nb, ks, tiles_n, base_lds + (ks > 1 ? red_lds : 0)};
}

}  // namespace

hipError_t launch_qgemm(const QGemmArgs& a, int64_t total_rows,
                        int64_t max_items, bool prefill, hipStream_t s,
                        const char* profile, const QGemmArgs* shared,
                        int64_t shared_rows) {
  if (!profile) profile = a.gated ? "qgemm_gated" : "qgemm_down";
  // a folded second problem: the same projection shape and format, its
  // items (or M-tiles) beside the routed ones in the same grid
  const int64_t items2 = shared ? (shared_rows + kWorkRows - 1) / kWorkRows : 0;
  if (shared && (shared->N != a.N || shared->K != a.K ||
                 shared->bits != a.bits || shared->gated != a.gated))
    return hipErrorInvalidValue;
  if (max_items + items2 <= 0) return hipSuccess;
  const QGemmArgs& b = shared ? *shared : a;
  // the M-tiled kernel reads x through a buffer of x's own rows (gathered
  // rows may lie anywhere in it: gather_mm / gather_qmm with lhs indices)
  const int64_t x_rows = a.x_rows > 0 ? a.x_rows : total_rows;
  if (prefill && prefill_supported(a, x_rows) &&
      (!shared || prefill_supported(*shared, shared_rows))) {
    const int tile_rows = prefill_tile_rows(total_rows, a.E, a.bits);
    return launch_qgemm_prefill(a, x_rows, tile_rows,
                                dispatch_max_tiles(total_rows, a.E, tile_rows), s, profile,
                                shared, shared_rows);
  }
  const int groups = a.K / 64;
  // Many (expert, block) items: the streaming kernel (one block per wave,
  // x in LDS, a ring of weight loads).  Few: the split-K kernel below, which
  // spreads each block over up to 16 waves.
  const int64_t all_items = max_items + items2;
  // (dense bf16 weights, bits 16, take the split-K kernel below)
  if (stream_eligible(a, b, all_items)) {
    constexpr int kWaves = MLXR_STREAM_WAVES;
    const StreamShape sh = stream_shape(a, all_items);
    const int nb = sh.nb, ks = sh.ks, tiles_n = sh.tiles_n;
    const size_t lds = sh.lds;
    const int items1 = (int)max_items;
    const int units1 = (int)(max_items * tiles_n);
    const dim3 grid((unsigned)(units1 + items2 * tiles_n));
    const int rows2 = (int)shared_rows;
    ProfileScope prof(profile, s);
#define MLXR_QS(B, G, D, D8, NB)                                          \
  do {                                                                    \
    if (ks == 4)                                                          \
      qgemm_stream_kernel<B, G, D, D8, 1, 4>                              \
          <<<grid, 64 * kWaves, lds, s>>>(a, tiles_n, b, units1, items1, rows2);  \
    else if (ks == 2)                                                     \
      qgemm_stream_kernel<B, G, D, D8, 1, 2>                              \
          <<<grid, 64 * kWaves, lds, s>>>(a, tiles_n, b, units1, items1, rows2);  \
    else                                                                  \
      qgemm_stream_kernel<B, G, D, D8, NB, 1>                             \
          <<<grid, 64 * kWaves, lds, s>>>(a, tiles_n, b, units1, items1, rows2);  \
  } while (0)
    if (a.bits == 4) {
#if MLXR_STREAM_GATED_NB > 1
      if (a.gated && nb == 2)
        MLXR_QS(4, true, MLXR_STREAM_DEPTH4G, MLXR_STREAM_DEPTH4G_TT8, 2);
      else
#endif
      if (a.gated)
        MLXR_QS(4, true, MLXR_STREAM_DEPTH4G, MLXR_STREAM_DEPTH4G_TT8, 1);
#if MLXR_STREAM_MAX_NB >= 4
      else if (nb == 4)
        MLXR_QS(4, false, MLXR_STREAM_DEPTH4, MLXR_STREAM_DEPTH4_TT8, 4);
#endif
      else if (nb == 2)
        MLXR_QS(4, false, MLXR_STREAM_DEPTH4, MLXR_STREAM_DEPTH4_TT8, 2);
      else
        MLXR_QS(4, false, MLXR_STREAM_DEPTH4, MLXR_STREAM_DEPTH4_TT8, 1);
    } else {
#if MLXR_STREAM_GATED_NB > 1
      if (a.gated && nb == 2)
        MLXR_QS(8, true, MLXR_STREAM_DEPTH8G, MLXR_STREAM_DEPTH8G_TT8, 2);
      else
#endif
      if (a.gated)
        MLXR_QS(8, true, MLXR_STREAM_DEPTH8G, MLXR_STREAM_DEPTH8G_TT8, 1);
#if MLXR_STREAM_MAX_NB >= 4
      else if (nb == 4)
        MLXR_QS(8, false, MLXR_STREAM_DEPTH8, MLXR_STREAM_DEPTH8_TT8, 4);
#endif
      else if (nb == 2)
        MLXR_QS(8, false, MLXR_STREAM_DEPTH8, MLXR_STREAM_DEPTH8_TT8, 2);
      else
        MLXR_QS(8, false, MLXR_STREAM_DEPTH8, MLXR_STREAM_DEPTH8_TT8, 1);
    }
#undef MLXR_QS
    return hipGetLastError();
  }
  // waves along the input dim: two groups each per pass (one step at 4-bit,
  // two at 8-bit), up to 16 waves; more groups take several passes
  constexpr int kGroupsPerWave = MLXR_SPLITK_GROUPS;
  const int kw = std::min(16, (groups + kGroupsPerWave - 1) / kGroupsPerWave);
  // channel blocks per workgroup: as many as keep >= ~1024 workgroups, with
  // the partial sums of the blocks within 64 KB of LDS
  const int nm = a.gated ? 2 : 1;
  const int nblk = a.N / 16;
  int cb = 1;
  // (the gated kernel keeps one block: two would spill under the 128-VGPR
  // budget of 16-wave workgroups)
  for (int c = 4; c > 1 && !a.gated; c >>= 1)
    if (nblk % c == 0 && all_items * (nblk / c) >= 1024 &&
        kw * c * nm <= 64) {
      cb = c;
      break;
    }
  const int tiles_n = nblk / cb;
  const size_t lds = (size_t)kw * cb * nm * 64 * sizeof(f32x4_t);
  const int items1 = (int)max_items;
  const int units1 = (int)(max_items * tiles_n);
  const int rows2 = (int)shared_rows;
  const dim3 grid((unsigned)(units1 + items2 * tiles_n));
  const dim3 block((unsigned)(64 * kw));
  ProfileScope prof(profile, s);
#define MLXR_QG(B, G, SPW)                                                  \
  do {                                                                      \
    if (cb == 4)                                                            \
      qgemm_decode_kernel<B, G, SPW, 4>                                     \
          <<<grid, block, lds, s>>>(a, tiles_n, b, units1, items1, rows2);                            \
    else if (cb == 2)                                                       \
      qgemm_decode_kernel<B, G, SPW, 2>                                     \
          <<<grid, block, lds, s>>>(a, tiles_n, b, units1, items1, rows2);                            \
    else                                                                    \
      qgemm_decode_kernel<B, G, SPW, 1>                                     \
          <<<grid, block, lds, s>>>(a, tiles_n, b, units1, items1, rows2);                            \
  } while (0)
  if (a.bits == 16) {
    if (a.gated)
      qgemm_decode_kernel<16, true, 2, 1><<<grid, block, lds, s>>>(a, tiles_n, b, units1, items1, rows2);
    else
      MLXR_QG(16, false, 2);
  } else if (a.bits == 4) {
    if (a.gated)
      qgemm_decode_kernel<4, true, 1, 1><<<grid, block, lds, s>>>(a, tiles_n, b, units1, items1, rows2);
    else
      MLXR_QG(4, false, 1);
  } else {
    if (a.gated)
      qgemm_decode_kernel<8, true, 2, 1><<<grid, block, lds, s>>>(a, tiles_n, b, units1, items1, rows2);
    else
      MLXR_QG(8, false, 2);
  }
#undef MLXR_QG
  return hipGetLastError();
}

hipError_t launch_qgemm_down_combine(const QGemmArgs& a, int64_t K, int64_t max_items,
                                     const QGemmArgs* shared, const DownCombine& c,
                                     hipStream_t s, bool* done) {
  *done = false;
  const QGemmArgs& b = shared ? *shared : a;
  if (a.gated || (a.bits != 4 && a.bits != 8) || K < 1 ||
      (shared && (shared->N != a.N || shared->K != a.K || shared->bits != a.bits ||
                  shared->gated)) ||
      (c.w_bf16 && !c.bf16) || (shared && !c.shared_logit))
    return hipSuccess;
  const int64_t items2 = shared ? 1 : 0;
  const int64_t all_items = max_items + items2;
  // (the group of row k reads work record k: the list holds K records)
  if (max_items < K || !stream_eligible(a, b, all_items)) return hipSuccess;
  // the separate down launch's K-slices, so every y value is the same
  const int ks = stream_shape(a, all_items).ks;
  const int nsub = (int)K + (int)items2;
  if (ks > 2 || nsub * ks > 16) return hipSuccess;
  const int groups = a.K / 64;
  // an expert can take more than kStreamTT4Rows of the K rows only when the
  // ids may repeat: then its item runs in the 8-token form, LDS sized for it
  const bool long_items = !c.distinct && K > kStreamTT4Rows;
  const size_t tt = long_items ? 8 : 4;
  const size_t sub_lds =
      ((tt * (a.K + 8) * 2 + 16 + (size_t)groups * tt * 4 + 15) & ~size_t(15)) +
      (((size_t)ks * 2 * 16 * groups * 2 + 15) & ~size_t(15)) +
      (ks > 1 ? (size_t)ks * 64 * 16 : 0);
  const size_t lds = (size_t)nsub * sub_lds + (size_t)nsub * 32;
  if (lds > 160 * 1024) return hipSuccess;
  const dim3 grid((unsigned)(a.N / 16)), block((unsigned)(64 * ks * nsub));
  ProfileScope prof("qgemm_down", s);
#define MLXR_DC2(B, KS_, LG)                                                              \
  do {                                                                                    \
    if (c.w_bf16)                                                                         \
      qgemm_down_combine_kernel<B, KS_, true, uint16_t, LG>                               \
          <<<grid, block, lds, s>>>(a, b, (int)K, nsub, (int)sub_lds, c);                 \
    else if (c.bf16)                                                                      \
      qgemm_down_combine_kernel<B, KS_, true, float, LG>                                  \
          <<<grid, block, lds, s>>>(a, b, (int)K, nsub, (int)sub_lds, c);                 \
    else                                                                                  \
      qgemm_down_combine_kernel<B, KS_, false, float, LG>                                 \
          <<<grid, block, lds, s>>>(a, b, (int)K, nsub, (int)sub_lds, c);                 \
  } while (0)
#define MLXR_DC(B, KS_)              \
  do {                               \
    if (long_items)                  \
      MLXR_DC2(B, KS_, true);        \
    else                             \
      MLXR_DC2(B, KS_, false);       \
  } while (0)
  if (a.bits == 4) {
    if (ks == 2)
      MLXR_DC(4, 2);
    else
      MLXR_DC(4, 1);
  } else {
    if (ks == 2)
      MLXR_DC(8, 2);
    else
      MLXR_DC(8, 1);
  }
#undef MLXR_DC
#undef MLXR_DC2
  *done = true;
  return hipGetLastError();
}

}  // namespace mlxr_moe
