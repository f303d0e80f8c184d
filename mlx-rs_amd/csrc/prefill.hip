// Grouped quantised expert GEMM for many rows per expert (prefill): an
// LDS-tiled bf16 MFMA GEMM that dequantises each weight tile once per
// workgroup.  The same kernel runs dense bf16 expert weights (gather_mm,
// bits = 16: the weight tile is staged as it is).
//
// Same operation as the decode kernels (gather_qmm with transpose = true,
// crates/mlxr/src/ops/quantization.rs:171-221, as called by
// QuantizedSwitchLinear::apply, crates/mlxr-lm/src/nn/switch.rs:148-167):
//   out[p, n] = sum_k x[row(p), k] * bf16(code[e, n, k] * scale + bias)
// over the sorted slots p of expert e.  Here the rows of an expert come in
// M-tiles (the dispatch lists them), and the work is compute-bound, so the
// weights are dequantised -- exactly the oracle's
// bf16(fmaf(code, scale, bias)) -- into LDS, where every wave of the
// workgroup reuses them.
//
// Workgroup: kWM x kWN waves (2 x 4, or 2 x 2 in the narrow forms); tile
// kBM rows x kBN = 64 kWN columns (the gated kernel's columns are gate
// channels then the same up channels, so each wave holds matching gate and
// up sums for the SwiGLU epilogue).  Tile heights 256, 128 and 64 rows
// (prefill_tile.inc is built once per shape): each wave 128 x 64, 64 x 64
// or 32 x 64 outputs as blocks of v_mfma_f32_32x32x16_bf16 (K = 16 per
// instruction, four per group).  A tall tile spreads the
// dequantisation (the VALU cost, about three instructions per weight) over
// more rows; waves whose rows lie past the expert's last row skip their
// MFMAs.  Global loads are raw buffer loads with the K step in the scalar
// offset: no per-step address arithmetic.
// K advances one quantisation group (64) per step.  Register buffers hold
// the loads of the next groups in flight, and LDS stages hold dequantised
// tiles: while the waves multiply stage s, the group loaded a step earlier
// is dequantised into the next stage, interleaved with the MFMAs.  One
// barrier per step.  When K has 16 or more groups, each tile's scales and
// biases are copied to LDS once (coalesced) instead of loaded every step:
// a step's per-column scale loads put a different cache line on every lane.
//
// LDS rows are 64 bf16 (128 bytes) with the eight 16-byte chunks of row r
// stored at chunk ^ ((r >> 1) & 7), which keeps the 16-byte operand reads of
// a wave on distinct banks.  The epilogue goes through LDS so that every
// output store is 16 bytes.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {
namespace {

// raw buffer resource word 3 (gfx9 family)
constexpr int kBufFlags = 0x00020000;
// XCDs of an MI355X (the workgroup numbering below assumes this many; any
// other count only changes which workgroups share an L2)
constexpr unsigned kXcds = 8;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
// f rounded to bf16 (the hardware conversion: round to nearest even)
__device__ __forceinline__ float bf16_hw(float f) { return (float)(__bf16)f; }
// silu(g) * u with the reference's bf16 rounding points
// (crates/mlxr-lm/src/activations.rs:187-200), the sigmoid from the
// hardware exp2 and reciprocal (about 1 ulp each in f32; the bf16 rounding
// that follows hides that except next to a rounding boundary)
__device__ __forceinline__ uint16_t swiglu_fast(float g_acc, float u_acc) {
  const float g = bf16_hw(g_acc), u = bf16_hw(u_acc);
  const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
  const float sg = bf16_hw(__builtin_amdgcn_rcpf(1.0f + e));
  const float h = bf16_hw(g * sg);
  return __builtin_bit_cast(uint16_t, (__bf16)(h * u));
}
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// a and b rounded to bf16 by one conversion (round to nearest even), as f32
__device__ __forceinline__ f32x2_t bf16_hw2(float a, float b) {
  const uint32_t p =
      __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
  return f32x2_t{__uint_as_float(p << 16), __uint_as_float(p & 0xffff0000u)};
}
// swiglu_fast of two elements, each rounding done for both at once; the
// results packed, the first in the low half (the same values as two calls)
__device__ __forceinline__ uint32_t swiglu_fast2(float g0_acc, float u0_acc, float g1_acc,
                                                 float u1_acc) {
  const f32x2_t g = bf16_hw2(g0_acc, g1_acc), u = bf16_hw2(u0_acc, u1_acc);
  const float e0 = __builtin_amdgcn_exp2f(-g.x * 1.4426950408889634f);
  const float e1 = __builtin_amdgcn_exp2f(-g.y * 1.4426950408889634f);
  const f32x2_t sg = bf16_hw2(__builtin_amdgcn_rcpf(1.0f + e0), __builtin_amdgcn_rcpf(1.0f + e1));
  const f32x2_t h = bf16_hw2(g.x * sg.x, g.y * sg.y);
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector(f32x2_t{h.x * u.x, h.y * u.y}, bf16x2_t));
}
// a compile-time flag as a type (for generic lambdas)
template <bool B>
struct PfFlag {
  static constexpr bool value = B;
};
// q = n / d for 0 <= n < 2^31, 1 <= d <= 2^16: a float estimate and one
// correction step either way
__device__ __forceinline__ int div_small(int n, int d, float rd) {
  int q = (int)((float)n * rd);
  q -= (q * d > n) ? 1 : 0;
  q += ((q + 1) * d <= n) ? 1 : 0;
  return q;
}

// x & m, opaque to the optimiser so that the byte extracts below stay
// v_cvt_f32_ubyte{0..3} (it would otherwise fold the masks into bit-field
// extracts plus a conversion)
__device__ __forceinline__ uint32_t and_opaque(uint32_t x, uint32_t m) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(x), "s"(m));
  return r;
}
// 8 four-bit codes of one word (little end first) -> 4 words of bf16 pairs,
// each bf16(fmaf(code, s, b)); the even codes sit in the low nibbles.
__device__ __forceinline__ void dequant4(uint32_t w, float s, float b,
                                         uint32_t* o) {
  const uint32_t lo = and_opaque(w, 0x0F0F0F0Fu);
  const uint32_t hi = and_opaque(w >> 4, 0x0F0F0F0Fu);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = pack_bf16(__builtin_fmaf((float)((lo >> (8 * j)) & 255u), s, b),
                     __builtin_fmaf((float)((hi >> (8 * j)) & 255u), s, b));
}
// 4 eight-bit codes -> 2 words of pairs
__device__ __forceinline__ void dequant8(uint32_t w, float s, float b,
                                         uint32_t* o) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
    o[j] = pack_bf16(__builtin_fmaf((float)((w >> (16 * j)) & 255u), s, b),
                     __builtin_fmaf((float)((w >> (16 * j + 8)) & 255u), s, b));
}

__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

// The tile shapes.  Tall tiles (256 x 256, waves of 128 x 64) dequantise
// each weight group for more rows and read fewer LDS bytes per MFMA; shorter
// ones (128 x 256, waves of 64 x 64; 64 x 256, waves of 32 x 64) waste less
// when the experts hold few rows.  prefill_tile_rows picks one per call, and the dispatch cuts the
// M-tiles to match.
namespace tile256 {
#define MLXR_PF_TILE_ROWS 256
#define MLXR_PF_MBLOCKS 4
#define MLXR_PF_WAVES_N 4
#define MLXR_PF_REGBUF 2
#include "prefill_tile.inc"
#undef MLXR_PF_TILE_ROWS
#undef MLXR_PF_MBLOCKS
#undef MLXR_PF_WAVES_N
#undef MLXR_PF_REGBUF
}  // namespace tile256
// register buffers of the 128-row tile (2 or 3 groups of loads in flight)
#ifndef MLXR_PF128_REGBUF
#define MLXR_PF128_REGBUF 2
#endif
namespace tile128 {
#define MLXR_PF_TILE_ROWS 128
#define MLXR_PF_MBLOCKS 2
#define MLXR_PF_WAVES_N 4
#define MLXR_PF_REGBUF MLXR_PF128_REGBUF
// two stages (96 KB) leave room for the scales and biases of K up to 4096
#define MLXR_PF_STAGES 2
#include "prefill_tile.inc"
#undef MLXR_PF_STAGES
#undef MLXR_PF_TILE_ROWS
#undef MLXR_PF_MBLOCKS
#undef MLXR_PF_WAVES_N
#undef MLXR_PF_REGBUF
}  // namespace tile128
// 64 x 256 tiles (waves of 32 x 64) for experts averaging under
// MLXR_PREFILL_SHORT_ROWS rows: a 128-row tile there multiplies mostly
// padding rows (2048 tokens, top 10 of 512 experts: 40 rows an expert).
// 8-bit weights keep the 128-row tile: dequantising a wider group for half
// the rows measured slower than the padding it saves.
namespace tile64 {
#define MLXR_PF_TILE_ROWS 64
#define MLXR_PF_MBLOCKS 1
#define MLXR_PF_WAVES_N 4
#define MLXR_PF_REGBUF 2
#define MLXR_PF_STAGES 2
#include "prefill_tile.inc"
#undef MLXR_PF_STAGES
#undef MLXR_PF_TILE_ROWS
#undef MLXR_PF_MBLOCKS
#undef MLXR_PF_WAVES_N
#undef MLXR_PF_REGBUF
}  // namespace tile64
// Narrow forms: 128 columns, 4 waves of 64 x 64 (128 rows) or 32 x 64 (64
// rows), two stages: 80 and 64 KB of LDS with the scales, so two
// workgroups share a CU and one's barrier waits and staging overlap the
// other's MFMAs (the 8-wave tiles fill a CU alone).  Measured against the
// 256-column tiles: c7 T=2048 gate/up 234 to 205 µs, c6 T=2048 176 to 164
// (down 109 to 103), c3 T=2048 191 to 184; 64 rows, gate/up: c4 T=2048
// 291 to 258, c3 T=512 126 to 118.  Not for 8-bit weights (c5 T=512
// gate/up 463 to 670) or the 64-row down GEMMs (c4 T=2048 135 to 141).
namespace tile128n {
#define MLXR_PF_TILE_ROWS 128
#define MLXR_PF_MBLOCKS 2
#define MLXR_PF_WAVES_N 2
#define MLXR_PF_REGBUF 2
#define MLXR_PF_STAGES 2
#include "prefill_tile.inc"
#undef MLXR_PF_STAGES
#undef MLXR_PF_TILE_ROWS
#undef MLXR_PF_MBLOCKS
#undef MLXR_PF_WAVES_N
#undef MLXR_PF_REGBUF
}  // namespace tile128n
namespace tile64n {
#define MLXR_PF_TILE_ROWS 64
#define MLXR_PF_MBLOCKS 1
#define MLXR_PF_WAVES_N 2
#define MLXR_PF_REGBUF 2
#define MLXR_PF_STAGES 2
#include "prefill_tile.inc"
#undef MLXR_PF_STAGES
#undef MLXR_PF_TILE_ROWS
#undef MLXR_PF_MBLOCKS
#undef MLXR_PF_WAVES_N
#undef MLXR_PF_REGBUF
}  // namespace tile64n

}  // namespace

// 8-bit weights take the 64-row tiles too (1) or always 128 (0)
#ifndef MLXR_PF8_SHORT
#define MLXR_PF8_SHORT 0
#endif
// the 64-row gate/up of 8-bit weights in the narrow form (1) or the wide one (0)
#ifndef MLXR_PF8_NARROW64
#define MLXR_PF8_NARROW64 1
#endif

int prefill_tile_rows(int64_t rows, int64_t experts, int bits) {
  const int64_t e = experts > 0 ? experts : 1;
  if (rows >= (int64_t)MLXR_PREFILL_TALL_ROWS * e) return tile256::kBM;
  if (rows >= (int64_t)MLXR_PREFILL_SHORT_ROWS * e || (bits == 8 && !MLXR_PF8_SHORT))
    return tile128::kBM;
  return tile64::kBM;
}

bool prefill_supported(const QGemmArgs& a, int64_t x_rows) {
  // buffer offsets are 32-bit: x, and one expert's weights, under 2 GB
  // outputs leave as 16-byte runs of a row
  const bool out16 = (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 && a.out_ld % 8 == 0;
  return (a.bits == 4 || a.bits == 8 || a.bits == 16) && a.K % 64 == 0 && a.N % 64 == 0 &&
         a.sorted != nullptr && out16 && a.row_div >= 1 && a.row_div <= 65536 &&
         x_rows * a.x_ld * 2 < ((int64_t)1 << 31) &&
         (int64_t)a.N * a.K * a.bits / 8 < ((int64_t)1 << 31);
}

hipError_t launch_qgemm_prefill(const QGemmArgs& a, int64_t x_rows,
                                int tile_rows, int64_t max_tiles,
                                hipStream_t s, const char* profile,
                                const QGemmArgs* shared, int64_t shared_rows) {
  if (tile_rows == tile256::kBM)
    return tile256::launch(a, x_rows, max_tiles, s, profile, shared, shared_rows);
  // (the dispatch's M-tiles fix the height; the width is the launch's own)
  if (tile_rows == tile128::kBM && a.bits != 8)
    return tile128n::launch(a, x_rows, max_tiles, s, profile, shared, shared_rows);
  if (tile_rows == tile64::kBM && a.gated && (a.bits != 8 || MLXR_PF8_NARROW64))
    return tile64n::launch(a, x_rows, max_tiles, s, profile, shared, shared_rows);
  if (tile_rows == tile128::kBM)
    return tile128::launch(a, x_rows, max_tiles, s, profile, shared, shared_rows);
  if (tile_rows == tile64::kBM)
    return tile64::launch(a, x_rows, max_tiles, s, profile, shared, shared_rows);
  return hipErrorInvalidValue;
}

}  // namespace mlxr_moe
