// Grouped quantised expert GEMM for many rows per expert (prefill): an
// LDS-tiled bf16 MFMA GEMM that dequantises each weight tile once per
// workgroup.
//
// Same operation as the decode kernels (gather_qmm with transpose = true,
// crates/mlxr/src/ops/quantization.rs:171-221, as called by
// QuantizedSwitchLinear::apply, crates/mlxr-lm/src/nn/switch.rs:148-167):
//   out[p, n] = sum_k x[row(p), k] * bf16(code[e, n, k] * scale + bias)
// over the sorted slots p of expert e.  Here the rows of an expert come in
// M-tiles of kPrefillTileRows (the dispatch lists them), and the work is
// compute-bound, so the weights are dequantised -- exactly the oracle's
// bf16(fmaf(code, scale, bias)) -- into LDS, where every wave of the
// workgroup reuses them.
//
// Workgroup: kWM x kWN waves (4 x 2); tile kBM = 256 rows x kBN = 128
// columns (the gated kernel's columns are 64 gate channels then the same 64
// up channels, so each wave holds matching gate and up sums for the SwiGLU
// epilogue).  A tall tile spreads the dequantisation (the VALU cost, about
// three instructions per weight) over many rows; waves whose rows lie past
// the expert's last row skip their MFMAs.  Global loads are raw buffer loads
// with the K step in the scalar offset: no per-step address arithmetic.
// K advances one quantisation group (64) per step.  Three register buffers
// hold the loads of the next groups in flight, and three LDS stages hold
// dequantised tiles: while the waves multiply stage s, the group loaded two
// steps ago is dequantised into the next stage, interleaved with the MFMAs.
// One barrier per step.
//
// Each wave owns 64 x 64 outputs as 2 x 2 blocks of v_mfma_f32_32x32x16_bf16
// (K = 16 per instruction, four per group).  LDS rows are 64 bf16 (128
// bytes) with the eight 16-byte chunks of row r stored at chunk ^ ((r >> 1)
// & 7), which keeps the 16-byte operand reads of a wave on distinct banks.
// The epilogue goes through LDS so that every output store is 16 bytes.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {
namespace {

constexpr int kWM = kPrefillTileRows / 64, kWN = kPrefillWavesN;
constexpr int kNT = 64 * kWM * kWN;     // threads
constexpr int kBM = 64 * kWM;           // rows per tile
constexpr int kBN = 64 * kWN;           // B columns per tile
constexpr int kACH = kBM * 8 / kNT;     // 16-byte x chunks per thread
constexpr int kPARTS = kNT / kBN;       // threads per B column per group
constexpr int kCODES = 64 / kPARTS;     // codes per thread per group
constexpr int kCPT = kCODES / 8;        // 16-byte bf16 runs per thread
static_assert(kBM * 8 % kNT == 0 && kNT % kBN == 0 &&
                  (kCODES == 16 || kCODES == 32), "tile split");
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

// LDS: three stages, each an x tile [kBM rows][128 B] and a dequantised
// weight tile [kBN rows][128 B].  Neither is padded: the eight 16-byte
// chunks of row r sit at positions chunk ^ ((r >> 1) & 7), which keeps the
// MFMA operand reads of 16 consecutive rows on distinct banks.
// three stages when one workgroup holds the CU, two when two share it
constexpr int kStages = kBM == 256 ? 3 : 2;
constexpr int kAStage = kBM * 128;  // bytes
constexpr int kBStage = kBN * 128;  // bytes
constexpr int kStage = kAStage + kBStage;
constexpr int kPrefillLds = kStages * kStage;

__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

// Everything the K-loop needs, in registers.
template <int BITS>
struct PrefillCtx {
  __amdgpu_buffer_rsrc_t xr, wr, sr, br;  // x, weights, scales, biases
  uint32_t aoff[kACH];                     // x chunk offsets (bytes)
  int awr[kACH];                           // where they go in an x stage
  uint32_t woff, soff;                     // code chunk / scale offsets
  int bwr[kCPT];                           // where the dequantised runs go
  char* lds;
  int aread[2], aswz[2];                   // A rows (bytes) and swizzles
  int bread[2], bswz[2];                   // B rows (bytes) and swizzles
  int hi, groups;
};

// One group's global loads, held in registers until they are staged.
template <int BITS>
struct PrefillRegs {
  static constexpr int kWords = kCODES * BITS / 32;  // code words per thread
  typedef uint32_t u32w_t __attribute__((ext_vector_type(kWords < 4 ? kWords : 4)));
  u32x4_t a[kACH];
  u32w_t b[kWords < 4 ? 1 : kWords / 4];
  uint32_t s, c;
};

template <int BITS>
__device__ __forceinline__ void prefill_load(const PrefillCtx<BITS>& c,
                                             PrefillRegs<BITS>& R, int g_in) {
  // the group index is uniform; said so, the step offsets stay scalar
  const int g = __builtin_amdgcn_readfirstlane(g_in);
#pragma unroll
  for (int j = 0; j < kACH; ++j)
    R.a[j] = __builtin_amdgcn_raw_buffer_load_b128(c.xr, c.aoff[j], 128 * g, 0);
  constexpr int kW = PrefillRegs<BITS>::kWords;
  if constexpr (kW == 2) {
    R.b[0] = __builtin_amdgcn_raw_buffer_load_b64(c.wr, c.woff, 32 * g, 0);
  } else {
#pragma unroll
    for (int i = 0; i < kW / 4; ++i)
      R.b[i] = __builtin_amdgcn_raw_buffer_load_b128(c.wr, c.woff + 16 * i,
                                                     8 * BITS * g, 0);
  }
  R.s = __builtin_amdgcn_raw_buffer_load_b16(c.sr, c.soff, 2 * g, 0);
  R.c = __builtin_amdgcn_raw_buffer_load_b16(c.br, c.soff, 2 * g, 0);
}

// x chunks as they are, codes dequantised to bf16 pairs, into stage st.
template <int BITS, int ST>
__device__ __forceinline__ void prefill_store(const PrefillCtx<BITS>& c,
                                              const PrefillRegs<BITS>& R) {
  char* A = c.lds + ST * kStage;
  char* B = A + kAStage;
#pragma unroll
  for (int j = 0; j < kACH; ++j)
    *reinterpret_cast<u32x4_t*>(A + c.awr[j]) = R.a[j];
  const float s = __uint_as_float(R.s << 16), b = __uint_as_float(R.c << 16);
  constexpr int kW = PrefillRegs<BITS>::kWords;
  uint32_t w[kW];
#pragma unroll
  for (int i = 0; i < kW; ++i) w[i] = R.b[i / 4][i % 4];
  uint32_t o[kCODES / 2];
#pragma unroll
  for (int i = 0; i < kW; ++i) {
    if constexpr (BITS == 4)
      dequant4(w[i], s, b, o + 4 * i);
    else
      dequant8(w[i], s, b, o + 2 * i);
  }
#pragma unroll
  for (int i = 0; i < kCPT; ++i)
    *reinterpret_cast<u32x4_t*>(B + c.bwr[i]) =
        u32x4_t{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
}

// The multiplies of one group from stage ST, with the staging of the next
// group (register buffer R, into stage SS) spread between them: a quarter
// of the x copies and of the dequantisation after each 16-wide K chunk's
// MFMAs, so the VALU work runs while the matrix core is busy.  Per chunk:
// the 2 B fragments and NMB A fragments, then their NMB x 2 MFMAs.
template <int BITS, int NMB, int ST, int SS>
__device__ __forceinline__ void prefill_mma_store(const PrefillCtx<BITS>& c,
                                                  const PrefillRegs<BITS>& R,
                                                  f32x16_t (&acc)[2][2]) {
  const char* A = c.lds + ST * kStage;
  const char* B = A + kAStage;
  char* As = c.lds + SS * kStage;
  char* Bs = As + kAStage;
  constexpr int kW = PrefillRegs<BITS>::kWords;
  constexpr int kWPK = (kW + 3) / 4;   // code words dequantised per chunk
  constexpr int kOPW = BITS == 4 ? 4 : 2;  // bf16 pair words per code word
  const float s = __uint_as_float(R.s << 16), b = __uint_as_float(R.c << 16);
  uint32_t o[kCODES / 2];
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    const int ch = 2 * kc + c.hi;  // 16-byte chunk of the 64-wide group
    bf16x8_t af[2], bf[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
      bf[nb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(
          B + c.bread[nb] + 16 * (ch ^ c.bswz[nb])));
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
      af[mb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(
          A + c.aread[mb] + 16 * (ch ^ c.aswz[mb])));
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        acc[mb][nb] = mfma32x32x16(af[mb], bf[nb], acc[mb][nb]);
    // staging, part kc
#pragma unroll
    for (int j = kc; j < kACH; j += 4)
      *reinterpret_cast<u32x4_t*>(As + c.awr[j]) = R.a[j];
#pragma unroll
    for (int i = kc * kWPK; i < kW && i < (kc + 1) * kWPK; ++i) {
      const uint32_t w = R.b[i / 4][i % 4];
      if constexpr (BITS == 4)
        dequant4(w, s, b, o + kOPW * i);
      else
        dequant8(w, s, b, o + kOPW * i);
    }
    // runs whose words are all done by the end of this part
#pragma unroll
    for (int r = 0; r < kCPT; ++r) {
      const int last_word = (4 * r + 3) / kOPW;  // word holding the run's end
      if (last_word / kWPK == kc)
        *reinterpret_cast<u32x4_t*>(Bs + c.bwr[r]) =
            u32x4_t{o[4 * r], o[4 * r + 1], o[4 * r + 2], o[4 * r + 3]};
    }
  }
}

// K-loop.  Group q lives in register buffer q % 3 and LDS stage
// q % kStages.  Step g: issue group g + 3's loads (its buffer held group g,
// staged a step ago), multiply group g while staging group g + 1 (loaded
// two steps ago; after the last group this stages a copy nobody reads),
// barrier.  The body unrolls lcm(3, kStages) steps.
template <int BITS, int NMB>
__device__ __forceinline__ void prefill_kloop(const PrefillCtx<BITS>& c,
                                              f32x16_t (&acc)[2][2]) {
  const int G = c.groups;
  // Every step issues the same loads (past the last group it reloads it, a
  // cache hit), so the compiler can count exactly which loads a staging
  // must wait for.
  PrefillRegs<BITS> R[3];
  prefill_load(c, R[0], 0);
  prefill_load(c, R[1], min(1, G - 1));
  prefill_load(c, R[2], min(2, G - 1));
  prefill_store<BITS, 0>(c, R[0]);
  __syncthreads();
#define MLXR_PF_STEP(K)                                                       \
  {                                                                           \
    const int gg = g + K;                                                     \
    prefill_load(c, R[K % 3], min(gg + 3, G - 1));                            \
    __builtin_amdgcn_sched_barrier(0); /* keep the loads first */             \
    prefill_mma_store<BITS, NMB, K % kStages, (K + 1) % kStages>(             \
        c, R[(K + 1) % 3], acc);                                              \
    __syncthreads();                                                          \
  }
  // whole bodies, then the steps left (no early exit from the unrolled
  // body: the accumulators then keep one set of registers)
  constexpr int U = kStages == 3 ? 3 : 6;
  int g = 0;
#pragma nounroll
  for (; g + U <= G; g += U) {
    MLXR_PF_STEP(0)
    MLXR_PF_STEP(1)
    MLXR_PF_STEP(2)
    if constexpr (U == 6) {
      MLXR_PF_STEP(3)
      MLXR_PF_STEP(4)
      MLXR_PF_STEP(5)
    }
  }
  if (g < G) MLXR_PF_STEP(0)
  if (g + 1 < G) MLXR_PF_STEP(1)
  if (g + 2 < G) MLXR_PF_STEP(2)
  if (U == 6 && g + 3 < G) MLXR_PF_STEP(3)
  if (U == 6 && g + 4 < G) MLXR_PF_STEP(4)
#undef MLXR_PF_STEP
}

template <int BITS, bool GATED>
__global__ __launch_bounds__(kNT) void qgemm_prefill_kernel(QGemmArgs a,
                                                           int tiles_n,
                                                           uint32_t x_bytes) {

  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Workgroups go to the XCDs round robin (blockIdx % kXcds).  Number them
  // so that the N-tiles of one M-tile run on one XCD, one after another:
  // they read the same x rows, which then come from that XCD's L2.
  // (The live units, num_tiles x tiles_n, are dealt out evenly: the grid
  // is sized for the most tiles the dispatch can make.)
  const unsigned live = (unsigned)*a.num_tiles * tiles_n;
  const unsigned per = (live + kXcds - 1) / kXcds, j = blockIdx.x / kXcds;
  const unsigned L = (blockIdx.x % kXcds) * per + j;
  if (j >= per || L >= live) return;
  const int tile = (int)(L / tiles_n), nt = (int)(L - (unsigned)tile * tiles_n);
  const int e = a.tiles[2 * tile], slot0 = a.tiles[2 * tile + 1];
  const int rows = min(kBM, a.offsets[e + 1] - slot0);
  const int groups = a.K >> 6;
  const int wm = wave / kWN, wn = wave - wm * kWN;

  // x: one buffer over all rows (rows past the tile read out of range, 0)
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x), 0, (int)x_bytes, kBufFlags);
  // x chunk j of this thread: row id / 8, chunk id % 8 (id = tid + kNT j),
  // stored at its swizzled position
  uint32_t aoff[kACH];
  int awr[kACH];
  const float rdiv = 1.0f / (float)a.row_div;
#pragma unroll
  for (int j = 0; j < kACH; ++j) {
    const int id = tid + kNT * j, r = id >> 3, c = id & 7;
    awr[j] = r * 128 + 16 * (c ^ swz(r));
    uint32_t off = 0xFFFFFFF0u;
    if (r < rows) {
      const int slot = slot0 + r;
      int64_t row;
      if (a.x_by_slot) {
        row = slot;
      } else {
        const int flat = a.sorted[slot];
        row = a.row_map ? a.row_map[flat] : div_small(flat, a.row_div, rdiv);
      }
      off = (uint32_t)(row * a.x_ld * 2 + 16 * c);
    }
    aoff[j] = off;
  }
  // weights: thread -> column col, codes [kCODES*part, +kCODES) of a group;
  // the gated tile's first kBN/2 columns are gate channels, the rest up
  // (whole waves on each side)
  const int col = tid / kPARTS, part = tid - col * kPARTS;
  // which projection, from the (uniform) wave index: a buffer resource
  // must sit in scalar registers
  const int m = GATED ? (__builtin_amdgcn_readfirstlane(wave) >= kWM * kWN / 2) : 0;
  const int ch = GATED ? nt * (kBN / 2) + (col - m * (kBN / 2)) : nt * kBN + col;
  const QWeights& W = m ? a.w1 : a.w0;
  const int64_t row_bytes = (int64_t)a.K * BITS / 8;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(W.w) + (int64_t)e * a.N * (row_bytes / 4), 0,
      (int)(a.N * row_bytes), kBufFlags);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(W.scales) + (int64_t)e * a.N * groups, 0,
      a.N * groups * 2, kBufFlags);
  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(W.biases) + (int64_t)e * a.N * groups, 0,
      a.N * groups * 2, kBufFlags);
  const uint32_t woff = (uint32_t)(ch * row_bytes + part * (kCODES * BITS / 8));
  const uint32_t soff = (uint32_t)(ch * groups * 2);

  // operand rows of this lane: A rows wm*64 + 32 mb + l%32, B columns
  const int arow = wm * 64 + (lane & 31);
  int bc[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
    bc[nb] = (GATED ? nb * (kBN / 2) + wn * 32 : wn * 64 + nb * 32) + (lane & 31);
  const int kh = 8 * (lane >> 5);

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  // M-blocks of this wave that hold rows of the tile (the rest would
  // multiply zeros): one K-loop per count, chosen once
  const int wm_u = __builtin_amdgcn_readfirstlane(wm);
  const int nmb = rows > wm_u * 64 + 32 ? 2 : (rows > wm_u * 64 ? 1 : 0);
  // this thread's kCODES dequantised weights: column col, runs
  // kCPT part .. kCPT part + kCPT - 1 of the group
  PrefillCtx<BITS> c{xr, wr, sr, br, {}, {}, woff, soff, {}, smem,
                     {arow * 128, (arow + 32) * 128}, {swz(arow), swz(arow + 32)},
                     {bc[0] * 128, bc[1] * 128}, {swz(bc[0]), swz(bc[1])},
                     kh >> 3, groups};
#pragma unroll
  for (int j = 0; j < kACH; ++j) {
    c.aoff[j] = aoff[j];
    c.awr[j] = awr[j];
  }
#pragma unroll
  for (int i = 0; i < kCPT; ++i)
    c.bwr[i] = col * 128 + 16 * ((kCPT * part + i) ^ swz(col));
  if (nmb == 2)
    prefill_kloop<BITS, 2>(c, acc);
  else if (nmb == 1)
    prefill_kloop<BITS, 1>(c, acc);
  else
    prefill_kloop<BITS, 0>(c, acc);

  // Epilogue through LDS (the K-loop's last barrier freed the stages): the
  // waves write the tile's bf16 outputs -- SwiGLU of the gate and up sums,
  // or the down sums -- as [row][channel], rows 64 wm..64 wm + 63 in the
  // stage region wm, then every thread stores whole 16-byte runs of a row.
  // D[8(r/4) + 4(l/32) + r%4][l%32] of each 32 x 32 block.
  constexpr int OC = GATED ? kBN / 2 : kBN;  // output channels of the tile
  constexpr int OST = OC + 8;                // LDS row stride (bf16)
  static_assert((size_t)kBM * OST * 2 + kBM * 4 <= (size_t)kPrefillLds,
                "epilogue fits");
  auto region = [&](int q) -> uint16_t* {
    return reinterpret_cast<uint16_t*>(smem) + q * 64 * OST;
  };
  uint16_t* O = region(wm);
  int32_t* orow_s = reinterpret_cast<int32_t*>(smem + kBM * OST * 2);
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 32 * mb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);  // in the region
      if constexpr (GATED) {
        O[row * OST + wn * 32 + (lane & 31)] = swiglu_fast(acc[mb][0][r], acc[mb][1][r]);
      } else {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          O[row * OST + wn * 64 + 32 * nb + (lane & 31)] =
              __builtin_bit_cast(uint16_t, (__bf16)acc[mb][nb][r]);
      }
    }
  }
  if (!GATED && a.out_by_flat)
    for (int i = tid; i < rows; i += kNT) orow_s[i] = a.sorted[slot0 + i];
  __syncthreads();
  constexpr int CPR = OC / 8;  // 16-byte runs per row
  const int och0 = GATED ? nt * (kBN / 2) : nt * kBN;
  for (int id = tid; id < rows * CPR; id += kNT) {
    const int row = id / CPR, c = id - row * CPR;
    const int64_t orow = (!GATED && a.out_by_flat) ? orow_s[row] : slot0 + row;
    *reinterpret_cast<u32x4_t*>(a.out + orow * a.out_ld + och0 + 8 * c) =
        *reinterpret_cast<const u32x4_t*>(region(row >> 6) + (row & 63) * OST + 8 * c);
  }
}

}  // namespace

bool prefill_supported(const QGemmArgs& a, int64_t x_rows) {
  const int cols = a.gated ? kBN / 2 : kBN;
  // buffer offsets are 32-bit: x, and one expert's weights, under 2 GB
  // outputs leave as 16-byte runs of a row
  const bool out16 = (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 && a.out_ld % 8 == 0;
  return (a.bits == 4 || a.bits == 8) && a.K % 64 == 0 && a.N % cols == 0 &&
         a.sorted != nullptr && out16 && a.row_div >= 1 && a.row_div <= 65536 &&
         x_rows * a.x_ld * 2 < ((int64_t)1 << 31) &&
         (int64_t)a.N * a.K * a.bits / 8 < ((int64_t)1 << 31);
}

hipError_t launch_qgemm_prefill(const QGemmArgs& a, int64_t x_rows,
                                int64_t max_tiles, hipStream_t s) {
  if (max_tiles <= 0) return hipSuccess;
  const int tiles_n = a.N / (a.gated ? kBN / 2 : kBN);
  const size_t lds = kPrefillLds;
  const dim3 grid((unsigned)((max_tiles * tiles_n + kXcds - 1) / kXcds * kXcds));
  const uint32_t x_bytes = (uint32_t)(x_rows * a.x_ld * 2);
  ProfileScope prof(a.gated ? "qgemm_gated" : "qgemm_down", s);
#define MLXR_PF(B, G) \
  qgemm_prefill_kernel<B, G><<<grid, kNT, lds, s>>>(a, tiles_n, x_bytes)
  if (a.bits == 4) {
    if (a.gated)
      MLXR_PF(4, true);
    else
      MLXR_PF(4, false);
  } else {
    if (a.gated)
      MLXR_PF(8, true);
    else
      MLXR_PF(8, false);
  }
#undef MLXR_PF
  return hipGetLastError();
}

}  // namespace mlxr_moe
