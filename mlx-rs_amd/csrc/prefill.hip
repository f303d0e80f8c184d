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
// Workgroup: WM x WN waves; tile BM = 64 WM rows x BN = 64 WN columns (the
// gated kernel's columns are BN/2 gate channels then the same BN/2 up
// channels, so each wave holds matching gate and up sums for the SwiGLU
// epilogue).  K advances one quantisation group (64) per step through two
// LDS stages: while the waves multiply stage s, the global loads of the next
// group are in flight in registers, and after the multiplies they are
// dequantised into stage s^1.  One barrier per step.
//
// Each wave owns 64 x 64 outputs as 2 x 2 blocks of v_mfma_f32_32x32x16_bf16
// (K = 16 per instruction, four per group).  LDS rows are 64 bf16 padded to
// 72 (144 bytes), which keeps the 16-byte operand reads of 16 lanes on
// distinct banks.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {
namespace {

constexpr int kRowPad = 72;  // LDS row stride (bf16)

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// 8 codes of one 32-bit word (little end first) -> 4 words of bf16 pairs,
// each bf16(fmaf(code, s, b)).
template <int BITS>
__device__ __forceinline__ void dequant_word(uint32_t w, float s, float b,
                                             uint32_t* o);
template <>
__device__ __forceinline__ void dequant_word<4>(uint32_t w, float s, float b,
                                                uint32_t* o) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float c0 = (float)((w >> (8 * j)) & 15u);
    const float c1 = (float)((w >> (8 * j + 4)) & 15u);
    o[j] = pack_bf16(__builtin_fmaf(c0, s, b), __builtin_fmaf(c1, s, b));
  }
}
// 8-bit: one word = 4 codes -> 2 words of pairs
__device__ __forceinline__ void dequant_word8(uint32_t w, float s, float b,
                                              uint32_t* o) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float c0 = (float)((w >> (16 * j)) & 255u);
    const float c1 = (float)((w >> (16 * j + 8)) & 255u);
    o[j] = pack_bf16(__builtin_fmaf(c0, s, b), __builtin_fmaf(c1, s, b));
  }
}

template <int BITS, bool GATED, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void qgemm_prefill_kernel(
    QGemmArgs a, int tiles_n) {
  constexpr int NT = 64 * WM * WN;      // threads
  constexpr int BM = 64 * WM;           // rows per tile
  constexpr int BN = 64 * WN;           // B columns per tile
  constexpr int ACH = BM * 8 / NT;      // 16-byte x chunks per thread
  constexpr int CPC = 64 * BITS / 128;  // 16-byte code chunks per column
  constexpr int BCH = BN * CPC / NT;    // code chunks per thread
  constexpr int CODES = 128 / BITS;     // codes per chunk
  static_assert(BM * 8 % NT == 0 && BN * CPC % NT == 0, "even split");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  uint16_t* As = reinterpret_cast<uint16_t*>(smem);  // [2][BM][kRowPad]
  uint16_t* Bs = As + 2 * BM * kRowPad;              // [2][BN][kRowPad]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tile = blockIdx.x / tiles_n, nt = blockIdx.x - tile * tiles_n;
  if (tile >= *a.num_tiles) return;
  const int e = a.tiles[2 * tile], slot0 = a.tiles[2 * tile + 1];
  const int rows = min(BM, a.offsets[e + 1] - slot0);
  const int groups = a.K >> 6;
  const int wm = wave / WN, wn = wave - wm * WN;

  // x rows of this thread's A chunks (row = id / 8, 16-byte column id % 8)
  const uint16_t* ap[ACH];
  bool av[ACH];
#pragma unroll
  for (int j = 0; j < ACH; ++j) {
    const int id = tid + NT * j, r = id >> 3, c = id & 7;
    av[j] = r < rows;
    int64_t xr = 0;
    if (av[j]) {
      const int slot = slot0 + r;
      if (a.x_by_slot) {
        xr = slot;
      } else {
        const int flat = a.sorted[slot];
        xr = a.row_map ? a.row_map[flat] : flat / a.row_div;
      }
    }
    ap[j] = a.x + xr * a.x_ld + 8 * c;
  }
  // code chunks of this thread: column col, chunk q of the group
  const uint32_t* bp[BCH];
  const uint16_t* sp[BCH];
  const uint16_t* bbp[BCH];
  int bcol[BCH], bq[BCH];
#pragma unroll
  for (int j = 0; j < BCH; ++j) {
    const int id = tid + NT * j, col = id / CPC, q = id - col * CPC;
    bcol[j] = col;
    bq[j] = q;
    int m = 0, ch;
    if constexpr (GATED) {
      m = col >= BN / 2;
      ch = nt * (BN / 2) + (col - m * (BN / 2));
    } else {
      ch = nt * BN + col;
    }
    const QWeights& W = m ? a.w1 : a.w0;
    const int64_t row = (int64_t)e * a.N + ch;
    bp[j] = W.w + row * groups * (2 * BITS) + q * 4;
    sp[j] = W.scales + row * groups;
    bbp[j] = W.biases + row * groups;
  }

  u32x4_t areg[ACH], breg[BCH];
  uint16_t sreg[BCH], creg[BCH];
  auto load = [&](int g) {
#pragma unroll
    for (int j = 0; j < ACH; ++j)
      areg[j] = av[j] ? *reinterpret_cast<const u32x4_t*>(ap[j] + 64 * g)
                      : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < BCH; ++j) {
      breg[j] = *reinterpret_cast<const u32x4_t*>(bp[j] + g * (2 * BITS));
      sreg[j] = sp[j][g];
      creg[j] = bbp[j][g];
    }
  };
  auto store = [&](int st) {
    uint16_t* A = As + st * BM * kRowPad;
    uint16_t* B = Bs + st * BN * kRowPad;
#pragma unroll
    for (int j = 0; j < ACH; ++j) {
      const int id = tid + NT * j;
      *reinterpret_cast<u32x4_t*>(A + (id >> 3) * kRowPad + 8 * (id & 7)) = areg[j];
    }
#pragma unroll
    for (int j = 0; j < BCH; ++j) {
      const float s = bf16_to_f32(sreg[j]), b = bf16_to_f32(creg[j]);
      uint32_t o[CODES / 2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (BITS == 4)
          dequant_word<4>(breg[j][i], s, b, o + 4 * i);
        else
          dequant_word8(breg[j][i], s, b, o + 2 * i);
      }
      uint16_t* dst = B + bcol[j] * kRowPad + bq[j] * CODES;
#pragma unroll
      for (int i = 0; i < CODES / 8; ++i)
        *reinterpret_cast<u32x4_t*>(dst + 8 * i) =
            u32x4_t{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  // operand rows of this lane: A rows wm*64 + 32 mb + l%32, B columns
  const int arow = wm * 64 + (lane & 31);
  int bc[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
    bc[nb] = (GATED ? nb * (BN / 2) + wn * 32 : wn * 64 + nb * 32) + (lane & 31);
  const int kh = 8 * (lane >> 5);

  load(0);
  store(0);
  __syncthreads();
  for (int g = 0; g < groups; ++g) {
    const int st = g & 1;
    if (g + 1 < groups) load(g + 1);
    const uint16_t* A = As + st * BM * kRowPad;
    const uint16_t* B = Bs + st * BN * kRowPad;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      bf16x8_t af[2], bf[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
        af[mb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(
            A + (arow + 32 * mb) * kRowPad + 16 * kc + kh));
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        bf[nb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(
            B + bc[nb] * kRowPad + 16 * kc + kh));
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[mb][nb] = mfma32x32x16(af[mb], bf[nb], acc[mb][nb]);
    }
    if (g + 1 < groups) store(st ^ 1);
    __syncthreads();
  }

  // D[8(r/4) + 4(l/32) + r%4][l%32] of each 32 x 32 block
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = wm * 64 + 32 * mb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (row >= rows) continue;
      const int slot = slot0 + row;
      if constexpr (GATED) {
        const int ch = nt * (BN / 2) + wn * 32 + (lane & 31);
        a.out[(int64_t)slot * a.out_ld + ch] =
            swiglu_bf16(bf16_round(acc[mb][0][r]), bf16_round(acc[mb][1][r]));
      } else {
        const int64_t orow = a.out_by_flat ? a.sorted[slot] : slot;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const int ch = nt * BN + wn * 64 + 32 * nb + (lane & 31);
          a.out[orow * a.out_ld + ch] = f32_to_bf16(acc[mb][nb][r]);
        }
      }
    }
  }
}

}  // namespace

bool prefill_supported(const QGemmArgs& a) {
  constexpr int BN = 64 * kPrefillWavesN;
  const int cols = a.gated ? BN / 2 : BN;
  return (a.bits == 4 || a.bits == 8) && a.K % 64 == 0 && a.N % cols == 0 &&
         a.sorted != nullptr;
}

hipError_t launch_qgemm_prefill(const QGemmArgs& a, int64_t max_tiles,
                                hipStream_t s) {
  constexpr int WM = kPrefillTileRows / 64, WN = kPrefillWavesN;
  constexpr int BM = 64 * WM, BN = 64 * WN;
  if (max_tiles <= 0) return hipSuccess;
  const int tiles_n = a.N / (a.gated ? BN / 2 : BN);
  const size_t lds = (size_t)2 * (BM + BN) * kRowPad * 2;
  const dim3 grid((unsigned)(max_tiles * tiles_n));
  ProfileScope prof(a.gated ? "qgemm_gated" : "qgemm_down", s);
#define MLXR_PF(B, G) \
  qgemm_prefill_kernel<B, G, WM, WN><<<grid, 64 * WM * WN, lds, s>>>(a, tiles_n)
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
