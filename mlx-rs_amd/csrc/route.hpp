// Device routines shared by the router and the dispatch kernels:
//   wave_topk       top-K of one token's logits on one wave (K rounds of a
//                   wave maximum of order-preserving keys, ties to the lower
//                   id), softmax and the renormalised top-K weights;
//   block_dispatch  stable counting sort of up to 1024 expert ids held in
//                   LDS by one 1024-thread workgroup.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {

// Values one block_exclusive_scan covers at most.
constexpr int kScanVals = 5;

// Order-preserving key of a float: larger float, larger key; -0 == +0.
__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Original float of an order-preserving key (-0 maps back to +0).
__device__ __forceinline__ float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// DPP lane moves within 16-lane rows (no LDS): quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror, row_mirror; row_shr:n; row_bcast:15/31.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xf, false);
}

// Maximum over the wave of v, uniform: within each row by DPP, then the
// four row results through scalar registers.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp<0xB1>(v));
  v = max(v, dpp<0x4E>(v));
  v = max(v, dpp<0x141>(v));
  v = max(v, dpp<0x140>(v));
  const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0),
                         (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
  const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32),
                         (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
  return max(a, b);
}

// Inclusive prefix sum over the wave (integers): row scans by DPP shifts,
// then rows 1-3 add the running totals of the rows before them.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += dpp<0x111>(v);
  v += dpp<0x112>(v);
  v += dpp<0x114>(v);
  v += dpp<0x118>(v);
  v += dpp<0x142, 0xa>(v);
  v += dpp<0x143, 0xc>(v);
  return v;
}

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Per-wave scratch for wave_topk (unused by the selection below; kept for
// the callers' LDS layout).
struct TopkScratch {
  uint32_t key[64];
  int32_t id[64];
  float val[64];
};

// Top-K of logits[e], e < E, for one token, selected on the logits (softmax
// is monotone): descending, ties to the lower expert id -- the selection of
// argpartition(-K) plus a deterministic order inside the partition
// (crates/mlxr/src/ops/sort.rs:186-226, whose order is undefined).  Then
// softmax over all E (max-subtracted, lane sums in expert order e = l + 64s,
// butterfly across lanes) and w_k = p_k / sum_k p_k (k in order).
// BF16 (bf16 logits of a quantised router): softmax_axis keeps the bf16
// dtype (ops/arithmetic.rs:1298-1311), so the selection is on the bf16
// probabilities, where distinct logits can tie.  p_e = bf16((float)(
// exp((double)l_e - m) / S)) with S summed in double in the order above
// (double makes p independent of exp's last bits on either side); then
// denom = bf16(sum_k p_k in f32, k in order), w_k = bf16(p_k / denom).
// GEMMA (gemma4 Router::forward, crates/mlxr-lm/src/gemma4/text/text.rs:
// 621-665, router_post activations.rs:309-331): the selection is on the
// bf16 scores as given; then softmax over the K selected scores in bf16
// (non-precise: d_k = bf16(s_k - m), e_k = bf16(exp(d_k)) with exp in
// double, S = bf16(sum_k e_k in f32, k in order), p_k = bf16(e_k / S)) and
// w_k = bf16(p_k * per_expert_scale[id_k]).
// Returns on lane k < K its expert id (*out_id) and weight (*out_w).
template <int SLOTS, bool BF16 = false, bool GEMMA = false>
__device__ void wave_topk(const float* __restrict__ logits, int E, int K,
                          TopkScratch* sc, int* out_id, float* out_w,
                          const uint16_t* __restrict__ pes = nullptr) {
  const int lane = threadIdx.x & 63;
  float v[SLOTS];
  uint32_t key[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const int e = lane + 64 * s;
    v[s] = e < E ? logits[e] : 0.0f;
  }
  if constexpr (BF16) {
    float m = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
      if (lane + 64 * s < E) m = fmaxf(m, v[s]);
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) m = fmaxf(m, __shfl_xor(m, msk, 64));
    double ex[SLOTS];
    double acc = 0.0;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      ex[s] = lane + 64 * s < E ? exp((double)v[s] - (double)m) : 0.0;
      if (lane + 64 * s < E) acc += ex[s];
    }
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) acc += __shfl_xor(acc, msk, 64);
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) v[s] = bf16_round((float)(ex[s] / acc));
  }
#pragma unroll
  for (int s = 0; s < SLOTS; ++s)
    key[s] = lane + 64 * s < E ? float_key(v[s]) : 0u;  // 0: below every real key
  // K rounds: the largest remaining key, the lowest expert id among equal
  // keys (ids ascend with the slot, then the lane); lane k keeps the k-th
  // pick -- the selection order of argpartition(-K) with the order inside
  // the partition defined (descending, ties to the lower id).
  int my_id = 0;
  float my_val = 0.0f;
  (void)sc;
  for (int k = 0; k < K; ++k) {
    uint32_t m = key[0];
#pragma unroll
    for (int s = 1; s < SLOTS; ++s) m = max(m, key[s]);
    const uint32_t M = wave_max_u32(m);
    int sel = 0;
    bool found = false;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const uint64_t b = __ballot(key[s] == M);
      if (!found && b) {
        sel = 64 * s + (int)__builtin_ctzll(b);
        found = true;
      }
    }
    float vs = v[0];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      if (s == (sel >> 6)) vs = v[s];
      if (s == (sel >> 6) && lane == (sel & 63)) key[s] = 0u;
    }
    vs = readlane_f(vs, sel & 63);
    if (lane == k) {
      my_id = sel;
      my_val = vs;
    }
  }
  const int id = lane < K ? my_id : 0;
  const float top = readlane_f(my_val, 0);  // the largest selected value
  if constexpr (GEMMA) {
    const float m = top;
    const float dk = lane < K ? bf16_round(my_val - m) : 0.0f;
    const float ek = lane < K ? bf16_round((float)exp((double)dk)) : 0.0f;
    float S = 0.0f;
    for (int k = 0; k < K; ++k) S += readlane_f(ek, k);
    const float pk = bf16_round(ek / bf16_round(S));
    *out_id = id;
    *out_w = lane < K ? bf16_round(pk * bf16_to_f32(pes[id])) : 0.0f;
    return;
  }
  if constexpr (BF16) {
    const float p = lane < K ? my_val : 0.0f;
    float psum = 0.0f;
    for (int k = 0; k < K; ++k) psum += readlane_f(p, k);
    *out_id = id;
    *out_w = bf16_round(p / bf16_round(psum));
    return;
  }
  const float m = top;
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s)
    if (lane + 64 * s < E) acc += expf(v[s] - m);
  const float S = wave_sum_butterfly(acc);
  const float p = lane < K ? expf(my_val - m) / S : 0.0f;
  float psum = 0.0f;
  for (int k = 0; k < K; ++k) psum += readlane_f(p, k);
  *out_id = id;
  *out_w = p / psum;
}

// LDS of block_dispatch: per-wave match counts [wave * E + expert], scan
// scratch, offsets.
struct DispatchScratch {
  uint16_t tab[(kDispatchBlock / 64) * kMaxExperts];
  int wsum[kDispatchBlock / 64 + 1][kScanVals];
  int off[kMaxExperts];
  int wpos[kMaxExperts];
};

// Exclusive scans of NV ints per thread over a 1024-thread workgroup at
// once: DPP wave scans, the wave totals through LDS (one barrier), and every
// thread adds the totals of the waves before its own.
template <int NV>
__device__ __forceinline__ void block_exclusive_scan(const int (&v)[NV],
                                                     int (&ex)[NV],
                                                     int (&total)[NV],
                                                     int (*wsum)[kScanVals]) {
  static_assert(NV <= kScanVals, "scan scratch holds kScanVals values");
  constexpr int kWaves = kDispatchBlock / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) inc[k] = (int)wave_incl_scan((uint32_t)v[k]);
  if (lane == 63) {
#pragma unroll
    for (int k = 0; k < NV; ++k) wsum[wave][k] = inc[k];
  }
  __syncthreads();
  int pre[NV], all[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) pre[k] = all[k] = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int t = wsum[w][k];
      pre[k] += w < wave ? t : 0;
      all[k] += t;
    }
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    ex[k] = pre[k] + inc[k] - v[k];
    total[k] = all[k];
  }
}

// Work items per expert of cnt rows, listed long form first: the items of
// experts above kStreamTT4Rows rows (the streaming GEMM's slower 8-token
// form) take positions [0, total_long), the others follow.
__device__ __forceinline__ void work_counts(int cnt, bool expert, int& nw_long,
                                            int& nw_short) {
  const int nw = expert ? (cnt + kWorkRows - 1) / kWorkRows : 0;
  nw_long = cnt > kStreamTT4Rows ? nw : 0;
  nw_short = cnt > kStreamTT4Rows ? 0 : nw;
}

// Stable counting sort of ids[0..n) (n <= 1024, read by thread i) by expert
// in [0, E): counts, offsets, the active-expert list, the work item records,
// the M-tile list and sorted/inv, exactly the permutation of a stable
// argsort.  Ids of -1 are left out silently; other ids outside [0, E) are
// left out and flag *status.  Every thread of the 1024-thread workgroup
// must call it.  Three barriers.
__device__ void block_dispatch(int id_in, int n, int E, int tile_rows,
                               const DispatchBuffers& b, DispatchScratch* ls) {
  constexpr int kWaves = kDispatchBlock / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t* tab32 = reinterpret_cast<uint32_t*>(ls->tab);
  for (int i = tid; i < (kWaves * E + 1) / 2; i += kDispatchBlock) tab32[i] = 0u;
  const bool valid = tid < n;
  const int id = valid ? id_in : -1;
  const bool ok = valid && id >= 0 && id < E;
  if (valid && !ok && id != -1) *b.status = 1;
  // threads of this wave with the same id: ballots over the id bits
  uint64_t match = __ballot(ok);
  const int id_bits = E > 1 ? 32 - __clz(E - 1) : 0;
  for (int bit = 0; bit < id_bits; ++bit) {
    const bool on = ok && ((id >> bit) & 1);
    const uint64_t bal = __ballot(on);
    match &= on ? bal : ~bal;
  }
  const int r = __popcll(match & ((1ull << lane) - 1ull));
  __syncthreads();  // the table is zero
  if (ok && r == 0) ls->tab[wave * E + id] = (uint16_t)__popcll(match);
  __syncthreads();
  // per expert: the 16 wave counts read at once, their exclusive prefix
  // written back (the rank base of each wave), the total
  int cnt = 0;
  if (tid < E) {
    int c[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) c[w] = ls->tab[w * E + tid];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      ls->tab[w * E + tid] = (uint16_t)cnt;
      cnt += c[w];
    }
  }
  // one scan: row offsets, active experts, work items (long form first),
  // M-tiles
  const int has = (tid < E && cnt > 0) ? 1 : 0;
  int nw_long, nw_short;
  work_counts(cnt, tid < E, nw_long, nw_short);
  const int nw = nw_long + nw_short;
  const int nt = tid < E ? (cnt + tile_rows - 1) / tile_rows : 0;
  int ex[5], tot[5];
  block_exclusive_scan<5>({cnt, has, nw_long, nw_short, nt}, ex, tot, ls->wsum);
  const int off = ex[0], apos = ex[1], tpos = ex[4];
  const int wpos = nw_long ? ex[2] : tot[2] + ex[3];
  if (tid < E) {
    ls->off[tid] = off;
    ls->wpos[tid] = wpos;
  }
  __syncthreads();
  if (ok) {
    const int rank = ls->tab[wave * E + id] + r;
    const int pos = ls->off[id] + rank;
    b.sorted[pos] = tid;
    b.inv[tid] = pos;
    b.work[kWorkInts * (ls->wpos[id] + rank / kWorkRows) + 4 +
           rank % kWorkRows] = tid;
  }
  if (tid < E) {
    b.counts[tid] = cnt;
    b.offsets[tid] = off;
  }
  if (has) b.active[apos] = tid;
  for (int j = 0; j < nw; ++j) {
    int32_t* w = b.work + kWorkInts * (wpos + j);
    w[0] = tid;
    w[1] = off + j * kWorkRows;
    w[2] = min(kWorkRows, cnt - j * kWorkRows);
    w[3] = cnt;
  }
  for (int j = 0; j < nt; ++j) {
    b.tiles[2 * (tpos + j)] = tid;
    b.tiles[2 * (tpos + j) + 1] = off + j * tile_rows;
  }
  if (tid == 0) {
    b.offsets[E] = tot[0];
    *b.num_active = tot[1];
    *b.num_work = tot[2] + tot[3];
    *b.num_tiles = tot[4];
  }
}

// LDS of wave_dispatch: per expert its row count, first sorted slot and
// first work item.
struct WaveDispatchScratch {
  int cnt[kMaxExperts];
  int pos[kMaxExperts];
  int item[kMaxExperts];
};

// The same sort for at most 64 ids, one per lane of one wave (lane i < n:
// id_in), with no barrier.  Equal ids meet by ballots over the id bits (an
// id's rank among equals, the expert's row count); the expert table is
// then scanned 64 experts per pass (DPP prefix sums of packed per-expert
// fields: rows, active, M-tiles, long-form items; and short-form items),
// which gives every expert's first sorted slot and first work item (the
// long-form items first, in expert order, then the short).  Writes every
// output block_dispatch writes.
__device__ void wave_dispatch(int id_in, int n, int E, int tile_rows,
                              const DispatchBuffers& b,
                              WaveDispatchScratch* ls) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < n;
  const int id = valid ? id_in : -1;
  const bool ok = valid && id >= 0 && id < E;
  if (valid && !ok && id != -1) *b.status = 1;
  uint64_t match = __ballot(ok);
  const int id_bits = E > 1 ? 32 - __clz(E - 1) : 0;
  for (int bit = 0; bit < id_bits; ++bit) {
    const bool on = ok && ((id >> bit) & 1);
    const uint64_t bal = __ballot(on);
    match &= on ? bal : ~bal;
  }
  const int r = __popcll(match & ((1ull << lane) - 1ull));  // rank among equals
  const int c = ok ? __popcll(match) : 0;                   // the expert's rows
  const bool leader = ok && r == 0;
  // long-form items over all experts: the short-form items start after them
  const uint32_t wl_own =
      leader && c > kStreamTT4Rows ? (uint32_t)((c + kWorkRows - 1) / kWorkRows) : 0u;
  const int tot_long = (int)readlane_u32(wave_incl_scan(wl_own), 63);
  for (int e = lane; e < E; e += 64) ls->cnt[e] = 0;
  if (leader) ls->cnt[id] = c;
  // packed exclusive prefixes: rows | active << 8 | tiles << 16 |
  // long items << 24 (each total <= 64), and short items
  uint32_t carry_a = 0u, carry_b = 0u;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const int ce = e < E ? ls->cnt[e] : 0;
    const int nw = (ce + kWorkRows - 1) / kWorkRows;
    const int nt = (ce + tile_rows - 1) / tile_rows;
    const bool lng = ce > kStreamTT4Rows;
    const uint32_t pa = (uint32_t)ce | (ce > 0 ? 1u << 8 : 0u) |
                        ((uint32_t)nt << 16) | (lng ? (uint32_t)nw << 24 : 0u);
    const uint32_t pb = lng ? 0u : (uint32_t)nw;
    const uint32_t ia = wave_incl_scan(pa), ib = wave_incl_scan(pb);
    const uint32_t xa = ia - pa + carry_a, xb = ib - pb + carry_b;
    carry_a += readlane_u32(ia, 63);
    carry_b += readlane_u32(ib, 63);
    const int off = (int)(xa & 0xffu);
    if (e < E) {
      b.counts[e] = ce;
      b.offsets[e] = off;
    }
    if (ce > 0) {
      const int first = lng ? (int)(xa >> 24) : tot_long + (int)xb;
      ls->pos[e] = off;
      ls->item[e] = first;
      b.active[(xa >> 8) & 0xffu] = e;
      for (int j = 0; j < nw; ++j) {
        int32_t* w = b.work + kWorkInts * (first + j);
        w[0] = e;
        w[1] = off + j * kWorkRows;
        w[2] = min(kWorkRows, ce - j * kWorkRows);
        w[3] = ce;
      }
      const int tb = (int)((xa >> 16) & 0xffu);
      for (int j = 0; j < nt; ++j) {
        b.tiles[2 * (tb + j)] = e;
        b.tiles[2 * (tb + j) + 1] = off + j * tile_rows;
      }
    }
  }
  if (ok) {
    const int pos = ls->pos[id] + r;
    b.sorted[pos] = lane;
    b.inv[lane] = pos;
    b.work[kWorkInts * (ls->item[id] + r / kWorkRows) + 4 + r % kWorkRows] = lane;
  }
  if (lane == 0) {
    b.offsets[E] = (int)(carry_a & 0xffu);
    *b.num_active = (int)((carry_a >> 8) & 0xffu);
    *b.num_work = tot_long + (int)carry_b;
    *b.num_tiles = (int)((carry_a >> 16) & 0xffu);
  }
}

}  // namespace mlxr_moe
