// Device routines shared by the router and the dispatch kernels:
//   wave_topk       top-K of one token's logits on one wave (radix select on
//                   order-preserving keys, ballots only), softmax and the
//                   renormalised top-K weights;
//   block_dispatch  stable counting sort of up to 1024 expert ids held in
//                   LDS by one 1024-thread workgroup.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {

// Order-preserving key of a float: larger float, larger key; -0 == +0.
__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Per-wave scratch for wave_topk: the K selected (key, id) pairs.
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
  const uint64_t below = (1ull << lane) - 1ull;
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
  // theta = largest key with at least K keys >= theta (the K-th largest)
  uint32_t theta = 0u;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = theta | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) cnt += __popcll(__ballot(key[s] >= cand));
    if (cnt >= K) theta = cand;
  }
  // keys above theta, then the lowest-id keys equal to theta
  int left = K;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) left -= __popcll(__ballot(key[s] > theta));
  int base = 0;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const uint64_t eq = __ballot(key[s] == theta);
    const int take = min(__popcll(eq), left);
    left -= take;
    const bool sel =
        key[s] > theta || (key[s] == theta && __popcll(eq & below) < take);
    const uint64_t sm = __ballot(sel);
    if (sel) {
      const int pos = base + __popcll(sm & below);
      sc->key[pos] = key[s];
      sc->id[pos] = lane + 64 * s;
      sc->val[pos] = v[s];
    }
    base += __popcll(sm);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // rank of each selected pair: larger key first, then lower id
  int my_id = 0, rank = 0;
  uint32_t my_key = 0u;
  float my_val = 0.0f;
  if (lane < K) {
    my_key = sc->key[lane];
    my_id = sc->id[lane];
    my_val = sc->val[lane];
    for (int j = 0; j < K; ++j) {
      const uint32_t kj = sc->key[j];
      const int ij = sc->id[j];
      rank += (kj > my_key || (kj == my_key && ij < my_id)) ? 1 : 0;
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < K) {
    sc->id[rank] = my_id;
    sc->val[rank] = my_val;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int id = lane < K ? sc->id[lane] : 0;
  if constexpr (GEMMA) {
    const float m = sc->val[0];
    const float dk = lane < K ? bf16_round(sc->val[lane] - m) : 0.0f;
    const float ek = lane < K ? bf16_round((float)exp((double)dk)) : 0.0f;
    float S = 0.0f;
    for (int k = 0; k < K; ++k) S += __shfl(ek, k, 64);
    const float pk = bf16_round(ek / bf16_round(S));
    *out_id = id;
    *out_w = lane < K ? bf16_round(pk * bf16_to_f32(pes[id])) : 0.0f;
    return;
  }
  if constexpr (BF16) {
    const float p = lane < K ? sc->val[lane] : 0.0f;
    float psum = 0.0f;
    for (int k = 0; k < K; ++k) psum += __shfl(p, k, 64);
    *out_id = id;
    *out_w = bf16_round(p / bf16_round(psum));
    return;
  }
  // the selected logits come from LDS: no dependent re-read of memory
  const float m = sc->val[0];
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s)
    if (lane + 64 * s < E) acc += expf(v[s] - m);
  const float S = wave_sum_butterfly(acc);
  const float p = lane < K ? expf(sc->val[lane] - m) / S : 0.0f;
  float psum = 0.0f;
  for (int k = 0; k < K; ++k) psum += __shfl(p, k, 64);
  *out_id = id;
  *out_w = p / psum;
}

// LDS of block_dispatch: per-wave match counts, scan scratch, offsets.
struct DispatchScratch {
  uint16_t tab[kDispatchBlock / 64][kMaxExperts];
  int wsum[kDispatchBlock / 64 + 1][4];
  int off[kMaxExperts];
  int wpos[kMaxExperts];
};

// Exclusive scans of four ints per thread over a 1024-thread workgroup at
// once: wave scans, then wave 0 scans the 16 wave totals.  Two barriers.
__device__ __forceinline__ void block_exclusive_scan4(const int (&v)[4],
                                                      int (&ex)[4],
                                                      int (&total)[4],
                                                      int (*wsum)[4]) {
  constexpr int kWaves = kDispatchBlock / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    inc[k] = v[k];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(inc[k], o, 64);
      if (lane >= o) inc[k] += u;
    }
  }
  if (lane == 63) {
#pragma unroll
    for (int k = 0; k < 4; ++k) wsum[wave][k] = inc[k];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int t = lane < kWaves ? wsum[lane][k] : 0;
      int s = t;
#pragma unroll
      for (int o = 1; o < kWaves; o <<= 1) {
        const int u = __shfl_up(s, o, 64);
        if (lane >= o) s += u;
      }
      if (lane < kWaves) wsum[lane][k] = s - t;
      if (lane == kWaves - 1) wsum[kWaves][k] = s;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    ex[k] = wsum[wave][k] + inc[k] - v[k];
    total[k] = wsum[kWaves][k];
  }
}

// Stable counting sort of ids[0..n) (n <= 1024, read by thread i) by expert
// in [0, E): counts, offsets, the active-expert list, the work item records,
// the M-tile list and sorted/inv, exactly the permutation of a stable
// argsort.  Ids of -1 are
// left out silently; other ids outside [0, E) are left out and flag
// *status.  Every thread of the 1024-thread workgroup must call it.
__device__ void block_dispatch(int id_in, int n, int E, int tile_rows,
                               const DispatchBuffers& b, DispatchScratch* ls) {
  constexpr int kWaves = kDispatchBlock / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kWaves * E; i += kDispatchBlock)
    ls->tab[i / E][i % E] = 0;
  __syncthreads();
  const bool valid = tid < n;
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
  const int r = __popcll(match & ((1ull << lane) - 1ull));
  if (ok && r == 0) ls->tab[wave][id] = (uint16_t)__popcll(match);
  __syncthreads();
  int cnt = 0;
  if (tid < E) {
    for (int w = 0; w < kWaves; ++w) {
      const int c = ls->tab[w][tid];
      ls->tab[w][tid] = (uint16_t)cnt;
      cnt += c;
    }
  }
  // one scan: row offsets, active experts, work items, M-tiles
  const int has = (tid < E && cnt > 0) ? 1 : 0;
  const int nw = tid < E ? (cnt + kWorkRows - 1) / kWorkRows : 0;
  const int nt = tid < E ? (cnt + tile_rows - 1) / tile_rows : 0;
  int ex[4], tot[4];
  block_exclusive_scan4({cnt, has, nw, nt}, ex, tot, ls->wsum);
  const int off = ex[0], apos = ex[1], wpos = ex[2], tpos = ex[3];
  if (tid < E) {
    b.counts[tid] = cnt;
    b.offsets[tid] = off;
    ls->off[tid] = off;
    ls->wpos[tid] = wpos;
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
    *b.num_work = tot[2];
    *b.num_tiles = tot[3];
  }
  __syncthreads();
  if (ok) {
    const int rank = ls->tab[wave][id] + r;
    const int pos = ls->off[id] + rank;
    b.sorted[pos] = tid;
    b.inv[tid] = pos;
    b.work[kWorkInts * (ls->wpos[id] + rank / kWorkRows) + 4 +
           rank % kWorkRows] = tid;
  }
}

}  // namespace mlxr_moe
