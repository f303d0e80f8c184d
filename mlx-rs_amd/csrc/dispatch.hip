// Token -> expert dispatch on gfx950: a stable counting sort of the flat
// (token, k) expert ids into per-expert contiguous row blocks.
//
// Replaces gather_sort / scatter_unsort
// (crates/mlxr-lm/src/nn/switch.rs:499-517): order = argsort(flat ids),
// inv = argsort(order).  Because the sort is stable the permutation equals
// that argsort exactly.  Two kernels:
//   rank  (one 1024-thread workgroup per 1024 ids): per-wave match masks from
//         ballots over the id bits give each id its rank among equal ids of
//         its wave; an LDS table of per-wave counts turns that into a rank
//         within the workgroup and a per-workgroup histogram.
//   scan  (one workgroup): per-expert prefix over workgroups, exclusive scan
//         over experts (offsets), the list of experts with rows, the work
//         item records and M-tile list for the GEMMs, and the scatter into
//         sorted/inv (and the flat rows of the work records).
// Ids outside [0, E) are left out of every expert and flagged in *status.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "route.hpp"

namespace mlxr_moe {
namespace {

constexpr int kWaves = kDispatchBlock / 64;
// tokens per workgroup of route_fused_kernel (a wave each; the other waves
// only join the sort of the last workgroup)
#ifndef MLXR_ROUTE_FUSED_TPW
#define MLXR_ROUTE_FUSED_TPW 4
#endif
#ifndef MLXR_ROUTE_SMALL_TOKENS
#define MLXR_ROUTE_SMALL_TOKENS 16
#endif

// The rank pass of one workgroup (1024 ids): per-wave counts of each
// expert in LDS, their prefix within the workgroup, the workgroup's
// histogram into block_hist (with COHERENT through agent-scope atomic
// stores, for a workgroup of the same launch to read) and each id's rank.
template <bool COHERENT>
__device__ __forceinline__ void dispatch_rank_body(const int32_t* __restrict__ ids, int n,
                                                   int E, int32_t* block_hist,
                                                   int32_t* __restrict__ rank,
                                                   int32_t* __restrict__ status, uint16_t* tab) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kWaves * E; i += kDispatchBlock) tab[i] = 0;
  __syncthreads();
  const int64_t gi = (int64_t)blockIdx.x * kDispatchBlock + tid;
  const bool valid = gi < n;
  const int id = valid ? ids[gi] : -1;
  const bool ok = valid && id >= 0 && id < E;
  if (valid && !ok && id != -1) *status = 1;
  uint64_t match = __ballot(ok);
  const int id_bits = E > 1 ? 32 - __clz(E - 1) : 0;
  for (int b = 0; b < id_bits; ++b) {
    const bool bit = ok && ((id >> b) & 1);
    const uint64_t bal = __ballot(bit);
    match &= bit ? bal : ~bal;
  }
  const uint64_t below = (1ull << lane) - 1ull;
  const int r = __popcll(match & below);
  if (ok && r == 0) tab[wave * E + id] = (uint16_t)__popcll(match);
  __syncthreads();
  for (int e = tid; e < E; e += kDispatchBlock) {
    // the 16 wave counts read at once, their exclusive prefix written back
    int c[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) c[w] = tab[w * E + e];
    int run = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      tab[w * E + e] = (uint16_t)run;
      run += c[w];
    }
    if constexpr (COHERENT)
      __hip_atomic_store(block_hist + (int64_t)blockIdx.x * E + e, run, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    else
      block_hist[(int64_t)blockIdx.x * E + e] = run;
  }
  __syncthreads();
  if (ok) rank[gi] = tab[wave * E + id] + r;
}

__global__ __launch_bounds__(kDispatchBlock) void dispatch_rank_kernel(
    const int32_t* __restrict__ ids, int n, int E,
    int32_t* __restrict__ block_hist, int32_t* __restrict__ rank,
    int32_t* __restrict__ status) {
  extern __shared__ uint16_t tab[];  // [kWaves][E]
  dispatch_rank_body<false>(ids, n, E, block_hist, rank, status, tab);
}

// Index of the last entry of the ascending start[0..n) that is <= v.
__device__ __forceinline__ int upper_slot(const int* start, int n, int v) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (start[mid] <= v)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// One workgroup: per-expert prefix over the workgroups' histograms,
// counts/offsets, the active list, and the work item and M-tile lists
// (written by all threads, each list entry finding its expert by binary
// search).  The scatter into sorted/inv is dispatch_scatter_kernel.
// (With COHERENT the histograms, written by other workgroups of the same
// launch, are read with agent-scope atomic loads.)
struct ScanScratch {
  int s_off[kMaxExperts], s_wlong[kMaxExperts], s_wshort[kMaxExperts], s_tpos[kMaxExperts];
  int wsum[kWaves + 1][kScanVals];
};
template <bool COHERENT>
__device__ __forceinline__ void dispatch_scan_body(int n, int E, int nb, int tile_rows,
                                                   const DispatchBuffers& b, ScanScratch& ss) {
  int *s_off = ss.s_off, *s_wlong = ss.s_wlong, *s_wshort = ss.s_wshort, *s_tpos = ss.s_tpos;
  auto& wsum = ss.wsum;
  const int tid = threadIdx.x;
  // exclusive prefix of each expert's column over the workgroups, 16 loads
  // in flight at a time (a load after a store of the same array would wait
  // for it)
  int cnt = 0;
  if (tid < E) {
    constexpr int kChunk = 16;
    for (int b0 = 0; b0 < nb; b0 += kChunk) {
      int c[kChunk];
#pragma unroll
      for (int j = 0; j < kChunk; ++j)
        c[j] = b0 + j >= nb ? 0
               : COHERENT ? __hip_atomic_load(b.block_hist + (int64_t)(b0 + j) * E + tid,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : b.block_hist[(int64_t)(b0 + j) * E + tid];
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        if (b0 + j < nb) b.block_hist[(int64_t)(b0 + j) * E + tid] = cnt;
        cnt += c[j];
      }
    }
  }
  // one scan: row offsets, active experts, work items (long form first),
  // M-tiles
  const int has = (tid < E && cnt > 0) ? 1 : 0;
  int nw_long, nw_short;
  work_counts(cnt, tid < E, nw_long, nw_short);
  const int nt = (tid < E) ? (cnt + tile_rows - 1) / tile_rows : 0;
  int ex[5], tot[5];
  block_exclusive_scan<5>({cnt, has, nw_long, nw_short, nt}, ex, tot, wsum);
  const int off = ex[0], tpos = ex[4];
  const int wpos = nw_long ? ex[2] : tot[2] + ex[3];
  const int total = tot[0], n_work = tot[2] + tot[3], n_tiles = tot[4];
  if (tid < E) {
    b.counts[tid] = cnt;
    b.offsets[tid] = off;
    s_off[tid] = off;
    s_wlong[tid] = ex[2];
    s_wshort[tid] = tot[2] + ex[3];
    b.work_first[tid] = wpos;
    s_tpos[tid] = tpos;
  }
  if (has) b.active[ex[1]] = tid;
  if (tid == 0) {
    b.offsets[E] = total;
    *b.num_active = tot[1];
    *b.num_work = n_work;
    *b.num_tiles = n_tiles;
  }
  __syncthreads();
  // experts with no items in a region share their start with the next: the
  // search (the long-form region, then the rest) finds the last expert
  // starting at or before the entry, which has items there
  for (int i = tid; i < n_work; i += kDispatchBlock) {
    const int* start = i < tot[2] ? s_wlong : s_wshort;
    const int e = upper_slot(start, E, i), j = i - start[e];
    const int cnt_e = (e + 1 < E ? s_off[e + 1] : total) - s_off[e];
    int32_t* w = b.work + kWorkInts * i;
    w[0] = e;
    w[1] = s_off[e] + j * kWorkRows;
    w[2] = min(kWorkRows, cnt_e - j * kWorkRows);
    w[3] = cnt_e;
  }
  for (int i = tid; i < n_tiles; i += kDispatchBlock) {
    const int e = upper_slot(s_tpos, E, i), j = i - s_tpos[e];
    b.tiles[2 * i] = e;
    b.tiles[2 * i + 1] = s_off[e] + j * tile_rows;
  }
}

__global__ __launch_bounds__(kDispatchBlock) void dispatch_scan_kernel(
    int n, int E, int nb, int tile_rows, DispatchBuffers b) {
  __shared__ ScanScratch ss;
  dispatch_scan_body<false>(n, E, nb, tile_rows, b, ss);
}

// The rank pass and the scan in one launch: every workgroup ranks its 1024
// ids and stores its histogram with agent-scope atomic stores, waits until
// they have completed and adds one to *counter; the workgroup whose add
// returns gridDim.x - 1 runs the scan, reading the histograms with
// agent-scope atomic loads (no fence: on this part a release or acquire
// fence writes back or invalidates the whole L2).  *counter is 0 when the
// launch starts (the router launch of the block forward clears it).
// Against the two launches (graph steps): c3 T=2048 344.5 to 342.5 µs,
// c3 T=4096 516.0 to 514.8, c2 T=256 164.5 to 163.4; bit-identical.
__global__ __launch_bounds__(kDispatchBlock) void dispatch_rank_scan_kernel(
    const int32_t* __restrict__ ids, int n, int E, int tile_rows, DispatchBuffers b,
    int32_t* counter) {
  extern __shared__ uint16_t tab[];  // [kWaves][E]
  __shared__ ScanScratch ss;
  __shared__ int last;
  dispatch_rank_body<true>(ids, n, E, b.block_hist, b.rank, b.status, tab);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (int)gridDim.x - 1;
  __syncthreads();
  if (last) dispatch_scan_body<true>(n, E, (int)gridDim.x, tile_rows, b, ss);
}

// Every workgroup of the rank pass again: sorted/inv and the flat rows of
// the work records, from the offsets and per-workgroup prefixes.
__global__ __launch_bounds__(kDispatchBlock) void dispatch_scatter_kernel(
    const int32_t* __restrict__ ids, int n, int E, DispatchBuffers b) {
  const int64_t i = (int64_t)blockIdx.x * kDispatchBlock + threadIdx.x;
  if (i >= n) return;
  const int e = ids[i];
  if (e < 0 || e >= E) return;
  const int base = b.offsets[e];
  const int r = b.block_hist[(int64_t)blockIdx.x * E + e] + b.rank[i];
  const int pos = base + r;
  b.sorted[pos] = (int32_t)i;
  b.inv[i] = pos;
  b.work[kWorkInts * (b.work_first[e] + r / kWorkRows) + 4 + r % kWorkRows] =
      (int32_t)i;
}

// n <= 1024 ids: the whole sort in one workgroup.
__global__ __launch_bounds__(kDispatchBlock) void dispatch_small_kernel(
    const int32_t* __restrict__ ids, int n, int E, int tile_rows,
    DispatchBuffers b, int reset_status) {
  __shared__ DispatchScratch ls;
  if (reset_status && threadIdx.x == 0) *b.status = 0;
  __syncthreads();
  const int id = (int)threadIdx.x < n ? ids[threadIdx.x] : -1;
  block_dispatch(id, n, E, tile_rows, b, &ls);
}

// Decode routing in one workgroup (T * K <= 1024): top-K of every token
// (16 waves over the tokens), the renormalised weights, the status reset and
// the counting sort of the T * K expert ids.
template <int SLOTS, bool BF16>
__global__ __launch_bounds__(kDispatchBlock) void route_small_kernel(
    const float* __restrict__ logits, int64_t ld, int T, int E, int K,
    int32_t* __restrict__ idx, float* __restrict__ wts, int tile_rows,
    DispatchBuffers b) {
  __shared__ DispatchScratch ls;
  __shared__ TopkScratch sc[kDispatchBlock / 64];
  __shared__ int ids[kDispatchBlock];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) *b.status = 0;
  for (int t = wave; t < T; t += kDispatchBlock / 64) {
    int id;
    float wt;
    wave_topk<SLOTS, BF16>(logits + (int64_t)t * ld, E, K, &sc[wave], &id, &wt);
    if (lane < K) {
      idx[(int64_t)t * K + lane] = id;
      wts[(int64_t)t * K + lane] = wt;
      ids[t * K + lane] = id;
    }
  }
  __syncthreads();
  const int n = T * K;
  block_dispatch((int)threadIdx.x < n ? ids[threadIdx.x] : -1, n, E,
                 tile_rows, b, &ls);
}

// Decode routing for at most 64 ids (T * K <= 64): one wave per token for
// the top-K (blockDim = 64 * min(T, 16)), then wave 0 sorts the ids
// (wave_dispatch: ballots and one scan of the expert table, no barrier).
template <int SLOTS, bool BF16>
__global__ __launch_bounds__(kDispatchBlock) void route_wave_kernel(
    const float* __restrict__ logits, int64_t ld, int T, int E, int K,
    int32_t* __restrict__ idx, float* __restrict__ wts, int tile_rows,
    DispatchBuffers b) {
  __shared__ WaveDispatchScratch ls;
  __shared__ int ids[64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  if (threadIdx.x == 0) *b.status = 0;
  for (int t = wave; t < T; t += waves) {
    int id;
    float wt;
    wave_topk<SLOTS, BF16>(logits + (int64_t)t * ld, E, K, nullptr, &id, &wt);
    if (lane < K) {
      idx[(int64_t)t * K + lane] = id;
      wts[(int64_t)t * K + lane] = wt;
      ids[t * K + lane] = id;
    }
  }
  __syncthreads();
  if (wave == 0) {
    const int n = T * K;
    wave_dispatch(lane < n ? ids[lane] : -1, n, E, tile_rows, b, &ls);
  }
}

// Decode routing of 16 < T tokens whose T * K ids fit one workgroup, in one
// launch: a wave per token for the top-K (MLXR_ROUTE_FUSED_TPW tokens per
// workgroup: spread over as many CUs as the separate top-K kernel), then the
// workgroup that finishes last runs the counting sort of all T * K ids.
// Measured against the top-K kernel plus the one-workgroup sort (graph steps
// of 8 forwards): c2 T=64 97.3 to 95.8 µs, c2 T=32 82.0 to 80.7, c4 T=64
// 185.2 to 183.9, c6 T=64 125.8 to 124.1; 16 tokens per workgroup lost at
// c4 T=64 (185.2 to 188.7).
// Every workgroup stores its ids with agent-scope atomic stores (written
// through to where every XCD reads them), waits until those stores have
// completed, then adds one to *counter; the workgroup whose add returns
// gridDim.x - 1 reads the ids back with agent-scope atomic loads.  No release
// or acquire fence: on this part those write back and invalidate the whole
// L2.  *counter is 0 when the launch starts (the logits launch before it
// clears it); the status word is cleared and set by the last workgroup only.
template <int SLOTS, bool BF16>
__global__ __launch_bounds__(kDispatchBlock) void route_fused_kernel(
    const float* __restrict__ logits, int64_t ld, int T, int E, int K,
    int32_t* idx, float* __restrict__ wts, int tile_rows, DispatchBuffers b,
    int32_t* counter) {
  __shared__ DispatchScratch ls;
  __shared__ int last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = (int)blockIdx.x * MLXR_ROUTE_FUSED_TPW + wave;
  if (wave < MLXR_ROUTE_FUSED_TPW && t < T) {
    int id;
    float wt;
    wave_topk<SLOTS, BF16>(logits + (int64_t)t * ld, E, K, nullptr, &id, &wt);
    if (lane < K) {
      __hip_atomic_store(idx + (int64_t)t * K + lane, id, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      wts[(int64_t)t * K + lane] = wt;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (int)gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  if (threadIdx.x == 0) *b.status = 0;
  __syncthreads();
  const int n = T * K;
  const int id = (int)threadIdx.x < n
                     ? __hip_atomic_load(idx + threadIdx.x, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT)
                     : -1;
  block_dispatch(id, n, E, tile_rows, b, &ls);
}

__global__ __launch_bounds__(256) void dispatch_identity_kernel(
    int n, int tile_rows, DispatchBuffers b) {
  const int tid = threadIdx.x;
  const int n_tiles = (n + tile_rows - 1) / tile_rows;
  if (tid == 0) {
    b.counts[0] = n;
    b.offsets[0] = 0;
    b.offsets[1] = n;
    b.active[0] = 0;
    *b.num_active = n > 0 ? 1 : 0;
    *b.num_work = (n + kWorkRows - 1) / kWorkRows;
    *b.num_tiles = n_tiles;
  }
  for (int j = tid; j < n_tiles; j += 256) {
    b.tiles[2 * j] = 0;
    b.tiles[2 * j + 1] = j * tile_rows;
  }
  for (int i = tid; i < n; i += 256) {
    b.sorted[i] = i;
    b.inv[i] = i;
  }
  for (int j = tid; j * kWorkRows < n; j += 256) {
    int32_t* w = b.work + kWorkInts * j;
    w[0] = 0;
    w[1] = j * kWorkRows;
    w[2] = min(kWorkRows, n - j * kWorkRows);
    w[3] = n;
    for (int i = 0; i < kWorkRows; ++i) w[4 + i] = j * kWorkRows + i;
  }
}

__global__ void zero_status_kernel(int32_t* status) { *status = 0; }

// gather_qmm row preparation: flat row r = b * M + m takes expert
// rhs[b] and x row xb(b) * M + m; rows with an index out of range get
// expert -1 (left out by the dispatch), a zero output row and *status = 1.
__global__ __launch_bounds__(256) void gather_prep_kernel(
    const uint32_t* __restrict__ lhs, const uint32_t* __restrict__ rhs,
    int64_t B, int64_t M, int64_t x_batch, int64_t E, int64_t N,
    int32_t* __restrict__ ids, int32_t* __restrict__ xrow,
    uint16_t* __restrict__ out, int32_t* __restrict__ status) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= B * M) return;
  const int64_t b = r / M, m = r % M;
  const int64_t xb = lhs ? (int64_t)lhs[b] : b / (B / x_batch);
  const uint32_t e = rhs[b];
  if (e >= (uint64_t)E || xb >= x_batch) {
    ids[r] = -1;
    xrow[r] = 0;
    *status = 1;
    for (int64_t n = 0; n < N; ++n) out[r * N + n] = 0;
    return;
  }
  ids[r] = (int32_t)e;
  xrow[r] = (int32_t)(xb * M + m);
}

}  // namespace

hipError_t launch_zero_status(int32_t* status, hipStream_t s) {
  zero_status_kernel<<<1, 1, 0, s>>>(status);
  return hipGetLastError();
}

int64_t dispatch_max_tiles(int64_t n, int64_t E, int tile_rows) {
  return (n + tile_rows - 1) / tile_rows + (E < n ? E : n);
}

hipError_t launch_dispatch(const int32_t* ids, int64_t n, int64_t E,
                           int tile_rows, const DispatchBuffers& b,
                           bool reset_status, hipStream_t s, int32_t* counter) {
  ProfileScope prof("dispatch", s);
  if (n <= kDispatchBlock) {
    dispatch_small_kernel<<<1, kDispatchBlock, 0, s>>>(
        ids, (int)n, (int)E, tile_rows, b, reset_status ? 1 : 0);
    return hipGetLastError();
  }
  const int nb = (int)((n + kDispatchBlock - 1) / kDispatchBlock);
  if (reset_status) zero_status_kernel<<<1, 1, 0, s>>>(b.status);
  if (counter) {
    dispatch_rank_scan_kernel<<<nb, kDispatchBlock, (size_t)kWaves * E * sizeof(uint16_t),
                                s>>>(ids, (int)n, (int)E, tile_rows, b, counter);
  } else {
    dispatch_rank_kernel<<<nb, kDispatchBlock,
                           (size_t)kWaves * E * sizeof(uint16_t), s>>>(
        ids, (int)n, (int)E, b.block_hist, b.rank, b.status);
    dispatch_scan_kernel<<<1, kDispatchBlock, 0, s>>>((int)n, (int)E, nb,
                                                      tile_rows, b);
  }
  dispatch_scatter_kernel<<<nb, kDispatchBlock, 0, s>>>(ids, (int)n, (int)E, b);
  return hipGetLastError();
}

template <bool BF16>
void route_small_launch(const float* logits, int64_t ld, int64_t T, int64_t E,
                        int64_t K, int32_t* idx, float* wts, int tile_rows,
                        const DispatchBuffers& b, hipStream_t s) {
  const int slots = (int)((E + 63) / 64);
  // at most 64 ids: a wave per token and the one-wave sort
  const bool one_wave = T * K <= 64;
  const unsigned threads = one_wave ? 64u * (unsigned)std::min<int64_t>(T, 16) : kDispatchBlock;
#define MLXR_RS(S)                                                         \
  do {                                                                     \
    if (one_wave)                                                          \
      route_wave_kernel<S, BF16><<<1, threads, 0, s>>>(                    \
          logits, ld, (int)T, (int)E, (int)K, idx, wts, tile_rows, b);     \
    else                                                                   \
      route_small_kernel<S, BF16><<<1, kDispatchBlock, 0, s>>>(            \
          logits, ld, (int)T, (int)E, (int)K, idx, wts, tile_rows, b);     \
  } while (0)
  if (slots <= 1)
    MLXR_RS(1);
  else if (slots <= 2)
    MLXR_RS(2);
  else if (slots <= 4)
    MLXR_RS(4);
  else if (slots <= 8)
    MLXR_RS(8);
  else
    MLXR_RS(16);
#undef MLXR_RS
}

template <bool BF16>
void route_fused_launch(const float* logits, int64_t ld, int64_t T, int64_t E,
                        int64_t K, int32_t* idx, float* wts, int tile_rows,
                        const DispatchBuffers& b, int32_t* counter, hipStream_t s) {
  const int slots = (int)((E + 63) / 64);
  const unsigned grid = (unsigned)((T + MLXR_ROUTE_FUSED_TPW - 1) / MLXR_ROUTE_FUSED_TPW);
#define MLXR_RF(S)                                                                 \
  route_fused_kernel<S, BF16><<<grid, kDispatchBlock, 0, s>>>(                     \
      logits, ld, (int)T, (int)E, (int)K, idx, wts, tile_rows, b, counter)
  if (slots <= 1)
    MLXR_RF(1);
  else if (slots <= 2)
    MLXR_RF(2);
  else if (slots <= 4)
    MLXR_RF(4);
  else if (slots <= 8)
    MLXR_RF(8);
  else
    MLXR_RF(16);
#undef MLXR_RF
}

hipError_t launch_route(const float* logits, int64_t ld, int64_t T, int64_t E,
                        int64_t K, bool bf16, int32_t* idx, float* wts,
                        int tile_rows, const DispatchBuffers& b,
                        hipStream_t s, int32_t* counter) {
  if (T == 0) return launch_zero_status(b.status, s);
  if (counter && T > MLXR_ROUTE_SMALL_TOKENS && T * K <= kDispatchBlock) {
    ProfileScope prof("router_topk", s);
    if (bf16)
      route_fused_launch<true>(logits, ld, T, E, K, idx, wts, tile_rows, b, counter, s);
    else
      route_fused_launch<false>(logits, ld, T, E, K, idx, wts, tile_rows, b, counter, s);
    return hipGetLastError();
  }
  // one workgroup while the T*K ids fit it and its 16 waves have at most
  // MLXR_ROUTE_SMALL_TOKENS / 16 tokens each; beyond that the top-k spreads
  // over the GPU (a wave per token) before the sort
  if (T > MLXR_ROUTE_SMALL_TOKENS || T * K > kDispatchBlock) {
    hipError_t e =
        launch_router_topk(logits, ld, T, E, K, bf16, idx, wts, b.status, s);
    if (e != hipSuccess) return e;
    return launch_dispatch(idx, T * K, E, tile_rows, b, false, s,
                           MLXR_DISPATCH_FUSED ? counter : nullptr);
  }
  ProfileScope prof("router_topk", s);
  if (bf16)
    route_small_launch<true>(logits, ld, T, E, K, idx, wts, tile_rows, b, s);
  else
    route_small_launch<false>(logits, ld, T, E, K, idx, wts, tile_rows, b, s);
  return hipGetLastError();
}

hipError_t launch_gather_prep(const uint32_t* lhs, const uint32_t* rhs,
                              int64_t B, int64_t M, int64_t x_batch, int64_t E,
                              int64_t N, int32_t* ids, int32_t* xrow,
                              uint16_t* out, int32_t* status, hipStream_t s) {
  const int64_t R = B * M;
  zero_status_kernel<<<1, 1, 0, s>>>(status);
  if (R > 0)
    gather_prep_kernel<<<(unsigned)((R + 255) / 256), 256, 0, s>>>(
        lhs, rhs, B, M, x_batch, E, N, ids, xrow, out, status);
  return hipGetLastError();
}

hipError_t launch_dispatch_identity(int64_t n, int tile_rows,
                                    const DispatchBuffers& b, hipStream_t s) {
  dispatch_identity_kernel<<<1, 256, 0, s>>>((int)n, tile_rows, b);
  return hipGetLastError();
}

}  // namespace mlxr_moe
