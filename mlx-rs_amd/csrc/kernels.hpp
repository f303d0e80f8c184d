// Host-side launchers for the MoE kernels.  Every launcher enqueues on the
// given stream and returns the launch status; none synchronises.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace mlxr_moe {

// ------------------------------------------------------------- profile.cpp
// Brackets one kernel launch with HIP events on its stream when that
// kernel's name is armed (profile_arm); a no-op otherwise.
class ProfileScope {
 public:
  ProfileScope(const char* kernel, hipStream_t s);
  ~ProfileScope();
  ProfileScope(const ProfileScope&) = delete;
  ProfileScope& operator=(const ProfileScope&) = delete;

 private:
  hipEvent_t stop_ = nullptr;
  hipStream_t stream_ = nullptr;
};
// kernel == nullptr or "" disarms.  Re-arming drops unread launches.
int profile_arm(const char* kernel);
// Launch count and elapsed milliseconds (total, min, max) of the armed
// kernel since profile_arm; waits for the last launch; disarms.
int profile_collect(int64_t* launches, double* total_ms, double* min_ms,
                    double* max_ms, std::string* err);

// ---------------------------------------------------------------- quant.hip
hipError_t launch_quantize(const void* w, bool w_bf16, int64_t rows,
                           int64_t cols, int group_size, int bits, uint32_t* wq,
                           void* scales, void* biases, hipStream_t s);
hipError_t launch_dequantize(const uint32_t* wq, const void* scales,
                             const void* biases, bool sb_bf16, int64_t rows,
                             int64_t cols, int group_size, int bits, void* out,
                             bool out_bf16, hipStream_t s);

// --------------------------------------------------------------- router.hip
// Router weights: an f32 Linear [E, d] (bits == 0), a bf16 Linear (bits ==
// 16), or a QuantizedLinear (bits 4 or 8, group 64): packed codes
// [E, d*bits/32], bf16 scales and biases [E, d/64].  The extra row (the shared-expert gate, logit column
// E) takes the same form when w_extra is set.
struct RouterWeights {
  int bits;
  const void* w;
  const uint16_t* scales;
  const uint16_t* biases;
  const void* w_extra;
  const uint16_t* scales_extra;
  const uint16_t* biases_extra;
};
inline RouterWeights router_weights_f32(const float* w, const float* w_extra) {
  return RouterWeights{0, w, nullptr, nullptr, w_extra, nullptr, nullptr};
}
// fast::rms_norm in front of the router: weight w [d] bf16, eps, and the
// normalised rows out [T, d] bf16 (written for the experts that follow).
struct RouterNorm {
  const uint16_t* w;
  float eps;
  uint16_t* out;
};
// logits[t, e] for e < E (+ bias[e] when given, f32 weights only) and
// column E from the extra row.  Quantised weights give bf16 logits (stored
// as their f32 values).  ld = row stride of logits.  With norm, the logits
// of rms_norm(x) (and the normalised rows in norm->out), bit-identical to
// launch_rms_norm followed by this call on its output.  With clear, the
// launch also sets *clear to 0 (the routing counter of launch_route).
hipError_t launch_router_logits(const uint16_t* x, int64_t T, int64_t d,
                                const RouterWeights& w, const float* bias,
                                int64_t E, float* logits, int64_t ld,
                                hipStream_t s, const RouterNorm* norm = nullptr,
                                int32_t* clear = nullptr);
// True when a router's logits of T tokens over d inputs, cols logit columns
// (the experts, plus one for a shared-expert gate), take the matrix-core
// order (router_logits_mfma_kernel; 16-byte aligned x and weights), false
// for the lane order.
bool router_matrix_order(int64_t T, int64_t d, int64_t cols);
// One wave per token; clears *status first when status != nullptr.  bf16:
// the logits are bf16 and the selection is on their bf16 probabilities,
// with bf16 weights (stored as f32).
hipError_t launch_router_topk(const float* logits, int64_t ld, int64_t T,
                              int64_t E, int64_t K, bool bf16, int32_t* idx,
                              float* wts, int32_t* status, hipStream_t s);
// out bf16 [T, d] = fast::rms_norm(x, w, eps) (gemma4's router prologue,
// the decoder layer's post-attention norm)
hipError_t launch_rms_norm(const uint16_t* x, int64_t T, int64_t d,
                           const uint16_t* w, float eps, uint16_t* out,
                           hipStream_t s);
// gemma4's router top-k on bf16 scores [T, ld]: idx [T, K], bf16 weights
// softmax(top-K scores) * per_expert_scale (pes, bf16 [E]).
hipError_t launch_gemma_topk(const float* scores, int64_t ld, int64_t T,
                             int64_t E, int64_t K, const uint16_t* pes,
                             int32_t* idx, uint16_t* wts, hipStream_t s);
hipError_t launch_argsort_rows(const float* a, int64_t rows, int64_t n,
                               uint32_t* out, hipStream_t s);
hipError_t launch_softmax_rows(const float* a, int64_t rows, int64_t n,
                               float* out, hipStream_t s);

// ------------------------------------------------------------- dispatch.hip
// Stable counting sort of ids [n] (values in [0, E)) by expert.
struct DispatchBuffers {
  int32_t* counts;      // [E]
  int32_t* offsets;     // [E + 1]
  int32_t* sorted;      // [n]  flat index per sorted slot
  int32_t* inv;         // [n]  sorted slot per flat index
  int32_t* active;      // [E]  experts with rows, ascending
  int32_t* num_active;  // [1]
  int32_t* work;        // [max_work][kWorkInts] work item records: each
                        // expert's rows in chunks of at most kWorkRows
  int32_t* num_work;    // [1]
  int32_t* work_first;  // [E] first work item of each expert
  int32_t* tiles;       // [max_tiles] packed (expert, first row) of M-tiles
  int32_t* num_tiles;   // [1]
  int32_t* block_hist;  // [ceil(n/1024), E] scratch
  int32_t* rank;        // [n] scratch
  int32_t* status;      // [1] 0 ok, 1 id out of range
};
constexpr int kDispatchBlock = 1024;
constexpr int kMaxExperts = 1024;
// Rows per decode work item: an expert with more rows becomes several items,
// so the decode GEMM's work items stay small and alike.
constexpr int kWorkRows = 8;
// Work item record: expert, first sorted slot, rows (<= kWorkRows), rows of
// the whole expert, then the flat row index (sorted[slot]) of each of the
// item's slots (unset past rows).  A GEMM workgroup learns its task, and
// where its x rows live, from these 48 bytes without a dependent load.
constexpr int kWorkInts = 4 + kWorkRows;
// The streaming decode GEMM runs the items of experts with at most this many
// rows in its 4-token MFMA form, the others in the 8-token form (longer per
// item: the dispatch lists their items first, so the long workgroups start
// in the first wave of the grid rather than making its tail).
#ifndef MLXR_STREAM_TT4_ROWS
#define MLXR_STREAM_TT4_ROWS 4
#endif
constexpr int kStreamTT4Rows = MLXR_STREAM_TT4_ROWS;
int64_t dispatch_max_tiles(int64_t n, int64_t E, int tile_rows);
// Bound on the work items of n flat rows over E experts.
inline int64_t dispatch_max_work(int64_t n, int64_t E) {
  return (E < n ? E : n) + n / kWorkRows;
}
// Clears a workspace status word with a one-thread kernel (no memset node,
// so the call stays valid under stream capture).
hipError_t launch_zero_status(int32_t* status, hipStream_t s);
// Ids equal to -1 are left out silently (rows excluded by the caller);
// other ids outside [0, E) are left out and set *status = 1.  n above 1024
// takes three kernels (rank, scan, scatter).
hipError_t launch_dispatch(const int32_t* ids, int64_t n, int64_t E,
                           int tile_rows, const DispatchBuffers& b,
                           bool reset_status, hipStream_t s, int32_t* counter = nullptr);
// With counter (an int that is 0 when the launch starts), more than 1024 ids
// rank and scan in one launch (the last workgroup to finish scans).
#ifndef MLXR_DISPATCH_FUSED
#define MLXR_DISPATCH_FUSED 1
#endif
// The one-launch routing (route_fused_kernel) for the block forward.
#ifndef MLXR_ROUTE_FUSED
#define MLXR_ROUTE_FUSED 1
#endif
// Top-K + renormalised weights of every token from its logits, then the
// counting sort of the T*K ids, clearing *b.status first.  T <= 16 runs as
// one workgroup; larger T as the top-k kernel plus launch_dispatch, or, with
// counter (an int that is 0 when this launch starts) and T*K <= 1024, as one
// launch whose last workgroup sorts.
hipError_t launch_route(const float* logits, int64_t ld, int64_t T, int64_t E,
                        int64_t K, bool bf16, int32_t* idx, float* wts,
                        int tile_rows, const DispatchBuffers& b,
                        hipStream_t s, int32_t* counter = nullptr);
// gather_qmm helper: per flat row r = b*M + m the expert id and x row.
hipError_t launch_gather_prep(const uint32_t* lhs, const uint32_t* rhs,
                              int64_t B, int64_t M, int64_t x_batch, int64_t E,
                              int64_t N, int32_t* ids, int32_t* xrow,
                              uint16_t* out, int32_t* status, hipStream_t s);
// Identity dispatch for a dense (always-on) expert: one expert, n rows.
hipError_t launch_dispatch_identity(int64_t n, int tile_rows,
                                    const DispatchBuffers& b, hipStream_t s);

// ---------------------------------------------------------------- qgemm.hip
// bits 4/8: packed codes plus scales and biases; bits 16: dense bf16
// weights [E, N, K] (gather_mm), no scales or biases.
struct QWeights {
  const uint32_t* w;       // [E, N, K*bits/32]
  const uint16_t* scales;  // [E, N, K/64] bf16
  const uint16_t* biases;  // [E, N, K/64] bf16
};
struct QGemmArgs {
  const uint16_t* x;       // activations (bf16)
  int64_t x_ld;            // row stride of x in elements
  int64_t x_rows;          // rows of x (the M-tiled kernel's x bounds);
                           // 0: the GEMM's total rows
  // x row of sorted slot p: p when x_by_slot; else, with f the flat row of
  // p (from the work record), row_map[f] when row_map is given, f / row_div
  // otherwise
  const int32_t* row_map;
  int32_t row_div;
  bool x_by_slot;
  const int32_t* offsets;  // [E+1] slot range of each expert
  const int32_t* active;   // [E] experts with rows
  const int32_t* num_active;
  const int32_t* work;     // work item records (kWorkInts each)
  const int32_t* num_work;
  const int32_t* tiles;    // M-tile list (prefill path)
  const int32_t* num_tiles;
  const int32_t* sorted;   // flat row of each sorted slot (prefill path)
  QWeights w0;             // gate (or the only projection)
  QWeights w1;             // up (gated mode only)
  int32_t E, N, K, bits;
  // weight rows per expert: N, or 2N for the packed gate/up tensor of
  // PackedSwitchFfn ([E, 2H, D]; w1 then points H rows past w0)
  int32_t e_rows;
  int32_t act;             // gated mode: kActSwiglu or kActGeglu
  uint16_t* out;           // bf16
  int64_t out_ld;
  bool out_by_flat;        // out row of slot p = its flat row (else p)
  bool gated;              // out = act(x.w0, x.w1)
};
constexpr int32_t kActSwiglu = 0;  // silu(g) * u  (Qwen3.5/3.6 experts)
constexpr int32_t kActGeglu = 1;   // gelu_approx(g) * u  (gemma4 experts)
// Largest input dim (K) of a projection: 8 waves x 8 groups of 64.
constexpr int kMaxInputDims = 4096;
// Prefill kernel M-tiles: 256 rows when the experts average at least
// MLXR_PREFILL_TALL_ROWS rows, 128 from MLXR_PREFILL_SHORT_ROWS (and always
// for 8-bit weights), else 64 (prefill_tile_rows).  The dispatch cuts its M-tile list with the same
// choice; tile lists are sized for the shortest tiles.
#ifndef MLXR_PREFILL_TALL_ROWS
#define MLXR_PREFILL_TALL_ROWS 192
#endif
#ifndef MLXR_PREFILL_SHORT_ROWS
#define MLXR_PREFILL_SHORT_ROWS 64
#endif
// 1: the prefill GEMM keeps each tile's scales and biases in LDS (where they
// fit) instead of loading them every K step
#ifndef MLXR_PREFILL_SCALES_LDS
#define MLXR_PREFILL_SCALES_LDS 1
#endif
constexpr int kPrefillMinTileRows = 64;
int prefill_tile_rows(int64_t rows, int64_t experts, int bits = 4);
// max_items bounds the number of work items (dispatch_max_work); prefill
// selects the M-tiled kernel (prefill.hip) where it applies.  Dense bf16
// weights (bits 16) take the split-K decode kernel or the M-tiled one.
// `profile` names the launch for ProfileScope (default "qgemm_gated" or
// "qgemm_down"; the shared expert's GEMMs are "shared_gated" /
// "shared_down").  `shared` folds a second problem into the same launch:
// the block's shared expert, whose shared_rows rows are the tokens in order
// (its work items or M-tiles are made in the kernel, no dispatch); it must
// have a's N, K, bits and mode.  (On the prefill path its tiles have the
// routed problem's height: each output's sum runs in the same order at any
// height.)
hipError_t launch_qgemm(const QGemmArgs& a, int64_t total_rows,
                        int64_t max_items, bool prefill, hipStream_t s,
                        const char* profile = nullptr,
                        const QGemmArgs* shared = nullptr,
                        int64_t shared_rows = 0);

// The combine of a single token folded into its down GEMM
// (launch_qgemm_down_combine): the routing weights [K] (f32, or bf16 with
// w_bf16), the shared expert's row [d] when it ran apart (a folded one
// comes from the same launch), its gate logit (null: no shared branch), the
// residual row [d] or null, and the output row [d] (bf16 when bf16, else
// f32) -- the arguments of launch_combine at T = 1.  `distinct`: the K ids
// name K different experts (the block's own top-K), so every work item holds
// one row; otherwise (caller indices) an expert may take several rows and
// its item then runs in the 8-token form, as in the separate down launch.
struct DownCombine {
  const void* w;
  bool w_bf16;
  const uint16_t* shared_y;
  const float* shared_logit;
  const uint16_t* residual;
  void* out;
  bool bf16;
  bool distinct;
};

// The down GEMM of ONE token (K routed rows, and the folded shared
// expert's row when `shared` is given) with the combine in the same launch:
// one workgroup per 16 output channels runs every row's item (the streaming
// kernel's per-item work, the same K-slices, so each y value is the one the
// separate down launch writes), keeps the bf16 rows in LDS and sums them in
// k order.  Sets *done = false, launching nothing, where the streaming
// kernel would not run the down launch or the rows do not fit one
// workgroup; the caller then launches the down GEMM and the combine.
hipError_t launch_qgemm_down_combine(const QGemmArgs& a, int64_t K, int64_t max_items,
                                     const QGemmArgs* shared, const DownCombine& c,
                                     hipStream_t s, bool* done);

// ---------------------------------------------------------------- prefill.hip
// x_rows bounds the rows of x the GEMM reads; tile_rows is the M-tile height
// the dispatch used (prefill_tile_rows); max_tiles bounds the M-tile list
// (dispatch_max_tiles).  shared (optional): a second problem of the same
// projection shape and format with shared_rows rows by slot (the block's
// shared expert), its M-tiles in the same launch.
bool prefill_supported(const QGemmArgs& a, int64_t x_rows);
hipError_t launch_qgemm_prefill(const QGemmArgs& a, int64_t x_rows,
                                int tile_rows, int64_t max_tiles,
                                hipStream_t s, const char* profile,
                                const QGemmArgs* shared = nullptr,
                                int64_t shared_rows = 0);

// -------------------------------------------------------------- combine.hip
// out f32 [T, d], or bf16 when bf16 (the routing weights are then bf16
// values and every op rounds to bf16).  w is f32 [T, K], or bf16 when
// w_bf16 (only with a bf16 out).  residual (bf16 [T, d], optional) is added
// last: out = residual + the combine's result in its own dtype.
hipError_t launch_combine(const uint16_t* y, const void* w, bool w_bf16,
                          int64_t T, int64_t K, int64_t d,
                          const uint16_t* shared_y, const float* shared_logit,
                          int64_t shared_ld, const uint16_t* residual,
                          void* out, bool bf16, hipStream_t s);

// ---------------------------------------------------------------- probe.hip
// One plain streaming read of bytes (a multiple of 16) from buf, timed as
// the profile kernel "read_probe"; sink: one device word it may write.
hipError_t launch_read_probe(const void* buf, size_t bytes, uint32_t* sink, hipStream_t s);

}  // namespace mlxr_moe
