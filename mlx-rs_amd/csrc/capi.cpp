// C ABI of the MI355X sparse-MoE block (declarations and reference
// citations in include/mlxr_moe.h).  Each entry point validates every
// host-visible argument, then enqueues kernels on the caller's stream.
// Errors never cross the ABI as exceptions: they return -1 and leave a
// thread-local message.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "../../include/mlxr_moe.h"
#include "kernels.hpp"
#include "nn.hpp"

using namespace mlxr_moe;

namespace {

thread_local std::string g_last_error;

int fail(const std::string& msg) {
  g_last_error = msg;
  return -1;
}

int finish(const Status& st) { return st.ok ? 0 : fail(st.what); }

}  // namespace

// The thread-local error of the C ABI, for entry points in other sources.
int mlxr_moe::capi_fail(const std::string& msg) { return fail(msg); }

namespace {

hipStream_t as_stream(mlxr_moe_stream s) {
  return reinterpret_cast<hipStream_t>(s);
}

bool dtype_ok(int dt) { return dt == MLXR_MOE_FLOAT32 || dt == MLXR_MOE_BFLOAT16; }

// mode, group_size and bits as mlx-c resolves them (defaults from
// crates/mlxr/src/ops/quantization.rs:11-13).
Status resolve_quant(const char* mode, mlxr_moe_optional_int gs,
                     mlxr_moe_optional_int bits, bool kernel_path, int* g_out,
                     int* b_out) {
  if (mode && std::strcmp(mode, "affine") != 0)
    return Status::error(std::string("unsupported quantization mode '") +
                         mode + "' (only 'affine')");
  const int g = gs.has_value ? gs.value : 64;
  const int b = bits.has_value ? bits.value : 4;
  if (kernel_path) {
    if (g != 64)
      return Status::error("group_size must be 64, got " + std::to_string(g));
    if (b != 4 && b != 8)
      return Status::error("bits must be 4 or 8, got " + std::to_string(b));
  } else {
    if (g != 32 && g != 64 && g != 128)
      return Status::error("group_size must be 32, 64 or 128, got " +
                           std::to_string(g));
    if (b != 2 && b != 4 && b != 8)
      return Status::error("bits must be 2, 4 or 8, got " + std::to_string(b));
  }
  *g_out = g;
  *b_out = b;
  return Status{};
}

bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

Status check_workspace(const Carve& plan, void* ws, size_t ws_size) {
  if (plan.off > ws_size)
    return Status::error("workspace too small: need " +
                         std::to_string(plan.off) + " bytes, got " +
                         std::to_string(ws_size));
  if (plan.off && !ws) return Status::error("workspace is NULL");
  if (ws && !aligned(ws, 256))
    return Status::error("workspace must be 256-byte aligned");
  return Status{};
}

// Workspace plans (the same carving the entry points run).
void plan_gather(Carve& c, int64_t B, int64_t M, int64_t E) {
  const int64_t R = B * M;
  c.take<int32_t>(1);  // status
  c.take<int32_t>(R);  // ids
  c.take<int32_t>(R);  // xrow
  carve_dispatch(c, R, E, nullptr);
}

// gather_qmm and gather_mm after their own checks: the grouped GEMM over
// the dispatch of the B*M rows (bits 16: dense bf16 weights).
int run_gather(const char* op, const void* x, int64_t x_batch, int64_t M,
               int64_t K, const uint32_t* w, const void* scales,
               const void* biases, int bits, int64_t E, int64_t N,
               const uint32_t* lhs_indices, const uint32_t* rhs_indices,
               int64_t B, void* out, void* workspace, size_t workspace_size,
               hipStream_t s) {
  const std::string o(op);
  if (!rhs_indices && B > 0) return fail(o + ": rhs_indices are required");
  if (E <= 0 || E > kMaxExperts)
    return fail(o + ": num_experts must be in [1, " +
                std::to_string(kMaxExperts) + "]");
  if (M <= 0 || K <= 0 || N <= 0 || B < 0 || x_batch <= 0)
    return fail(o + ": bad shape");
  if (K % 64 || N % 64)
    return fail(o + ": K and N must be multiples of 64");
  if (K > kMaxInputDims)
    return fail(o + ": K above " + std::to_string(kMaxInputDims) +
                " is not supported");
  if (!lhs_indices && B % x_batch)
    return fail(o + ": x batch " + std::to_string(x_batch) +
                " does not broadcast against " + std::to_string(B) +
                " indices");
  if (B * M > INT32_MAX / 2) return fail(o + ": too many rows");
  if (bits == 16 && x_batch * M * K * 2 >= ((int64_t)1 << 31))
    return fail(o + ": x must be under 2 GB");  // the M-tiled kernel's buffer
  if (N * K * bits / 8 >= ((int64_t)1 << 31))
    return fail(o + ": one expert's weights must be under 2 GB");
  if (B > 0 && (!x || !w || !out)) return fail(o + ": null array");
  if (!aligned(x, 16) || !aligned(w, 16))
    return fail(o + ": x and w must be 16-byte aligned");
  Carve plan(nullptr);
  plan_gather(plan, B, M, E);
  Status st = check_workspace(plan, workspace, workspace_size);
  if (!st.ok) return finish(st);
  if (B == 0) return 0;

  const int64_t R = B * M;
  Carve c(workspace);
  int32_t* status = c.take<int32_t>(1);
  int32_t* ids = c.take<int32_t>(R);
  int32_t* xrow = c.take<int32_t>(R);
  const DispatchBuffers db = carve_dispatch(c, R, E, status);
  uint16_t* ob = static_cast<uint16_t*>(out);
  st = from_hip(launch_gather_prep(lhs_indices, rhs_indices, B, M, x_batch, E,
                                   N, ids, xrow, ob, status, s),
                (o + " prep").c_str());
  if (st.ok)
    st = from_hip(launch_dispatch(ids, R, E, prefill_tile_rows(R, E, bits), db, false, s),
                  (o + " dispatch").c_str());
  if (!st.ok) return finish(st);
  QGemmArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_ld = K;
  a.x_rows = x_batch * M;
  a.row_map = xrow;
  a.row_div = 1;
  a.x_by_slot = false;
  a.offsets = db.offsets;
  a.active = db.active;
  a.num_active = db.num_active;
  a.work = db.work;
  a.num_work = db.num_work;
  a.tiles = db.tiles;
  a.num_tiles = db.num_tiles;
  a.sorted = db.sorted;
  a.w0 = QWeights{w, static_cast<const uint16_t*>(scales),
                  static_cast<const uint16_t*>(biases)};
  a.E = (int32_t)E;
  a.N = (int32_t)N;
  a.e_rows = (int32_t)N;
  a.act = kActSwiglu;
  a.K = (int32_t)K;
  a.bits = bits;
  a.out = ob;
  a.out_ld = N;
  a.out_by_flat = true;
  a.gated = false;
  return finish(from_hip(launch_qgemm(a, R, dispatch_max_work(R, E),
                                      nn::use_prefill_path(R, E, bits), s),
                         op));
}

}  // namespace

extern "C" {

const char* mlxr_moe_last_error(void) { return g_last_error.c_str(); }

int mlxr_moe_version(void) { return 301; }

int mlxr_moe_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols,
                      mlxr_moe_optional_int group_size,
                      mlxr_moe_optional_int bits, const char* mode,
                      uint32_t* wq, void* scales, void* biases,
                      mlxr_moe_stream stream) {
  int g, b;
  Status st = resolve_quant(mode, group_size, bits, false, &g, &b);
  if (!st.ok) return finish(st);
  if (!dtype_ok(w_dtype)) return fail("quantize: w dtype must be f32 or bf16");
  if (rows < 0 || cols <= 0) return fail("quantize: bad shape");
  if (cols % g)
    return fail("quantize: last dim " + std::to_string(cols) +
                " is not a multiple of group_size " + std::to_string(g));
  if (rows && (!w || !wq || !scales || !biases))
    return fail("quantize: null array");
  return finish(from_hip(launch_quantize(w, w_dtype == MLXR_MOE_BFLOAT16, rows,
                                         cols, g, b, wq, scales, biases,
                                         as_stream(stream)),
                         "quantize"));
}

int mlxr_moe_dequantize(const uint32_t* wq, const void* scales,
                        const void* biases, int sb_dtype, int64_t rows,
                        int64_t cols, mlxr_moe_optional_int group_size,
                        mlxr_moe_optional_int bits, const char* mode,
                        void* out, int out_dtype, mlxr_moe_stream stream) {
  int g, b;
  Status st = resolve_quant(mode, group_size, bits, false, &g, &b);
  if (!st.ok) return finish(st);
  if (!dtype_ok(sb_dtype) || !dtype_ok(out_dtype))
    return fail("dequantize: dtypes must be f32 or bf16");
  if (rows < 0 || cols <= 0 || cols % g) return fail("dequantize: bad shape");
  if (!biases) return fail("dequantize: biases are required for affine mode");
  if (rows && (!wq || !scales || !out)) return fail("dequantize: null array");
  return finish(from_hip(
      launch_dequantize(wq, scales, biases, sb_dtype == MLXR_MOE_BFLOAT16, rows,
                        cols, g, b, out, out_dtype == MLXR_MOE_BFLOAT16,
                        as_stream(stream)),
      "dequantize"));
}

size_t mlxr_moe_gather_qmm_workspace_size(int64_t B, int64_t M,
                                          int64_t num_experts) {
  Carve c(nullptr);
  plan_gather(c, B, M, num_experts);
  return c.off;
}

int mlxr_moe_gather_qmm(const void* x, int x_dtype, int64_t x_batch,
                        int64_t M, int64_t K, const uint32_t* w,
                        const void* scales, const void* biases, int sb_dtype,
                        int64_t E, int64_t N, const uint32_t* lhs_indices,
                        const uint32_t* rhs_indices, int64_t B, int transpose,
                        mlxr_moe_optional_int group_size,
                        mlxr_moe_optional_int bits, const char* mode,
                        int sorted_indices, void* out, int out_dtype,
                        void* workspace, size_t workspace_size,
                        mlxr_moe_stream stream) {
  (void)sorted_indices;
  int g, b;
  Status st = resolve_quant(mode, group_size, bits, true, &g, &b);
  if (!st.ok) return finish(st);
  if (!transpose)
    return fail("gather_qmm: only transpose=true (the [E, N, K] layout of "
                "QuantizedSwitchLinear) is supported");
  if (x_dtype != MLXR_MOE_BFLOAT16 || sb_dtype != MLXR_MOE_BFLOAT16 ||
      out_dtype != MLXR_MOE_BFLOAT16)
    return fail("gather_qmm: x, scales/biases and out must be bf16");
  if (!biases) return fail("gather_qmm: biases are required for affine mode");
  if (!scales) return fail("gather_qmm: null array");
  return run_gather("gather_qmm", x, x_batch, M, K, w, scales, biases, b, E, N,
                    lhs_indices, rhs_indices, B, out, workspace,
                    workspace_size, as_stream(stream));
}

size_t mlxr_moe_gather_mm_workspace_size(int64_t B, int64_t M,
                                         int64_t num_experts) {
  return mlxr_moe_gather_qmm_workspace_size(B, M, num_experts);
}

int mlxr_moe_gather_mm(const void* a, int a_dtype, int64_t a_batch, int64_t M,
                       int64_t K, const void* b, int b_dtype, int64_t E,
                       int64_t N, int b_transposed,
                       const uint32_t* lhs_indices,
                       const uint32_t* rhs_indices, int64_t B,
                       int sorted_indices, void* out, int out_dtype,
                       void* workspace, size_t workspace_size,
                       mlxr_moe_stream stream) {
  (void)sorted_indices;
  if (!b_transposed)
    return fail("gather_mm: only b_transposed=1 (b stored [E, N, K], the "
                "swap_axes view of SwitchLinear's weight) is supported");
  if (a_dtype != MLXR_MOE_BFLOAT16 || b_dtype != MLXR_MOE_BFLOAT16 ||
      out_dtype != MLXR_MOE_BFLOAT16)
    return fail("gather_mm: a, b and out must be bf16");
  return run_gather("gather_mm", a, a_batch, M, K,
                    static_cast<const uint32_t*>(b), nullptr, nullptr, 16, E,
                    N, lhs_indices, rhs_indices, B, out, workspace,
                    workspace_size, as_stream(stream));
}

int mlxr_moe_router_matrix_order(int64_t T, int64_t d, int64_t columns) {
  if (T < 0 || d < 0 || columns < 0) return -1;
  return router_matrix_order(T, d, columns) ? 1 : 0;
}

int mlxr_moe_gather_qmm_tiled(int64_t rows, int64_t num_experts) {
  if (rows < 0 || num_experts < 0) return -1;
  return nn::use_prefill_path(rows, num_experts) ? 1 : 0;
}

int mlxr_moe_argpartition(const float* a, int64_t rows, int64_t n, int kth,
                          int axis, uint32_t* out, mlxr_moe_stream stream) {
  if (axis != -1 && axis != 1)
    return fail("argpartition: axis " + std::to_string(axis) +
                " is out of bounds for a 2-d array [rows, n] (use -1 or 1)");
  if (rows < 0 || n <= 0) return fail("argpartition: bad shape");
  if (kth < -n || kth >= n)
    return fail("argpartition: kth " + std::to_string(kth) +
                " is out of bounds for axis of size " + std::to_string(n));
  if (n > 4096) return fail("argpartition: rows longer than 4096");
  if (rows && (!a || !out)) return fail("argpartition: null array");
  return finish(from_hip(launch_argsort_rows(a, rows, n, out,
                                             as_stream(stream)),
                         "argpartition"));
}

int mlxr_moe_softmax(const float* a, int64_t rows, int64_t n, int axis,
                     int precise, float* out, mlxr_moe_stream stream) {
  (void)precise;
  if (axis != -1 && axis != 1)
    return fail("softmax: axis " + std::to_string(axis) +
                " is out of bounds for a 2-d array");
  if (rows < 0 || n <= 0) return fail("softmax: bad shape");
  if (rows && (!a || !out)) return fail("softmax: null array");
  return finish(from_hip(launch_softmax_rows(a, rows, n, out,
                                             as_stream(stream)),
                         "softmax"));
}

size_t mlxr_moe_router_workspace_size(int64_t T, int64_t E) {
  Carve c(nullptr);
  c.take<float>(T * E);
  return c.off;
}

int mlxr_moe_router_topk(const void* x, int64_t T, int64_t d,
                         const float* gate_w, int64_t E, int64_t K,
                         int32_t* topk_idx, float* topk_w, void* workspace,
                         size_t workspace_size, mlxr_moe_stream stream) {
  if (T < 0 || d <= 0 || E <= 0) return fail("router_topk: bad shape");
  if (d % 4) return fail("router_topk: hidden size must be a multiple of 4");
  if (E > kMaxExperts)
    return fail("router_topk: at most " + std::to_string(kMaxExperts) +
                " experts");
  if (K < 1 || K > E || K > 64)
    return fail("router_topk: k must be in [1, min(E, 64)], got " +
                std::to_string(K));
  if (T && (!x || !gate_w || !topk_idx || !topk_w))
    return fail("router_topk: null array");
  if (!aligned(gate_w, 16) || !aligned(x, 8))
    return fail("router_topk: gate_w must be 16-byte and x 8-byte aligned");
  Carve plan(nullptr);
  plan.take<float>(T * E);
  Status st = check_workspace(plan, workspace, workspace_size);
  if (!st.ok) return finish(st);
  Carve c(workspace);
  float* logits = c.take<float>(T * E);
  hipStream_t s = as_stream(stream);
  st = from_hip(launch_router_logits(static_cast<const uint16_t*>(x), T, d,
                                     router_weights_f32(gate_w, nullptr),
                                     nullptr, E, logits, E, s),
                "router logits");
  if (st.ok)
    st = from_hip(launch_router_topk(logits, E, T, E, K, false, topk_idx,
                                     topk_w, nullptr, s),
                  "router top-k");
  return finish(st);
}

int mlxr_moe_router_topk_quantized(const void* x, int64_t T,
                                   const mlxr_moe_qlinear* gate, int64_t K,
                                   int32_t* topk_idx, float* topk_w,
                                   void* workspace, size_t workspace_size,
                                   mlxr_moe_stream stream) {
  if (!gate) return fail("router_topk_quantized: null gate");
  const int64_t E = gate->output_dims, d = gate->input_dims;
  if (T < 0 || d <= 0 || E <= 0 || gate->num_experts != 1)
    return fail("router_topk_quantized: bad shape (gate must be one "
                "[E, d] QuantizedLinear)");
  const bool dense = gate->bits == 16;  // a bf16 Linear
  if (!dense && ((gate->bits != 4 && gate->bits != 8) || gate->group_size != 64))
    return fail("router_topk_quantized: bits must be 4 or 8 with group size "
                "64, or 16 (a bf16 Linear)");
  if (d % 64) return fail("router_topk_quantized: d must be a multiple of 64");
  if (E > kMaxExperts)
    return fail("router_topk_quantized: at most " +
                std::to_string(kMaxExperts) + " experts");
  if (K < 1 || K > E || K > 64)
    return fail("router_topk_quantized: k must be in [1, min(E, 64)], got " +
                std::to_string(K));
  if (dense && (gate->scales || gate->biases))
    return fail("router_topk_quantized: a bf16 Linear gate takes no scales "
                "or biases");
  if (!gate->weight || (!dense && (!gate->scales || !gate->biases)) ||
      (T && (!x || !topk_idx || !topk_w)))
    return fail("router_topk_quantized: null array");
  if (!aligned(x, 8) || !aligned(gate->weight, dense ? 8 : 4) ||
      !aligned(gate->scales, 2) || !aligned(gate->biases, 2))
    return fail("router_topk_quantized: x must be 8-byte and the weights "
                "4-byte (bf16: 8-byte) aligned");
  Carve plan(nullptr);
  plan.take<float>(T * E);
  Status st = check_workspace(plan, workspace, workspace_size);
  if (!st.ok) return finish(st);
  Carve c(workspace);
  float* logits = c.take<float>(T * E);
  hipStream_t s = as_stream(stream);
  const RouterWeights rw{gate->bits,
                         gate->weight,
                         static_cast<const uint16_t*>(gate->scales),
                         static_cast<const uint16_t*>(gate->biases),
                         nullptr,
                         nullptr,
                         nullptr};
  st = from_hip(launch_router_logits(static_cast<const uint16_t*>(x), T, d, rw,
                                     nullptr, E, logits, E, s),
                "router logits");
  if (st.ok)
    st = from_hip(launch_router_topk(logits, E, T, E, K, true, topk_idx,
                                     topk_w, nullptr, s),
                  "router top-k");
  return finish(st);
}

size_t mlxr_moe_dispatch_workspace_size(int64_t n, int64_t E) {
  Carve c(nullptr);
  c.take<int32_t>(1);
  carve_dispatch(c, n, E, nullptr);
  return c.off;
}

int mlxr_moe_dispatch(const int32_t* ids, int64_t n, int64_t E,
                      int32_t* counts, int32_t* offsets, int32_t* sorted,
                      int32_t* inv, void* workspace, size_t workspace_size,
                      mlxr_moe_stream stream) {
  if (n < 0 || E <= 0 || E > kMaxExperts) return fail("dispatch: bad shape");
  if (n > INT32_MAX / 2) return fail("dispatch: too many ids");
  if (!counts || !offsets || (n && (!ids || !sorted || !inv)))
    return fail("dispatch: null array");
  Carve plan(nullptr);
  plan.take<int32_t>(1);
  carve_dispatch(plan, n, E, nullptr);
  Status st = check_workspace(plan, workspace, workspace_size);
  if (!st.ok) return finish(st);
  Carve c(workspace);
  int32_t* status = c.take<int32_t>(1);
  DispatchBuffers db = carve_dispatch(c, n, E, status);
  db.counts = counts;
  db.offsets = offsets;
  db.sorted = sorted;
  db.inv = inv;
  return finish(from_hip(launch_dispatch(ids, n, E, prefill_tile_rows(n, E), db, true,
                                         as_stream(stream)),
                         "dispatch"));
}

int mlxr_moe_combine(const void* y, const float* w, int64_t T, int64_t K,
                     int64_t d, const void* shared_y,
                     const float* shared_logit, float* out,
                     mlxr_moe_stream stream) {
  if (T < 0 || K < 1 || d <= 0) return fail("combine: bad shape");
  if (d % 8) return fail("combine: d must be a multiple of 8");
  if (T && (!y || !w || !out)) return fail("combine: null array");
  if ((shared_y == nullptr) != (shared_logit == nullptr))
    return fail("combine: shared_y and shared_logit go together");
  if (!aligned(y, 16) || !aligned(out, 16) ||
      (shared_y && !aligned(shared_y, 16)))
    return fail("combine: y, shared_y and out must be 16-byte aligned");
  return finish(from_hip(
      launch_combine(static_cast<const uint16_t*>(y), w, false, T, K, d,
                     static_cast<const uint16_t*>(shared_y), shared_logit, 1,
                     nullptr, out, false, as_stream(stream)),
      "combine"));
}

int mlxr_moe_rms_norm(const void* x, int64_t T, int64_t d, const void* weight,
                      float eps, void* out, mlxr_moe_stream stream) {
  if (T < 0 || d <= 0) return fail("rms_norm: bad shape");
  if (d % 4) return fail("rms_norm: d must be a multiple of 4");
  if (!(eps >= 0.0f)) return fail("rms_norm: eps must be >= 0");
  if (T && (!x || !weight || !out)) return fail("rms_norm: null array");
  if (!aligned(x, 8) || !aligned(out, 8))
    return fail("rms_norm: x and out must be 8-byte aligned");
  return finish(from_hip(
      launch_rms_norm(static_cast<const uint16_t*>(x), T, d,
                      static_cast<const uint16_t*>(weight), eps,
                      static_cast<uint16_t*>(out), as_stream(stream)),
      "rms_norm"));
}

size_t mlxr_moe_switch_glu_workspace_size(const mlxr_moe_switch_glu* ffn,
                                          int64_t T, int64_t K) {
  if (!ffn) return 0;
  Carve c(nullptr);
  c.take<int32_t>(1);
  nn::SplitSwitchFfn::plan(c, T, K, ffn->gate_proj.input_dims,
                           ffn->gate_proj.output_dims,
                           ffn->gate_proj.num_experts);
  return c.off;
}

int mlxr_moe_switch_glu_forward(const mlxr_moe_switch_glu* ffn, const void* x,
                                int64_t T, const int32_t* indices,
                                const float* weights, int64_t K, float* out,
                                void* workspace, size_t workspace_size,
                                mlxr_moe_stream stream) {
  if (!ffn) return fail("switch_glu: null module");
  const int64_t d = ffn->gate_proj.input_dims, f = ffn->gate_proj.output_dims;
  const int64_t E = ffn->gate_proj.num_experts;
  nn::SplitSwitchFfn m(*ffn);
  Status st = m.validate(d, f, E);
  if (!st.ok) return finish(st);
  if (T < 0 || K < 1 || K > E) return fail("switch_glu: bad T or K");
  if (T && (!x || !indices || !weights || !out))
    return fail("switch_glu: null array");
  if (!aligned(x, 16) || !aligned(out, 16))
    return fail("switch_glu: x and out must be 16-byte aligned");
  Carve plan(nullptr);
  plan.take<int32_t>(1);
  nn::SplitSwitchFfn::plan(plan, T, K, d, f, E);
  st = check_workspace(plan, workspace, workspace_size);
  if (!st.ok) return finish(st);
  if (T == 0) return 0;
  hipStream_t s = as_stream(stream);
  Carve c(workspace);
  int32_t* status = c.take<int32_t>(1);
  st = m.forward_with_combine(static_cast<const uint16_t*>(x), T, indices,
                                weights, false, K, out, nullptr, nullptr, 0,
                                c, status, s);
  return finish(st);
}

int mlxr_moe_switch_glu_experts(const mlxr_moe_switch_glu* ffn, const void* x,
                                int64_t T, const int32_t* indices, int64_t K,
                                void* y, void* workspace,
                                size_t workspace_size, mlxr_moe_stream stream) {
  if (!ffn) return fail("switch_glu: null module");
  const int64_t d = ffn->gate_proj.input_dims, f = ffn->gate_proj.output_dims;
  const int64_t E = ffn->gate_proj.num_experts;
  nn::SplitSwitchFfn m(*ffn);
  Status st = m.validate(d, f, E);
  if (!st.ok) return finish(st);
  if (T < 0 || K < 1 || K > E) return fail("switch_glu: bad T or K");
  if (T && (!x || !indices || !y)) return fail("switch_glu: null array");
  if (!aligned(x, 16)) return fail("switch_glu: x must be 16-byte aligned");
  Carve plan(nullptr);
  plan.take<int32_t>(1);
  nn::SplitSwitchFfn::plan(plan, T, K, d, f, E);
  st = check_workspace(plan, workspace, workspace_size);
  if (!st.ok) return finish(st);
  if (T == 0) return 0;
  hipStream_t s = as_stream(stream);
  Carve c(workspace);
  int32_t* status = c.take<int32_t>(1);
  c.take<uint16_t>(T * K * d);  // the combine's y slot, unused here
  st = m.forward(static_cast<const uint16_t*>(x), T, indices, K,
                   static_cast<uint16_t*>(y), c, status, s);
  return finish(st);
}

namespace {

void gemma_router_plan(Carve& c, const mlxr_moe_gemma_router& r, int64_t T) {
  c.take<uint16_t>(T * r.hidden_size);  // normed x
  c.take<float>(T * r.num_experts);     // scores
}

}  // namespace

size_t mlxr_moe_gemma_router_workspace_size(const mlxr_moe_gemma_router* r,
                                            int64_t T) {
  if (!r) return 0;
  Carve c(nullptr);
  gemma_router_plan(c, *r, T);
  return c.off;
}

int mlxr_moe_gemma_router_forward(const mlxr_moe_gemma_router* r,
                                  const void* x, int64_t T, int32_t* topk_idx,
                                  void* topk_w, void* workspace,
                                  size_t workspace_size,
                                  mlxr_moe_stream stream) {
  if (!r) return fail("gemma_router: null module");
  const int64_t d = r->hidden_size, E = r->num_experts, K = r->top_k;
  const bool q = r->proj_q.weight != nullptr;
  if (T < 0 || d <= 0 || E <= 0) return fail("gemma_router: bad shape");
  if (d % (q ? 64 : 4))
    return fail(std::string("gemma_router: hidden_size must be a multiple of ") +
                (q ? "64" : "4"));
  if (E > kMaxExperts)
    return fail("gemma_router: at most " + std::to_string(kMaxExperts) +
                " experts");
  if (K < 1 || K > E || K > 64)
    return fail("gemma_router: top_k must be in [1, min(num_experts, 64)], got " +
                std::to_string(K));
  if (!(r->eps >= 0.0f)) return fail("gemma_router: eps must be >= 0");
  if (q == (r->proj_weight != nullptr))
    return fail("gemma_router: give exactly one of proj_weight and proj_q");
  if (q) {
    const mlxr_moe_qlinear& p = r->proj_q;
    if ((p.bits != 4 && p.bits != 8) || p.group_size != 64)
      return fail("gemma_router: proj_q must be 4- or 8-bit with group size 64");
    if (p.num_experts != 1 || p.output_dims != E || p.input_dims != d ||
        !p.scales || !p.biases)
      return fail("gemma_router: proj_q must be one [num_experts, "
                  "hidden_size] QuantizedLinear with scales and biases");
    if (!aligned(p.weight, 4) || !aligned(p.scales, 2) || !aligned(p.biases, 2))
      return fail("gemma_router: proj_q arrays misaligned");
  } else if (!aligned(r->proj_weight, 8)) {
    return fail("gemma_router: proj_weight must be 8-byte aligned");
  }
  if (!r->norm_weight || !r->per_expert_scale ||
      (T && (!x || !topk_idx || !topk_w)))
    return fail("gemma_router: null array");
  if (!aligned(x, 8) || !aligned(r->norm_weight, 2) ||
      !aligned(r->per_expert_scale, 2) || !aligned(topk_w, 2))
    return fail("gemma_router: x must be 8-byte aligned");
  Carve plan(nullptr);
  gemma_router_plan(plan, *r, T);
  Status st = check_workspace(plan, workspace, workspace_size);
  if (!st.ok) return finish(st);
  if (T == 0) return 0;
  Carve c(workspace);
  uint16_t* normed = c.take<uint16_t>(T * d);
  float* scores = c.take<float>(T * E);
  hipStream_t s = as_stream(stream);
  const RouterWeights rw =
      q ? RouterWeights{r->proj_q.bits,
                        r->proj_q.weight,
                        static_cast<const uint16_t*>(r->proj_q.scales),
                        static_cast<const uint16_t*>(r->proj_q.biases),
                        nullptr,
                        nullptr,
                        nullptr}
        : RouterWeights{16, r->proj_weight, nullptr, nullptr, nullptr, nullptr, nullptr};
  // RMSNorm folded into the score kernel (the normalised rows land in
  // `normed`)
  const RouterNorm nm{static_cast<const uint16_t*>(r->norm_weight), r->eps, normed};
  st = from_hip(launch_router_logits(static_cast<const uint16_t*>(x), T, d, rw,
                                     nullptr, E, scores, E, s, &nm),
                "gemma_router scores");
  if (st.ok)
    st = from_hip(launch_gemma_topk(scores, E, T, E, K,
                                    static_cast<const uint16_t*>(r->per_expert_scale),
                                    topk_idx, static_cast<uint16_t*>(topk_w), s),
                  "gemma_router top-k");
  return finish(st);
}

size_t mlxr_moe_packed_switch_glu_workspace_size(
    const mlxr_moe_packed_switch_glu* ffn, int64_t T, int64_t K) {
  if (!ffn) return 0;
  Carve c(nullptr);
  c.take<int32_t>(1);
  const mlxr_moe_qlinear& gu = ffn->gate_up_proj;
  nn::SwitchFfn::plan(c, T, K, gu.input_dims, gu.output_dims / 2,
                      gu.num_experts);
  return c.off;
}

namespace {

// Shared checks and set-up of the two PackedSwitchFfn entry points.
Status packed_prologue(const mlxr_moe_packed_switch_glu* ffn, const void* x,
                       int64_t T, const int32_t* indices, int64_t K,
                       const void* out, void* workspace, size_t workspace_size,
                       nn::PackedSwitchFfn& m) {
  Status st = m.validate();
  if (!st.ok) return st;
  const nn::SwitchWeights& w = m.weights();
  if (T < 0 || K < 1 || K > w.E)
    return Status::error("packed_switch_glu: bad T or K");
  if (T && (!x || !indices || !out))
    return Status::error("packed_switch_glu: null array");
  if (!aligned(x, 16) || !aligned(out, 16))
    return Status::error("packed_switch_glu: x and out must be 16-byte aligned");
  Carve plan(nullptr);
  plan.take<int32_t>(1);
  nn::SwitchFfn::plan(plan, T, K, w.d, w.f, w.E);
  return check_workspace(plan, workspace, workspace_size);
}

}  // namespace

int mlxr_moe_packed_switch_glu_forward(const mlxr_moe_packed_switch_glu* ffn,
                                       const void* x, int64_t T,
                                       const int32_t* indices,
                                       const void* weights, int weights_dtype,
                                       int64_t K, void* out, void* workspace,
                                       size_t workspace_size,
                                       mlxr_moe_stream stream) {
  if (!ffn) return fail("packed_switch_glu: null module");
  if (weights_dtype != MLXR_MOE_FLOAT32 && weights_dtype != MLXR_MOE_BFLOAT16)
    return fail("packed_switch_glu: weights must be f32 or bf16");
  nn::PackedSwitchFfn m(*ffn);
  Status st = packed_prologue(ffn, x, T, indices, K, out, workspace,
                              workspace_size, m);
  if (!st.ok) return finish(st);
  if (T && !weights) return fail("packed_switch_glu: null array");
  if (T == 0) return 0;
  hipStream_t s = as_stream(stream);
  Carve c(workspace);
  int32_t* status = c.take<int32_t>(1);
  st = m.forward_with_combine(static_cast<const uint16_t*>(x), T, indices,
                                weights, weights_dtype == MLXR_MOE_BFLOAT16, K,
                                out, nullptr, nullptr, 0, c, status, s);
  return finish(st);
}

int mlxr_moe_packed_switch_glu_experts(const mlxr_moe_packed_switch_glu* ffn,
                                       const void* x, int64_t T,
                                       const int32_t* indices, int64_t K,
                                       void* y, void* workspace,
                                       size_t workspace_size,
                                       mlxr_moe_stream stream) {
  if (!ffn) return fail("packed_switch_glu: null module");
  nn::PackedSwitchFfn m(*ffn);
  Status st = packed_prologue(ffn, x, T, indices, K, y, workspace,
                              workspace_size, m);
  if (!st.ok) return finish(st);
  if (T == 0) return 0;
  hipStream_t s = as_stream(stream);
  Carve c(workspace);
  int32_t* status = c.take<int32_t>(1);
  c.take<uint16_t>(T * K * m.weights().d);  // the combine's y slot, unused
  st = m.forward(static_cast<const uint16_t*>(x), T, indices, K,
                   static_cast<uint16_t*>(y), c, status, s);
  return finish(st);
}

size_t mlxr_moe_block_workspace_size(const mlxr_moe_block* block, int64_t T) {
  if (!block) return 0;
  Carve c(nullptr);
  c.take<int32_t>(1);
  nn::Qwen35MoeBlock::plan(c, *block, T);
  return c.off;
}

int mlxr_moe_block_forward(const mlxr_moe_block* block, const void* x,
                           int64_t T, void* out, int32_t* topk_idx,
                           float* topk_w, void* workspace,
                           size_t workspace_size, mlxr_moe_stream stream) {
  if (!block) return fail("block: null module");
  nn::Qwen35MoeBlock m(*block);
  Status st = m.validate();
  if (!st.ok) return finish(st);
  if (T < 0) return fail("block: bad T");
  if (T && (!x || !out)) return fail("block: null array");
  if (!aligned(x, 16) || !aligned(out, 16) ||
      !aligned(block->gate_weight, 16) ||
      (block->shared_expert_gate_weight &&
       !aligned(block->shared_expert_gate_weight, 16)))
    return fail("block: x, out and router weights must be 16-byte aligned");
  const size_t rq_align = block->gate_q.bits == 16 ? 8 : 4;  // bf16 Linear: 8
  if (!aligned(block->gate_q.weight, rq_align) ||
      !aligned(block->shared_expert_gate_q.weight, rq_align) ||
      !aligned(block->gate_q.scales, 2) || !aligned(block->gate_q.biases, 2) ||
      !aligned(block->shared_expert_gate_q.scales, 2) ||
      !aligned(block->shared_expert_gate_q.biases, 2))
    return fail("block: quantised router words must be 4-byte (bf16 "
                "weights 8-byte) and its scales and biases 2-byte aligned");
  Carve plan(nullptr);
  plan.take<int32_t>(1);
  nn::Qwen35MoeBlock::plan(plan, *block, T);
  st = check_workspace(plan, workspace, workspace_size);
  if (!st.ok) return finish(st);
  if (T == 0) return 0;
  hipStream_t s = as_stream(stream);
  Carve c(workspace);
  c.take<int32_t>(1);  // status word, cleared by the routing kernel
  return finish(m.forward(static_cast<const uint16_t*>(x), T, out, topk_idx,
                          topk_w, c, s));
}

size_t mlxr_moe_block_residual_workspace_size(const mlxr_moe_block* block,
                                              int64_t T) {
  if (!block) return 0;
  Carve c(nullptr);
  c.take<int32_t>(1);
  c.take<uint16_t>(T * block->hidden_size);  // the normed rows
  nn::Qwen35MoeBlock::plan(c, *block, T);
  return c.off;
}

int mlxr_moe_block_forward_residual(const mlxr_moe_block* block,
                                    const void* norm_weight, float eps,
                                    const void* h, int64_t T, void* out,
                                    int32_t* topk_idx, float* topk_w,
                                    void* workspace, size_t workspace_size,
                                    mlxr_moe_stream stream) {
  if (!block) return fail("block_residual: null module");
  nn::Qwen35MoeBlock m(*block);
  Status st = m.validate();
  if (!st.ok) return finish(st);
  if (T < 0) return fail("block_residual: bad T");
  if (!(eps >= 0.0f)) return fail("block_residual: eps must be >= 0");
  if (T && (!h || !out || !norm_weight)) return fail("block_residual: null array");
  if (!aligned(h, 16) || !aligned(out, 16) || !aligned(block->gate_weight, 16) ||
      (block->shared_expert_gate_weight &&
       !aligned(block->shared_expert_gate_weight, 16)))
    return fail("block_residual: h, out and router weights must be 16-byte "
                "aligned");
  const size_t rq_align = block->gate_q.bits == 16 ? 8 : 4;
  if (!aligned(block->gate_q.weight, rq_align) ||
      !aligned(block->shared_expert_gate_q.weight, rq_align) ||
      !aligned(block->gate_q.scales, 2) || !aligned(block->gate_q.biases, 2) ||
      !aligned(block->shared_expert_gate_q.scales, 2) ||
      !aligned(block->shared_expert_gate_q.biases, 2))
    return fail("block_residual: quantised router words must be 4-byte "
                "(bf16 weights 8-byte) and its scales and biases 2-byte "
                "aligned");
  if (workspace_size < mlxr_moe_block_residual_workspace_size(block, T))
    return fail("workspace too small: need " +
                std::to_string(mlxr_moe_block_residual_workspace_size(block, T)) +
                " bytes, got " + std::to_string(workspace_size));
  if (T == 0) return 0;
  if (!workspace || !aligned(workspace, 256))
    return fail("workspace must be non-NULL and 256-byte aligned");
  hipStream_t s = as_stream(stream);
  Carve c(workspace);
  c.take<int32_t>(1);  // status word, cleared by the routing kernel
  uint16_t* normed = c.take<uint16_t>(T * block->hidden_size);
  const uint16_t* hb = static_cast<const uint16_t*>(h);
  // post_attention_layernorm (layer.rs:137) folded into the router's
  // logits kernel, which writes the normalised rows for the experts; the
  // residual add (layer.rs:138) rides in the combine
  const RouterNorm nm{static_cast<const uint16_t*>(norm_weight), eps, normed};
  return finish(m.forward(hb, T, out, topk_idx, topk_w, c, s, hb, &nm));
}

int mlxr_moe_profile_start(const char* kernel) {
  static const char* const kNames[] = {"router_logits", "router_topk",
                                       "dispatch",      "qgemm_gated",
                                       "qgemm_down",    "combine",
                                       "shared_gated",  "shared_down",
                                       "rms_norm",      "read_probe"};
  if (kernel && *kernel) {
    bool known = false;
    for (const char* n : kNames) known = known || std::strcmp(n, kernel) == 0;
    if (!known)
      return fail(std::string("profile_start: unknown kernel '") + kernel +
                  "'");
  }
  return profile_arm(kernel);
}

int mlxr_moe_profile_stop(int64_t* launches, double* total_ms, double* min_ms,
                          double* max_ms) {
  std::string err;
  if (profile_collect(launches, total_ms, min_ms, max_ms, &err) != 0)
    return fail(err);
  return 0;
}

int mlxr_moe_profile_read(const void* buf, size_t bytes, void* sink,
                          mlxr_moe_stream stream) {
  if (!buf || !sink) return fail("profile_read: buf and sink are required");
  if (bytes % 16 || (reinterpret_cast<uintptr_t>(buf) & 15))
    return fail("profile_read: buf must be 16-byte aligned and bytes a multiple of 16");
  return finish(from_hip(
      launch_read_probe(buf, bytes, static_cast<uint32_t*>(sink), as_stream(stream)),
      "profile_read"));
}

int mlxr_moe_workspace_status(const void* workspace, size_t workspace_size,
                              mlxr_moe_stream stream) {
  if (!workspace || workspace_size < sizeof(int32_t))
    return fail("workspace_status: no workspace");
  int32_t v = -1;
  hipStream_t s = as_stream(stream);
  hipError_t e = hipMemcpyAsync(&v, workspace, sizeof(v),
                                hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return finish(from_hip(e, "workspace_status"));
  return v;
}

}  // extern "C"
