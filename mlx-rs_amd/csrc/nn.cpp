// C++ host mirror of mlxr-lm's MoE modules (see nn.hpp for the reference
// mapping).  Orchestration only: every array op is a kernel launch on the
// caller's stream.
#include "nn.hpp"

#include <algorithm>
#include <cstdlib>

// The single-token combine in the down launch (0: always the separate
// combine launch)
#ifndef MLXR_DOWN_COMBINE
#define MLXR_DOWN_COMBINE 1
#endif

namespace mlxr_moe {

Status from_hip(hipError_t e, const char* where) {
  if (e == hipSuccess) return Status{};
  return Status::error(std::string(where) + ": " + hipGetErrorString(e));
}

Status check_qlinear(const mlxr_moe_qlinear& q, int64_t experts, int64_t out,
                     int64_t in, const char* name) {
  const std::string n(name);
  // bits 16: a dense bf16 SwitchLinear / Linear (weight [E, out, in] bf16,
  // no scales or biases; group_size unused)
  const bool dense = q.bits == 16;
  if (dense && (!q.weight || q.scales || q.biases))
    return Status::error(n + ": a dense (bits 16) weight takes no scales or "
                             "biases");
  if (!dense && (!q.weight || !q.scales || !q.biases))
    return Status::error(n + ": weight, scales and biases are required "
                             "(affine mode)");
  if (q.bits != 4 && q.bits != 8 && !dense)
    return Status::error(n + ": bits must be 4 or 8 (16 for dense bf16 "
                             "weights), got " + std::to_string(q.bits));
  if (!dense && q.group_size != 64)
    return Status::error(n + ": group_size must be 64, got " +
                         std::to_string(q.group_size));
  if (q.num_experts != experts || q.output_dims != out || q.input_dims != in)
    return Status::error(
        n + ": shape [" + std::to_string(q.num_experts) + ", " +
        std::to_string(q.output_dims) + ", " + std::to_string(q.input_dims) +
        "] does not match the expected [" + std::to_string(experts) + ", " +
        std::to_string(out) + ", " + std::to_string(in) + "]");
  if (out % 64 || in % 64)
    return Status::error(n + ": input and output dims must be multiples of "
                             "64");
  if (in > kMaxInputDims)
    return Status::error(n + ": input dims above " +
                         std::to_string(kMaxInputDims) + " are not supported");
  if ((reinterpret_cast<uintptr_t>(q.weight) & 15) ||
      (reinterpret_cast<uintptr_t>(q.scales) & 1) ||
      (reinterpret_cast<uintptr_t>(q.biases) & 1))
    return Status::error(n + ": weight must be 16-byte aligned");
  if (dense && (int64_t)out * in * 2 >= ((int64_t)1 << 31))
    return Status::error(n + ": one expert's dense weights must be under 2 GB");
  return Status{};
}

DispatchBuffers carve_dispatch(Carve& c, int64_t n, int64_t E,
                               int32_t* status) {
  DispatchBuffers b{};
  const int64_t nb = (n + kDispatchBlock - 1) / kDispatchBlock;
  b.counts = c.take<int32_t>(E);
  b.offsets = c.take<int32_t>(E + 1);
  b.sorted = c.take<int32_t>(n);
  b.inv = c.take<int32_t>(n);
  b.active = c.take<int32_t>(E);
  b.num_active = c.take<int32_t>(1);
  b.work = c.take<int32_t>(kWorkInts * dispatch_max_work(n, E));
  b.num_work = c.take<int32_t>(1);
  b.work_first = c.take<int32_t>(E);
  b.tiles = c.take<int32_t>(2 * dispatch_max_tiles(n, E, kPrefillMinTileRows));
  b.num_tiles = c.take<int32_t>(1);
  b.block_hist = c.take<int32_t>(nb * E);
  b.rank = c.take<int32_t>(n);
  b.status = status;
  return b;
}

namespace nn {

bool use_prefill_path(int64_t rows, int64_t experts, int bits) {
  // Dense bf16 weights: the split-K kernel reads an expert's weights once
  // per work item (kWorkRows rows), the M-tiled one once per M-tile, with
  // no dequantisation to pay for; it takes over from
  // MLXR_DENSE_TILED_ROWS rows per expert (measured on the c8 block: 2),
  // given rows enough for its tiles to fill the GPU (one expert with 16
  // rows makes four gate/up tiles).
  if (bits == 16)
    return rows >= (int64_t)MLXR_DENSE_TILED_ROWS * experts && rows >= 512;
  // the M-tiled kernel pays once the experts average MLXR_QUANT_TILED_ROWS
  // rows and there are rows enough for its tiles to spread over the GPU
  return rows >= (int64_t)MLXR_QUANT_TILED_ROWS * experts && rows >= 512;
}

namespace {

// MLXR_MOE_DOWN_COMBINE=0 in the environment sends one token through the
// separate down and combine launches as well (bit-identical; read at every
// call, so a test can compare the two forms in one process).
bool down_combine_on() {
  if (!MLXR_DOWN_COMBINE) return false;
  const char* v = std::getenv("MLXR_MOE_DOWN_COMBINE");
  return !(v && v[0] == '0');
}

QWeights qw(const mlxr_moe_qlinear& q) {
  return QWeights{q.weight, static_cast<const uint16_t*>(q.scales),
                  static_cast<const uint16_t*>(q.biases)};
}

}  // namespace

// ------------------------------------------------------------- SwigluMlp
Status SwigluMlp::validate(int64_t d, int64_t f) const {
  Status st = check_qlinear(gate_, 1, f, d, "shared_expert.gate_proj");
  if (st.ok) st = check_qlinear(up_, 1, f, d, "shared_expert.up_proj");
  if (st.ok) st = check_qlinear(down_, 1, d, f, "shared_expert.down_proj");
  if (st.ok && (gate_.bits != up_.bits || gate_.bits != down_.bits))
    st = Status::error("shared_expert: projections must share bits");
  return st;
}

void SwigluMlp::plan(Carve& ws, int64_t T, int64_t d, int64_t f) {
  (void)d;
  carve_dispatch(ws, T, 1, nullptr);
  ws.take<uint16_t>(T * f);
}

// SwigluMlp::forward (swiglu_mlp.rs:63-70): down(swiglu(gate(x), up(x))).
// The dense MLP runs through the grouped kernels as one expert that every
// token selects.
Status SwigluMlp::forward(const uint16_t* x, int64_t T, uint16_t* y,
                          Carve& ws, int32_t* status, hipStream_t s) const {
  const int64_t d = gate_.input_dims, f = gate_.output_dims;
  const DispatchBuffers db = carve_dispatch(ws, T, 1, status);
  uint16_t* act = ws.take<uint16_t>(T * f);
  Status st = from_hip(launch_dispatch_identity(T, prefill_tile_rows(T, 1, gate_.bits), db, s),
                       "shared_expert dispatch");
  if (!st.ok) return st;
  const bool prefill = use_prefill_path(T, 1, gate_.bits);
  QGemmArgs g{};
  g.x = x;
  g.x_ld = d;
  g.x_rows = T;
  g.row_map = nullptr;
  g.row_div = 1;
  g.x_by_slot = false;
  g.out_by_flat = false;
  g.offsets = db.offsets;
  g.active = db.active;
  g.num_active = db.num_active;
  g.work = db.work;
  g.num_work = db.num_work;
  g.tiles = db.tiles;
  g.num_tiles = db.num_tiles;
  g.sorted = db.sorted;
  g.w0 = qw(gate_);
  g.w1 = qw(up_);
  g.E = 1;
  g.N = (int32_t)f;
  g.e_rows = (int32_t)f;
  g.act = kActSwiglu;
  g.K = (int32_t)d;
  g.bits = gate_.bits;
  g.out = act;
  g.out_ld = f;
  g.gated = true;
  const int64_t items = dispatch_max_work(T, 1);
  st = from_hip(launch_qgemm(g, T, items, prefill, s, "shared_gated"),
                "shared_expert gate/up");
  if (!st.ok) return st;
  QGemmArgs h = g;
  h.x = act;
  h.x_ld = f;
  h.x_rows = T;
  h.x_by_slot = true;
  h.w0 = qw(down_);
  h.w1 = QWeights{};
  h.N = (int32_t)d;
  h.e_rows = (int32_t)d;
  h.K = (int32_t)f;
  h.out = y;
  h.out_ld = d;
  h.gated = false;
  return from_hip(launch_qgemm(h, T, items, prefill, s, "shared_down"),
                  "shared_expert down");
}

SharedFold SwigluMlp::fold(Carve ws, int64_t T, uint16_t* y) const {
  (void)carve_dispatch(ws, T, 1, nullptr);  // (unused when folded)
  SharedFold f{};
  f.gate = qw(gate_);
  f.up = qw(up_);
  f.down = qw(down_);
  f.act = ws.take<uint16_t>(T * gate_.output_dims);
  f.y = y;
  return f;
}

// ----------------------------------------------------------- switch FFNs
SplitSwitchFfn::SplitSwitchFfn(const mlxr_moe_switch_glu& w) : w_(w) {
  sw_.gate = qw(w.gate_proj);
  sw_.up = qw(w.up_proj);
  sw_.down = qw(w.down_proj);
  sw_.E = w.gate_proj.num_experts;
  sw_.d = w.gate_proj.input_dims;
  sw_.f = w.gate_proj.output_dims;
  sw_.bits = w.gate_proj.bits;
  sw_.gate_rows = (int32_t)sw_.f;
  sw_.act = kActSwiglu;
}

Status SplitSwitchFfn::validate(int64_t d, int64_t f, int64_t E) const {
  Status st = check_qlinear(w_.gate_proj, E, f, d, "switch_mlp.gate_proj");
  if (st.ok) st = check_qlinear(w_.up_proj, E, f, d, "switch_mlp.up_proj");
  if (st.ok)
    st = check_qlinear(w_.down_proj, E, d, f, "switch_mlp.down_proj");
  if (st.ok && (w_.gate_proj.bits != w_.up_proj.bits ||
                w_.gate_proj.bits != w_.down_proj.bits))
    st = Status::error("switch_mlp: projections must share bits");
  if (st.ok && E > kMaxExperts)
    st = Status::error("switch_mlp: at most " + std::to_string(kMaxExperts) +
                       " experts");
  return st;
}

// The packed tensor's up half starts H rows into each expert: the same
// tensor seen twice, H rows apart, with 2H rows per expert.
PackedSwitchFfn::PackedSwitchFfn(const mlxr_moe_packed_switch_glu& w) : w_(w) {
  const mlxr_moe_qlinear& gu = w.gate_up_proj;
  sw_.E = gu.num_experts;
  sw_.d = gu.input_dims;
  sw_.f = gu.output_dims / 2;
  sw_.bits = gu.bits;
  sw_.gate = qw(gu);
  sw_.up = sw_.gate;
  if (gu.weight && gu.bits > 0) {
    const int64_t words = sw_.f * sw_.d * gu.bits / 32;
    sw_.up.w = gu.weight + words;
    if (gu.bits != 16 && gu.scales && gu.biases) {
      const int64_t g = sw_.d / (gu.group_size > 0 ? gu.group_size : 64);
      sw_.up.scales = sw_.gate.scales + sw_.f * g;
      sw_.up.biases = sw_.gate.biases + sw_.f * g;
    }
  }
  sw_.down = qw(w.down_proj);
  sw_.gate_rows = (int32_t)gu.output_dims;
  sw_.act = w.activation == MLXR_MOE_ACT_GEGLU ? kActGeglu : kActSwiglu;
}

Status PackedSwitchFfn::validate() const {
  const mlxr_moe_qlinear &gu = w_.gate_up_proj, &dn = w_.down_proj;
  const int64_t E = gu.num_experts, d = gu.input_dims, h2 = gu.output_dims;
  if (h2 <= 0 || h2 % 2)
    return Status::error("packed_switch_glu: gate_up_proj output_dims must "
                         "be 2 * hidden_dims");
  if (w_.activation != MLXR_MOE_ACT_SWIGLU && w_.activation != MLXR_MOE_ACT_GEGLU)
    return Status::error("packed_switch_glu: activation must be "
                         "MLXR_MOE_ACT_SWIGLU or MLXR_MOE_ACT_GEGLU");
  Status st = check_qlinear(gu, E, h2, d, "packed_switch_glu.gate_up_proj");
  if (st.ok) st = check_qlinear(dn, E, d, h2 / 2, "packed_switch_glu.down_proj");
  if (st.ok && gu.bits != dn.bits)
    st = Status::error("packed_switch_glu: projections must share bits");
  if (st.ok && E > kMaxExperts)
    st = Status::error("packed_switch_glu: at most " +
                       std::to_string(kMaxExperts) + " experts");
  return st;
}

void SwitchFfn::plan(Carve& ws, int64_t T, int64_t K, int64_t d, int64_t f,
                     int64_t E) {
  ws.take<uint16_t>(T * K * d);  // y (forward_with_combine)
  carve_dispatch(ws, T * K, E, nullptr);
  ws.take<uint16_t>(T * K * f);
}

// SplitSwitchFfn::forward / PackedSwitchFfn::forward (switch.rs:417-442,
// 290-315) on the sorted path: dispatch (gather_sort), then the expert
// products.
Status SwitchFfn::forward(const uint16_t* x, int64_t T, const int32_t* indices,
                          int64_t K, uint16_t* y, Carve& ws, int32_t* status,
                          hipStream_t s, const DownCombine* dc, bool* combined) const {
  if (combined) *combined = false;
  const int64_t E = sw_.E;
  const int64_t n = T * K;
  const DispatchBuffers db = carve_dispatch(ws, n, E, status);
  // (the dispatch clears *status first: no launch of its own for that)
  Status st = from_hip(
      launch_dispatch(indices, n, E, prefill_tile_rows(n, E, sw_.bits), db, true, s),
      "switch_mlp dispatch");
  if (!st.ok) return st;
  return experts(x, T, K, db, y, ws, s, nullptr, dc, combined);
}

// The expert products given the dispatch: gate and up gather_qmm fused with
// the activation (switch.rs:432-434; the packed layout's split_sections,
// switch.rs:305-307, is the H-row offset of the up half), down gather_qmm
// whose rows land at their flat (t, k) position (scatter_unsort,
// switch.rs:437-439).
bool SwitchFfn::can_fold(const SwigluMlp& m, int64_t T, int64_t K) const {
  if (m.bits() != sw_.bits || m.hidden() != sw_.f) return false;
  const bool routed_tiled = use_prefill_path(T * K, sw_.E, sw_.bits);
  const bool shared_tiled = use_prefill_path(T, 1, m.bits());
  // both on the decode kernels (quantised: the streaming kernel), or both
  // on the M-tiled one
  if (!routed_tiled && !shared_tiled) return sw_.bits != 16;
  return routed_tiled && shared_tiled;
}

Status SwitchFfn::experts(const uint16_t* x, int64_t T, int64_t K,
                          const DispatchBuffers& db, uint16_t* y, Carve& ws,
                          hipStream_t s, const SharedFold* fold,
                          const DownCombine* dc, bool* combined) const {
  if (combined) *combined = false;
  const int64_t d = sw_.d, f = sw_.f, E = sw_.E;
  const int64_t n = T * K;
  uint16_t* act = ws.take<uint16_t>(n * f);
  const int64_t max_items = dispatch_max_work(n, E);
  const bool prefill = use_prefill_path(n, E, sw_.bits);
  QGemmArgs g{};
  g.x = x;
  g.x_ld = d;
  g.x_rows = T;
  g.row_map = nullptr;
  g.row_div = (int32_t)K;
  g.x_by_slot = false;
  g.out_by_flat = false;
  g.offsets = db.offsets;
  g.active = db.active;
  g.num_active = db.num_active;
  g.work = db.work;
  g.num_work = db.num_work;
  g.tiles = db.tiles;
  g.num_tiles = db.num_tiles;
  g.sorted = db.sorted;
  g.w0 = sw_.gate;
  g.w1 = sw_.up;
  g.E = (int32_t)E;
  g.N = (int32_t)f;
  g.e_rows = sw_.gate_rows;
  g.act = sw_.act;
  g.K = (int32_t)d;
  g.bits = sw_.bits;
  g.out = act;
  g.out_ld = f;
  g.gated = true;
  // the folded shared expert: every token once, x rows by slot, SwiGLU
  QGemmArgs g2 = g;
  if (fold) {
    g2.row_div = 1;
    g2.x_by_slot = true;
    g2.w0 = fold->gate;
    g2.w1 = fold->up;
    g2.E = 1;
    g2.e_rows = (int32_t)f;
    g2.act = kActSwiglu;
    g2.out = fold->act;
  }
  Status st = from_hip(launch_qgemm(g, n, max_items, prefill, s, nullptr,
                                    fold ? &g2 : nullptr, fold ? T : 0),
                       "switch_mlp gate/up");
  if (!st.ok) return st;
  QGemmArgs h = g;
  h.x = act;
  h.x_ld = f;
  h.x_rows = n;
  h.x_by_slot = true;
  h.w0 = sw_.down;
  h.w1 = QWeights{};
  h.N = (int32_t)d;
  h.e_rows = (int32_t)d;
  h.K = (int32_t)f;
  h.out = y;
  h.out_ld = d;
  h.out_by_flat = true;
  h.gated = false;
  QGemmArgs h2 = h;
  if (fold) {
    h2.x = fold->act;
    h2.x_rows = T;
    h2.w0 = fold->down;
    h2.E = 1;
    h2.out = fold->y;
    h2.out_by_flat = false;
  }
  if (dc && T == 1 && !prefill && down_combine_on()) {
    bool done = false;
    st = from_hip(launch_qgemm_down_combine(h, K, max_items, fold ? &h2 : nullptr, *dc, s,
                                            &done),
                  "switch_mlp down + combine");
    if (!st.ok || done) {
      if (combined) *combined = done;
      return st;
    }
  }
  return from_hip(launch_qgemm(h, n, max_items, prefill, s, nullptr,
                               fold ? &h2 : nullptr, fold ? T : 0),
                  "switch_mlp down");
}

// forward_with_combine (switch.rs:446-474, 322-335) + combine_with_weights
// (switch.rs:223-234); the block's shared branch is added in the same pass.
Status SwitchFfn::forward_with_combine(
    const uint16_t* x, int64_t T, const int32_t* indices, const void* weights,
    bool w_bf16, int64_t K, void* out, const uint16_t* shared_y,
    const float* shared_logit, int64_t shared_ld, Carve& ws, int32_t* status,
    hipStream_t s) const {
  uint16_t* y = ws.take<uint16_t>(T * K * sw_.d);
  // one token: the combine rides in the down launch where it can
  // (caller indices may name one expert several times)
  const DownCombine dc{weights, w_bf16, shared_y, shared_y ? shared_logit : nullptr, nullptr,
                       out, w_bf16, false};
  bool combined = false;
  Status st = forward(x, T, indices, K, y, ws, status, s, T == 1 ? &dc : nullptr, &combined);
  if (!st.ok || combined) return st;
  return from_hip(launch_combine(y, weights, w_bf16, T, K, sw_.d, shared_y,
                                 shared_logit, shared_ld, nullptr, out, w_bf16,
                                 s),
                  "combine");
}

// -------------------------------------------------------- Qwen35MoeBlock
Status Qwen35MoeBlock::validate() const {
  const int64_t d = b_.hidden_size, E = b_.num_experts;
  const int64_t K = b_.num_experts_per_tok, f = b_.moe_intermediate_size;
  if (d <= 0 || E <= 0 || f <= 0)
    return Status::error("block: hidden_size, num_experts and "
                         "moe_intermediate_size must be positive");
  if (K < 1 || K > E || K > 64)
    return Status::error("block: num_experts_per_tok must be in [1, "
                         "min(num_experts, 64)], got " + std::to_string(K));
  if (d % 64)
    return Status::error("block: hidden_size must be a multiple of 64");
  if (quantised_router()) {
    // QuantizedLinear router and shared gate (layers/quantized.rs:356-373),
    // or bf16 Linears (bits 16, layers/linear.rs:91-95): bf16 logits
    const mlxr_moe_qlinear& g = b_.gate_q;
    if (b_.gate_weight || b_.gate_bias || b_.shared_expert_gate_weight)
      return Status::error("block: a quantised or bf16 router (gate_q) "
                           "replaces gate_weight, gate_bias and "
                           "shared_expert_gate_weight; leave them NULL");
    const bool dense = g.bits == 16;
    if (!dense && ((g.bits != 4 && g.bits != 8) || g.group_size != 64))
      return Status::error("block: gate_q must be 4- or 8-bit with group "
                           "size 64, or a bf16 Linear (bits 16)");
    if (g.num_experts != 1 || g.output_dims != E || g.input_dims != d ||
        (dense ? (g.scales || g.biases) : (!g.scales || !g.biases)))
      return Status::error("block: gate_q must be one [num_experts, "
                           "hidden_size] QuantizedLinear with scales and "
                           "biases, or a bf16 Linear without them");
    const mlxr_moe_qlinear& sg = b_.shared_expert_gate_q;
    if (sg.weight &&
        (sg.bits != g.bits || (!dense && sg.group_size != 64) ||
         sg.num_experts != 1 || sg.output_dims != 1 || sg.input_dims != d ||
         (dense ? (sg.scales || sg.biases) : (!sg.scales || !sg.biases))))
      return Status::error("block: shared_expert_gate_q must be a [1, "
                           "hidden_size] linear of gate_q's form (same bits; "
                           "group size 64 when quantised)");
  } else if (!b_.gate_weight) {
    return Status::error("block: gate_weight (or gate_q) is required");
  }
  Status st = SplitSwitchFfn(b_.switch_mlp).validate(d, f, E);
  if (st.ok && has_shared()) {
    const int64_t fs = b_.shared_expert_intermediate_size;
    st = SwigluMlp(b_.shared_gate_proj, b_.shared_up_proj,
                   b_.shared_down_proj)
             .validate(d, fs);
  }
  return st;
}

void Qwen35MoeBlock::plan(Carve& ws, const mlxr_moe_block& b, int64_t T) {
  const int64_t d = b.hidden_size, E = b.num_experts;
  const int64_t K = b.num_experts_per_tok, f = b.moe_intermediate_size;
  const bool shared = Qwen35MoeBlock(b).has_shared();
  ws.take<float>(T * (E + (shared ? 1 : 0)));
  ws.take<int32_t>(T * K);
  ws.take<float>(T * K);
  if (shared) {
    ws.take<uint16_t>(T * d);
    SwigluMlp::plan(ws, T, d, b.shared_expert_intermediate_size);
  }
  SplitSwitchFfn::plan(ws, T, K, d, f, E);
}

// Qwen35MoeBlock::forward (moe.rs:116-146).  Kernels: router logits (with
// the shared-expert gate as one more column), routing (top-k, weights and
// the expert dispatch), [shared expert], gate/up, down, combine.
Status Qwen35MoeBlock::forward(const uint16_t* x, int64_t T, void* out,
                               int32_t* topk_idx, float* topk_w, Carve& ws,
                               hipStream_t s, const uint16_t* residual,
                               const RouterNorm* norm) const {
  const int64_t d = b_.hidden_size, E = b_.num_experts;
  const int64_t K = b_.num_experts_per_tok;
  const bool shared = has_shared();
  const bool bf16 = quantised_router();
  const int64_t ld = E + (shared ? 1 : 0);
  int32_t* status = reinterpret_cast<int32_t*>(ws.base);
  float* logits = ws.take<float>(T * ld);
  int32_t* idx = ws.take<int32_t>(T * K);
  float* wts = ws.take<float>(T * K);
  if (topk_idx) idx = topk_idx;
  if (topk_w) wts = topk_w;
  uint16_t* sy = shared ? ws.take<uint16_t>(T * d) : nullptr;
  Carve shared_ws = ws;  // the shared expert's scratch (plan order)
  if (shared) SwigluMlp::plan(ws, T, d, b_.shared_expert_intermediate_size);
  uint16_t* y = ws.take<uint16_t>(T * K * d);
  const DispatchBuffers db = carve_dispatch(ws, T * K, E, status);
  // gate.forward + shared_expert_gate.forward (moe.rs:118,123) in one pass.
  RouterWeights rw = router_weights_f32(
      b_.gate_weight, shared ? b_.shared_expert_gate_weight : nullptr);
  if (bf16) {
    const mlxr_moe_qlinear &g = b_.gate_q, &sg = b_.shared_expert_gate_q;
    rw = RouterWeights{g.bits,
                       g.weight,
                       static_cast<const uint16_t*>(g.scales),
                       static_cast<const uint16_t*>(g.biases),
                       shared ? sg.weight : nullptr,
                       static_cast<const uint16_t*>(sg.scales),
                       static_cast<const uint16_t*>(sg.biases)};
  }
  // the routing counter of the one-launch top-K and sort: the status
  // word's slot has room beside it, and the logits launch clears it
  int32_t* route_counter = MLXR_ROUTE_FUSED ? status + 1 : nullptr;
  Status st = from_hip(
      launch_router_logits(x, T, d, rw, b_.gate_bias, E, logits, ld, s, norm, route_counter),
      "router logits");
  if (!st.ok) return st;
  if (norm) x = norm->out;  // the experts read the normalised rows
  // softmax, argpartition top-k, renormalise (moe.rs:124-138) + gather_sort
  st = from_hip(launch_route(logits, ld, T, E, K, bf16, idx, wts,
                             prefill_tile_rows(T * K, E, b_.switch_mlp.gate_proj.bits),
                             db, s, route_counter),
                "router top-k / dispatch");
  if (!st.ok) return st;
  const SplitSwitchFfn mlp(b_.switch_mlp);
  const SwigluMlp smlp(b_.shared_gate_proj, b_.shared_up_proj,
                       b_.shared_down_proj);
  // on the decode kernels the shared expert rides in the routed launches
  const bool fold = shared && mlp.can_fold(smlp, T, K);
  if (shared && !fold) {
    st = smlp.forward(x, T, sy, shared_ws, status, s);
    if (!st.ok) return st;
  }
  SharedFold sf{};
  if (fold) sf = smlp.fold(shared_ws, T, sy);
  // one token: the combine rides in the down launch where it can
  // (top-K picks K different experts: one row per work item)
  const DownCombine dc{wts, false, sy, shared ? logits + E : nullptr, residual, out, bf16,
                       true};
  bool combined = false;
  st = mlp.experts(x, T, K, db, y, ws, s, fold ? &sf : nullptr, T == 1 ? &dc : nullptr,
                   &combined);
  if (!st.ok || combined) return st;
  return from_hip(launch_combine(y, wts, false, T, K, d, sy,
                                 shared ? logits + E : nullptr, ld, residual,
                                 out, bf16, s),
                  "combine");
}

}  // namespace nn
}  // namespace mlxr_moe
