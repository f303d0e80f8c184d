// C++ host mirror of mlxr-lm's MoE modules over the gfx950 kernels.
//
//   SwigluMlp        crates/mlxr-lm/src/nn/swiglu_mlp.rs:24-75
//   SplitSwitchFfn   crates/mlxr-lm/src/nn/switch.rs:366-491
//   Qwen35MoeBlock   crates/mlxr-lm/src/qwen3_5/text/moe.rs:43-159
//
// Modules hold non-owning views of caller-owned device weights (the
// mlxr_moe_* descriptors of the C ABI).  forward() enqueues on a stream and
// takes scratch from a caller-provided workspace; the sizes come from the
// same carving code run without a base pointer, so plan and execution
// cannot disagree.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/mlxr_moe.h"
#include "kernels.hpp"

namespace mlxr_moe {

// Bump allocator over a workspace; with base == nullptr it only measures.
struct Carve {
  char* base;
  size_t off = 0;
  explicit Carve(void* b) : base(static_cast<char*>(b)) {}
  template <class T>
  T* take(int64_t count) {
    off = (off + 255) & ~size_t(255);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += size_t(count > 0 ? count : 0) * sizeof(T);
    return p;
  }
};

// Failure inside a module: a message for mlxr_moe_last_error().
struct Status {
  bool ok = true;
  std::string what;
  static Status error(std::string m) { return Status{false, std::move(m)}; }
};

// Sets the C ABI's thread-local error (mlxr_moe_last_error) and returns -1.
int capi_fail(const std::string& msg);

Status check_qlinear(const mlxr_moe_qlinear& q, int64_t experts, int64_t out,
                     int64_t in, const char* name);
Status from_hip(hipError_t e, const char* where);

// Dispatch buffers for n flat rows over E experts, carved from a workspace.
DispatchBuffers carve_dispatch(Carve& c, int64_t n, int64_t E,
                               int32_t* status);

namespace nn {

// Rows per expert above which the MFMA tile kernel with LDS-dequantised
// weights runs instead of the register-dequant kernel (the reference
// switches to its sorted path at T*K >= SORT_THRESHOLD = 2048, switch.rs:40;
// here the choice is about GEMM shape, not sorting, which always happens).
// Dense bf16 GEMMs (bits 16) switch at MLXR_DENSE_TILED_ROWS rows per
// expert.  Measured for the quantised ones (graph steps): at 16 rows per
// expert the tile kernel wins (c6 T=512 391 to 262 µs, c2 T=256 219 to
// 175, c5 T=256 1055 to 676); at 8-10 it does not (c2 T=160 169 to 171,
// c6 T=320 260 to 273, c2 T=128 141 to 162).
#ifndef MLXR_QUANT_TILED_ROWS
#define MLXR_QUANT_TILED_ROWS 16
#endif
#ifndef MLXR_DENSE_TILED_ROWS
#define MLXR_DENSE_TILED_ROWS 2
#endif
bool use_prefill_path(int64_t rows, int64_t experts, int bits = 4);

// A shared expert folded into the routed decode GEMM launches (its gate/up
// and down run as the second problem of the same launches).
struct SharedFold {
  QWeights gate, up, down;
  uint16_t* act;  // [T, f] its activations
  uint16_t* y;    // [T, d] its output
};

class SwigluMlp {
 public:
  SwigluMlp(const mlxr_moe_qlinear& gate, const mlxr_moe_qlinear& up,
            const mlxr_moe_qlinear& down)
      : gate_(gate), up_(up), down_(down) {}
  Status validate(int64_t d, int64_t f) const;
  // y bf16 [T, d] = down(silu(gate(x)) * up(x))
  Status forward(const uint16_t* x, int64_t T, uint16_t* y, Carve& ws,
                 int32_t* status, hipStream_t s) const;
  static void plan(Carve& ws, int64_t T, int64_t d, int64_t f);
  // The fold of this MLP into the routed launches, with its activations in
  // its own workspace region (plan order) and output y.
  SharedFold fold(Carve ws, int64_t T, uint16_t* y) const;
  int bits() const { return gate_.bits; }
  int64_t hidden() const { return gate_.output_dims; }

 private:
  mlxr_moe_qlinear gate_, up_, down_;
};

// The projections of a switch FFN as the kernels see them: gate and up
// (separate tensors, or halves of one packed tensor), down, and the
// activation between them.
struct SwitchWeights {
  QWeights gate, up, down;
  int64_t E, d, f;
  int32_t bits;
  int32_t gate_rows;  // weight rows per expert of the gate/up tensor(s)
  int32_t act;        // kActSwiglu / kActGeglu
};

// The forward shared by both expert layouts (switch.rs:417-474).
class SwitchFfn {
 public:
  // forward: y bf16 [T, K, d] per-expert outputs; clears *status first
  // (in its dispatch launch).
  // With `dc`, as experts().
  Status forward(const uint16_t* x, int64_t T, const int32_t* indices,
                 int64_t K, uint16_t* y, Carve& ws, int32_t* status,
                 hipStream_t s, const DownCombine* dc = nullptr,
                 bool* combined = nullptr) const;
  // The expert products given a dispatch of the T*K flat ids; with `fold`,
  // the shared expert's products in the same launches.  With `dc` at T = 1
  // the combine runs in the down launch where it can
  // (launch_qgemm_down_combine): *combined says whether it did (y is then
  // not written).
  Status experts(const uint16_t* x, int64_t T, int64_t K,
                 const DispatchBuffers& db, uint16_t* y, Carve& ws,
                 hipStream_t s, const SharedFold* fold = nullptr,
                 const DownCombine* dc = nullptr, bool* combined = nullptr) const;
  // Whether a SwiGLU shared expert can fold into this FFN's launches at T
  // tokens: same bits and hidden size, and both on the streaming decode
  // kernel or both on the M-tiled one.
  bool can_fold(const SwigluMlp& m, int64_t T, int64_t K) const;
  // forward_with_combine: out [T, d] = sum_k w * y (+ shared branch); f32
  // weights give an f32 out, bf16 weights (w_bf16) a bf16 out.
  Status forward_with_combine(const uint16_t* x, int64_t T,
                              const int32_t* indices, const void* weights,
                              bool w_bf16, int64_t K, void* out,
                              const uint16_t* shared_y,
                              const float* shared_logit, int64_t shared_ld,
                              Carve& ws, int32_t* status,
                              hipStream_t s) const;
  static void plan(Carve& ws, int64_t T, int64_t K, int64_t d, int64_t f,
                   int64_t E);
  const SwitchWeights& weights() const { return sw_; }

 protected:
  SwitchWeights sw_{};
};

// SplitSwitchFfn<SwigluActivation> (switch.rs:366-491): gate_proj and
// up_proj [E, f, d], down_proj [E, d, f].
class SplitSwitchFfn : public SwitchFfn {
 public:
  explicit SplitSwitchFfn(const mlxr_moe_switch_glu& w);
  Status validate(int64_t d, int64_t f, int64_t E) const;

 private:
  mlxr_moe_switch_glu w_;
};

// PackedSwitchFfn (switch.rs:236-335): gate_up_proj [E, 2H, d] split at H
// (gate channels first), down_proj [E, d, H]; GeGLU for gemma4's
// GemmaSwitchGlu (gemma4/text/mod.rs:27) or SwiGLU.
class PackedSwitchFfn : public SwitchFfn {
 public:
  explicit PackedSwitchFfn(const mlxr_moe_packed_switch_glu& w);
  Status validate() const;

 private:
  mlxr_moe_packed_switch_glu w_;
};

class Qwen35MoeBlock {
 public:
  explicit Qwen35MoeBlock(const mlxr_moe_block& b) : b_(b) {}
  Status validate() const;
  // bf16 router: QuantizedLinear (or bf16 Linear) gate and shared gate
  bool quantised_router() const { return b_.gate_q.weight != nullptr; }
  bool has_shared() const {
    return quantised_router() ? b_.shared_expert_gate_q.weight != nullptr
                              : b_.shared_expert_gate_weight != nullptr;
  }
  // out f32 [T, d], bf16 with a quantised router; with residual (bf16
  // [T, d]) out = residual + the block's output (the decoder layer's add,
  // qwen3_5/text/layer.rs:138), fused into the combine
  // With norm, x is the un-normalised input: the router normalises it and
  // writes norm->out, which the experts then read.
  Status forward(const uint16_t* x, int64_t T, void* out, int32_t* topk_idx,
                 float* topk_w, Carve& ws, hipStream_t s,
                 const uint16_t* residual = nullptr,
                 const RouterNorm* norm = nullptr) const;
  static void plan(Carve& ws, const mlxr_moe_block& b, int64_t T);

 private:
  mlxr_moe_block b_;
};

}  // namespace nn
}  // namespace mlxr_moe
