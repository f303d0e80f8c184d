/*
 * moe_oracle.h -- CPU restatement of mlxr-lm's sparse-MoE block.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity checker for the HIP path
 * and the "port" CPU baseline timed by bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product library (libmlxr_moe.so) never links or calls it.
 *
 * The reference (flukejones/mlx-rs) binds MLX C++ v0.31.2 through mlx-c.
 * Neither is present in /root/reference, so every function below restates
 * the reference's op sequence from its Rust call sites (cited per function)
 * and fixes the numerics MLX leaves unspecified.  The choices are the same
 * on CPU and GPU:
 *   - bf16 conversion is round-to-nearest-even; NaN -> 0x7FC0.
 *   - dequantised weight = round(fmaf(code, scale, bias)) to the scales'
 *     dtype (one rounding).
 *   - router logits use a fixed 64-lane summation order (see
 *     orc_router_logits), so expert selection is bit-reproducible.
 *   - top-k selects on logits (softmax is monotone), descending, ties to
 *     the lower expert id.  With a quantised (bf16) router it selects on the
 *     bf16 probabilities, as the reference does, whose softmax is computed
 *     in double on both sides so that they agree bit for bit.
 *
 * Parity status (what pins each function) is listed in the header of
 * moe_oracle.c and checked by tests/test_oracle.py.
 */
#ifndef MLXR_MOE_ORACLE_H
#define MLXR_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype tags shared with the product C-ABI */
#define ORC_F32 0
#define ORC_BF16 1

float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

/* MLX affine quantisation of w [rows, cols] (cols % group_size == 0).
 * bits in {2,4,8}; group_size in {32,64,128}.  wq [rows, cols*bits/32],
 * scales/biases [rows, cols/group_size] in w's dtype.  Returns 0 or -1. */
int orc_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols,
                 int group_size, int bits, uint32_t* wq, void* scales,
                 void* biases);

/* Inverse: out [rows, cols] in out_dtype.  Returns 0 or -1. */
int orc_dequantize(const uint32_t* wq, const void* scales, const void* biases,
                   int sb_dtype, int64_t rows, int64_t cols, int group_size,
                   int bits, void* out, int out_dtype);

/* logits[t, e] = x[t, :] . w[e, :]  (x bf16 [T,d], w f32 [E,d]) in the
 * fixed lane order described in moe_oracle.c. */
void orc_router_logits(const uint16_t* x, const float* w, int64_t T,
                       int64_t d, int64_t E, float* logits);
/* The same logits in the matrix-core router's order (d % 64 == 0, else -1):
 * four quarters of d, each an fmaf chain over 16-element chunks taken as
 * j, j+8, j+1, j+9, ..., j+7, j+15, the quarters then added in order. */
int orc_router_logits_mfma(const uint16_t* x, const float* w, int64_t T,
                           int64_t d, int64_t E, float* logits);

/* softmax(precise) -> top-K -> renormalise, per row of logits [T, E].
 * idx [T, K] (descending logit, ties -> lower id), weights [T, K]. */
void orc_router_topk(const float* logits, int64_t T, int64_t E, int64_t K,
                     int32_t* idx, float* weights);

/* Router as QuantizedLinear: logits [T, E] (bf16 values as f32) =
 * bf16(x . dequant(wq[e])) with the f32 weights fmaf(code, scale, bias) in
 * orc_router_logits' lane order.  wq [E, d*bits/32], scales/biases bf16
 * [E, d/64]; bits 4 or 8, d % 64 == 0.  Returns 0 or -1. */
int orc_router_logits_q(const uint16_t* x, const uint32_t* wq,
                        const uint16_t* scales, const uint16_t* biases,
                        int bits, int64_t T, int64_t d, int64_t E,
                        float* logits);
/* orc_router_logits_q in the matrix-core order (orc_router_logits_mfma on
 * the same f32 weights, then the bf16 rounding). */
int orc_router_logits_q_mfma(const uint16_t* x, const uint32_t* wq,
                             const uint16_t* scales, const uint16_t* biases,
                             int bits, int64_t T, int64_t d, int64_t E,
                             float* logits);

/* Top-K of bf16 logits [T, E] with bf16 probabilities: selection on the
 * probabilities (descending, ties -> lower id), weights bf16 (as f32). */
void orc_router_topk_bf16(const float* logits, int64_t T, int64_t E,
                          int64_t K, int32_t* idx, float* weights);

/* Stable counting sort of ids [n] by expert (== argsort(flat ids)).
 * counts [E], offsets [E+1], sorted [n] (flat index per sorted slot),
 * inv [n] (sorted slot per flat index).  Returns 0 or -1 (id out of range). */
int orc_dispatch(const int32_t* ids, int64_t n, int64_t E, int32_t* counts,
                 int32_t* offsets, int32_t* sorted, int32_t* inv);

/* gather_qmm with transpose=true:
 *   out[b, m, :] = x[xb(b), m, :] . dequant(w[rhs[b]])^T
 * x bf16 [x_batch, M, Kd]; w u32 [E, N, Kd*bits/32]; scales/biases bf16
 * [E, N, Kd/group]; xb(b) = lhs[b] if lhs else b / (B / x_batch).
 * fp32 accumulation, bf16 output [B, M, N].  tiled = 0: weights
 * dequantised in f32 (vector form); tiled = 1: dequantised weights rounded
 * to bf16 first (tiled form, gather_mm(x, dequantize(w)^T)).  Returns 0 or
 * -1. */
int orc_gather_qmm(const uint16_t* x, int64_t x_batch, int64_t M, int64_t Kd,
                   const uint32_t* w, const uint16_t* scales,
                   const uint16_t* biases, int64_t E, int64_t N,
                   const int32_t* lhs, const int32_t* rhs, int64_t B,
                   int group_size, int bits, int tiled, uint16_t* out,
                   int nthreads);

/* act = silu(g) * u with MLX's per-op bf16 rounding. */
/* gather_mm with the SwitchLinear layout: w bf16 [E, N, Kd] as stored
 * (SwitchLinear::apply passes swap_axes(weight)); otherwise as
 * orc_gather_qmm (same x broadcast, f32 accumulation, bf16 out).  The
 * expert GEMMs of orc_block_forward / orc_packed_switch_glu take dense
 * weights the same way: bits = 16, w the bf16 tensor, scales and biases
 * NULL.  Returns 0 or -1. */
int orc_gather_mm(const uint16_t* x, int64_t x_batch, int64_t M, int64_t Kd,
                  const uint16_t* w, int64_t E, int64_t N, const int32_t* lhs,
                  const int32_t* rhs, int64_t B, uint16_t* out, int nthreads);

void orc_swiglu(const uint16_t* g, const uint16_t* u, int64_t n,
                uint16_t* out);

/* out[t, :] = sum_k w[t,k] * y[t,k,:]  (+ shared[t,:] * sigmoid(sg[t])). */
void orc_combine(const uint16_t* y, const float* w, int64_t T, int64_t K,
                 int64_t d, const uint16_t* shared_y, const float* shared_logit,
                 float* out);

/* act = gelu_approx(g) * u with MLX's per-op bf16 rounding (gemma4). */
void orc_geglu(const uint16_t* g, const uint16_t* u, int64_t n,
               uint16_t* out);

/* fast::rms_norm: out bf16 [T, d] = bf16(w * bf16(x * r)). */
void orc_rms_norm(const uint16_t* x, int64_t T, int64_t d, const uint16_t* w,
                  float eps, uint16_t* out);

/* out bf16 [T, d]: combine with bf16 routing weights (w holds bf16
 * values), every op rounded to bf16. */
void orc_combine_bf16(const uint16_t* y, const float* w, int64_t T, int64_t K,
                      int64_t d, const uint16_t* shared_y,
                      const float* shared_logit, uint16_t* out);

/* One quantised linear bank: w [E, out, in*bits/32], scales/biases bf16. */
typedef struct {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
} orc_qlinear;

typedef struct {
  int64_t hidden;           /* d */
  int64_t num_experts;      /* E */
  int64_t top_k;            /* K */
  int64_t intermediate;     /* f */
  int64_t shared_intermediate; /* f_s, 0 = no shared expert */
  int32_t bits;
  int32_t group_size;
  const float* router_w;    /* [E, d] f32 */
  const float* router_b;    /* [E] f32 or NULL (addmm: dot + bias) */
  orc_qlinear gate_proj, up_proj, down_proj;      /* switch_mlp */
  orc_qlinear shared_gate, shared_up, shared_down; /* E = 1 */
  const float* shared_gate_w; /* [1, d] f32 */
  int32_t switch_tiled;     /* gather_qmm form of the routed experts */
  int32_t shared_tiled;     /* and of the shared expert (see orc_gather_qmm) */
  /* Quantised router (QuantizedLinear, group 64): router_q.w != NULL
   * replaces router_w/router_b (and shared_gate_q replaces shared_gate_w),
   * and the block computes in bf16: bf16 logits, probabilities, weights
   * and out.  E = 1 views of [E, d*bits/32] and [1, d*bits/32]. */
  orc_qlinear router_q;
  orc_qlinear shared_gate_q;
  int32_t router_bits;
  /* router and shared gate, any format: 1 = the matrix-core order
   * (orc_router_logits_mfma / orc_router_logits_q_mfma, the GPU's router
   * for many tokens; needs d % 64 == 0), 0 = the lane order */
  int32_t router_mfma;
} orc_block;

/* PackedSwitchFfn::forward_with_combine: gate_up [E, 2H, d] (gate rows
 * first), down [E, d, H], act 0 = SwiGLU, 1 = GeGLU; w f32 [T, K] holding
 * f32 (w_bf16 = 0, out f32) or bf16 values (w_bf16 = 1, out bf16 as
 * uint16).  y_out (optional) receives the per-expert rows bf16 [T*K, d].
 * Returns 0 or -1. */
int orc_packed_switch_glu(const uint16_t* x, int64_t T, int64_t d, int64_t H,
                          int64_t E, const uint32_t* gu_w,
                          const uint16_t* gu_s, const uint16_t* gu_b,
                          const uint32_t* dn_w, const uint16_t* dn_s,
                          const uint16_t* dn_b, int bits, int act,
                          const int32_t* idx, const float* w, int w_bf16,
                          int64_t K, int tiled, void* out, uint16_t* y_out,
                          int nthreads);

/* gemma4 Router::forward: idx [T, K], weights_out bf16 [T, K].  proj_bf16
 * [E, d] bf16, or proj_q (4/8-bit, group 64) with bits.  mfma: the scores
 * in the matrix-core order (d % 64 == 0).  Returns 0 or -1. */
int orc_gemma_router(const uint16_t* x, int64_t T, int64_t d, int64_t E,
                     int64_t K, const uint16_t* norm_w, float eps,
                     const uint16_t* proj_bf16, const orc_qlinear* proj_q,
                     int bits, const uint16_t* pes, int32_t* idx,
                     uint16_t* weights_out, int mfma);

/* Qwen35MoeBlock::forward on x bf16 [T, d] -> out [T, d], f32 with an f32
 * router, bf16 (uint16 bits) with a quantised one.  idx_out/w_out
 * (optional) receive the routing.  nthreads <= 0 means 1. */
int orc_block_forward(const orc_block* blk, const uint16_t* x, int64_t T,
                      void* out, int32_t* idx_out, float* w_out,
                      int nthreads);

/* out = h + orc_block_forward(orc_rms_norm(h, norm_w, eps)) (DecoderLayer::
 * forward, qwen3_5/text/layer.rs:134-138): f32 out (f32(h) + mlp_out), or
 * bf16 with a bf16 router (bf16(h + mlp_out)).  Returns 0 or -1. */
int orc_block_forward_residual(const orc_block* blk, const uint16_t* norm_w,
                               float eps, const uint16_t* h, int64_t T,
                               void* out, int32_t* idx_out, float* w_out,
                               int nthreads);

#ifdef __cplusplus
}
#endif
#endif
