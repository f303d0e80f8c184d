/*
 * moe_oracle.c -- CPU restatement of mlxr-lm's sparse-MoE block.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the
 * "port" CPU baseline.  Never linked into the product library.
 *
 * Reference op sequence (paths relative to /root/reference):
 *   Qwen35MoeBlock::forward      crates/mlxr-lm/src/qwen3_5/text/moe.rs:116-146
 *   SplitSwitchFfn::forward*     crates/mlxr-lm/src/nn/switch.rs:417-474
 *   combine_with_weights         crates/mlxr-lm/src/nn/switch.rs:223-234
 *   gather_sort / scatter_unsort crates/mlxr-lm/src/nn/switch.rs:499-517
 *   QuantizedSwitchLinear::apply crates/mlxr-lm/src/nn/switch.rs:148-167
 *   SwigluMlp::forward           crates/mlxr-lm/src/nn/swiglu_mlp.rs:63-70
 *   swiglu / silu                crates/mlxr-lm/src/activations.rs:187-200,
 *                                crates/mlxr/src/layers/activation.rs:869-873
 *   quantize/dequantize/gather_qmm crates/mlxr/src/ops/quantization.rs:47-221
 *   argpartition_axis            crates/mlxr/src/ops/sort.rs:186-226
 *   packed layout + dequant      crates/mlxr-lm/src/attention/kernel_source.rs:30-35,96-107
 *   host scalar dequant mirror   crates/mlxr-lm/src/cache/fused_quantized_sdpa.rs:448-530
 *
 * What pins each function (tests/test_oracle.py):
 *   orc_quantize      reference test quantization.rs:299-315 (max error
 *                     bound at bits 2/4/8), closed forms (constant group,
 *                     exact code ladders), brute-force optimality of codes.
 *                     The fp32 scale/bias recipe itself is MLX v0.31.2's
 *                     affine quantiser restated from its published source;
 *                     no reference-held vector pins its last bits.
 *   orc_dequantize    closed form code*scale+bias; round trip with
 *                     orc_quantize; slot layout of kernel_source.rs:101-104.
 *   orc_router_logits fp64 dot products (rounding bound), permutation of
 *                     experts, one-hot inputs.
 *   orc_router_logits_mfma  the same, plus order pins: +-2^24 pairs and a 1
 *                     whose survival depends on the interleave within a
 *                     chunk and on the grouping of the quarters.
 *   orc_router_topk   full sort on small E, softmax sums to 1, renorm.
 *   orc_dispatch      equals a stable argsort (switch.rs:499-512), inverse.
 *   orc_gather_qmm    equals gather_mm(x, dequant(w)^T) in fp64
 *                     (quantization.rs:344-421), lhs/rhs index cases;
 *                     the tiled form bit-for-bit equals that gather_mm on
 *                     bf16 weights up to f32 accumulation (fp64 bound).
 *   orc_swiglu        reference test activations.rs:341-351.
 *   orc_router_logits_q  equals orc_router_logits on the dequantised
 *                     weights, then one bf16 rounding (same lane order);
 *                     fp64 bound.
 *   orc_router_logits_q_mfma  equals orc_router_logits_mfma (pinned
 *                     above) on the dequantised weights, then one bf16
 *                     rounding, at 4, 8 and 16 bits; orc_gemma_router's
 *                     mfma flag takes the same order.
 *   orc_router_topk_bf16 full sort of the bf16 probabilities on small E,
 *                     ties to the lower id; probabilities within one bf16
 *                     rounding of the exact softmax.
 *   orc_combine_bf16  per-op bf16 roundings restated elementwise in numpy.
 *   orc_block_forward sorted and unsorted dispatch give identical outputs
 *                     (switch.rs:446-474); K=1 reduces to one expert;
 *                     linearity in the routing weights.  With dense bf16
 *                     experts: bit-equal to the 4-bit block (tiled
 *                     numerics) whose weights dequantise to them.
 *   orc_gather_mm     the reference's doc example (arithmetic.rs:1565-1575,
 *                     ones -> 32); fp64 bound; bit-equal to the tiled
 *                     orc_gather_qmm at 4 bits on the bf16-dequantised
 *                     weights (quantization.rs:344-421 states that
 *                     identity).
 *   dense router      (lane_dot_q, bits 16) bit-equal to the 8-bit router
 *                     whose codes dequantise exactly to the bf16 weights.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ bf16 */

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0; /* NaN */
  u += 0x7fffu + ((u >> 16) & 1u);                      /* RNE */
  return (uint16_t)(u >> 16);
}

static inline float load_val(const void* p, int dtype, int64_t i) {
  return dtype == ORC_BF16 ? orc_bf16_to_f32(((const uint16_t*)p)[i])
                           : ((const float*)p)[i];
}

static inline void store_val(void* p, int dtype, int64_t i, float v) {
  if (dtype == ORC_BF16)
    ((uint16_t*)p)[i] = orc_f32_to_bf16(v);
  else
    ((float*)p)[i] = v;
}

static inline float round_to(int dtype, float v) {
  return dtype == ORC_BF16 ? orc_bf16_to_f32(orc_f32_to_bf16(v)) : v;
}

static int valid_quant(int group_size, int bits) {
  return (bits == 2 || bits == 4 || bits == 8) &&
         (group_size == 32 || group_size == 64 || group_size == 128);
}

/* the expert GEMMs also take dense bf16 weights (bits 16, gather_mm) */
static int valid_gemm(int group_size, int bits) {
  return valid_quant(group_size, bits) || bits == 16;
}

/* -------------------------------------------------------------- quantize */
/* MLX affine quantiser (mlx v0.31.2, called via mlx_quantize from
 * crates/mlxr/src/ops/quantization.rs:47-70).  Per group of group_size
 * consecutive elements of a row, in fp32:
 *   n_bins = 2^bits - 1
 *   scale  = max((max - min) / n_bins, 1e-7), negated unless |min| > |max|
 *   edge   = |min| > |max| ? min : max
 *   q0     = rint(edge / scale); if q0 != 0: scale = edge / q0, bias = edge
 *   code   = clamp(rint((w - bias) / scale), 0, n_bins)   (unrounded s, b)
 * scale and bias are stored rounded to w's dtype.  Codes pack little-end
 * first: element k of a word sits at bits [k*bits, (k+1)*bits). */
int orc_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols,
                 int group_size, int bits, uint32_t* wq, void* scales,
                 void* biases) {
  if (!valid_quant(group_size, bits) || cols % group_size) return -1;
  const float n_bins = (float)((1 << bits) - 1);
  const int per_word = 32 / bits;
  const int64_t groups = cols / group_size;
  const int64_t words_per_row = cols / per_word;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < groups; ++g) {
      const int64_t base = r * cols + g * group_size;
      float wmax = -INFINITY, wmin = INFINITY;
      for (int j = 0; j < group_size; ++j) {
        float v = load_val(w, w_dtype, base + j);
        wmax = fmaxf(wmax, v);
        wmin = fminf(wmin, v);
      }
      const int neg_edge = fabsf(wmin) > fabsf(wmax);
      float scale = fmaxf((wmax - wmin) / n_bins, 1e-7f);
      scale = neg_edge ? scale : -scale;
      const float edge = neg_edge ? wmin : wmax;
      const float q0 = rintf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      for (int wi = 0; wi < group_size / per_word; ++wi) {
        uint32_t word = 0;
        for (int k = 0; k < per_word; ++k) {
          float v = load_val(w, w_dtype, base + wi * per_word + k);
          float q = rintf((v - bias) / scale);
          q = fminf(fmaxf(q, 0.0f), n_bins);
          word |= (uint32_t)q << (k * bits);
        }
        wq[r * words_per_row + (g * group_size) / per_word + wi] = word;
      }
      store_val(scales, w_dtype, r * groups + g, scale);
      store_val(biases, w_dtype, r * groups + g, bias);
    }
  }
  return 0;
}

/* ------------------------------------------------------------ dequantize */
/* w = code * scale + bias  (kernel_source.rs:96-107; the host mirror at
 * fused_quantized_sdpa.rs:471-480 does the same in f32), evaluated as one
 * fused multiply-add and rounded once to out_dtype. */
int orc_dequantize(const uint32_t* wq, const void* scales, const void* biases,
                   int sb_dtype, int64_t rows, int64_t cols, int group_size,
                   int bits, void* out, int out_dtype) {
  if (!valid_quant(group_size, bits) || cols % group_size) return -1;
  const int per_word = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const int64_t groups = cols / group_size;
  const int64_t words_per_row = cols / per_word;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      const uint32_t word = wq[r * words_per_row + c / per_word];
      const uint32_t code = (word >> ((c % per_word) * bits)) & mask;
      const float s = load_val(scales, sb_dtype, r * groups + c / group_size);
      const float b = load_val(biases, sb_dtype, r * groups + c / group_size);
      store_val(out, out_dtype, r * cols + c, fmaf((float)code, s, b));
    }
  }
  return 0;
}

/* --------------------------------------------------------------- router */
/* Router projection (moe.rs:123 -> Linear::forward, linear.rs:91-95:
 * matmul(x, W^T) with x bf16 promoted to f32).  Summation order, shared
 * with the HIP kernel: 64 lanes; lane l owns elements j = 4l + 256i + c
 * (c = 0..3), accumulates fmaf(x_j, w_j, acc) over i then c; lanes are then
 * combined by the butterfly v += v[l ^ m] for m = 32, 16, 8, 4, 2, 1. */
static float lane_dot(const uint16_t* xrow, const float* wrow, int64_t d) {
  float lane[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int64_t i = 0; 4 * l + 256 * i < d; ++i) {
      for (int c = 0; c < 4; ++c) {
        int64_t j = 4 * l + 256 * i + c;
        if (j < d) acc = fmaf(orc_bf16_to_f32(xrow[j]), wrow[j], acc);
      }
    }
    lane[l] = acc;
  }
  for (int m = 32; m >= 1; m >>= 1) {
    float nxt[64];
    for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ m];
    memcpy(lane, nxt, sizeof(lane));
  }
  return lane[0];
}

void orc_router_logits(const uint16_t* x, const float* w, int64_t T,
                       int64_t d, int64_t E, float* logits) {
  for (int64_t t = 0; t < T; ++t)
    for (int64_t e = 0; e < E; ++e)
      logits[t * E + e] = lane_dot(x + t * d, w + e * d, d);
}

/* The same dot product in the order of the matrix-core router (many
 * tokens, d a multiple of 64): four quarters of d, each a chain of fmaf in
 * chunks of 16 elements taken as j, j + 8, j + 1, j + 9, ..., j + 7, j + 15
 * (one v_mfma_f32_32x32x2_f32 adds two products as fmaf(a1, b1,
 * fmaf(a0, b0, c)), the first from lanes 0-31, which hold elements j..j+7,
 * the second from lanes 32-63, which hold j+8..j+15), then the quarters
 * added as ((q0 + q1) + q2) + q3. */
static float mfma_dot(const uint16_t* xrow, const float* wrow, int64_t d) {
  const int64_t dq = d / 4;
  float q[4];
  for (int i = 0; i < 4; ++i) {
    float acc = 0.0f;
    for (int64_t j = i * dq; j < (i + 1) * dq; j += 16)
      for (int s = 0; s < 8; ++s) {
        acc = fmaf(orc_bf16_to_f32(xrow[j + s]), wrow[j + s], acc);
        acc = fmaf(orc_bf16_to_f32(xrow[j + 8 + s]), wrow[j + 8 + s], acc);
      }
    q[i] = acc;
  }
  return ((q[0] + q[1]) + q[2]) + q[3];
}

int orc_router_logits_mfma(const uint16_t* x, const float* w, int64_t T,
                           int64_t d, int64_t E, float* logits) {
  if (d % 64) return -1;
  for (int64_t t = 0; t < T; ++t)
    for (int64_t e = 0; e < E; ++e)
      logits[t * E + e] = mfma_dot(x + t * d, w + e * d, d);
  return 0;
}

/* softmax_axis(precise) + argpartition(-K) + take_along_axis + sum + divide
 * (moe.rs:124-138).  Selection on logits, descending, ties to the lower id.
 * Softmax: m = max, S = sum exp(l - m) accumulated per lane (lane l holds
 * experts l, l+64, ...) then the same butterfly as above; p = exp(l - m)/S;
 * weights = p_k / (p_0 + ... + p_{K-1}) summed in k order. */
void orc_router_topk(const float* logits, int64_t T, int64_t E, int64_t K,
                     int32_t* idx, float* weights) {
  char* taken = (char*)malloc((size_t)E);
  float* p = (float*)malloc(sizeof(float) * (size_t)K);
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    memset(taken, 0, (size_t)E);
    for (int64_t k = 0; k < K; ++k) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || l[e] > l[best]) best = e;
      }
      taken[best] = 1;
      idx[t * K + k] = (int32_t)best;
    }
    const float m = l[idx[t * K]];
    float lane[64];
    for (int ln = 0; ln < 64; ++ln) {
      float acc = 0.0f;
      for (int64_t e = ln; e < E; e += 64) acc += expf(l[e] - m);
      lane[ln] = acc;
    }
    for (int msk = 32; msk >= 1; msk >>= 1) {
      float nxt[64];
      for (int ln = 0; ln < 64; ++ln) nxt[ln] = lane[ln] + lane[ln ^ msk];
      memcpy(lane, nxt, sizeof(lane));
    }
    const float S = lane[0];
    float psum = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      p[k] = expf(l[idx[t * K + k]] - m) / S;
      psum += p[k];
    }
    for (int64_t k = 0; k < K; ++k) weights[t * K + k] = p[k] / psum;
  }
  free(p);
  free(taken);
}

/* ------------------------------------------------------ quantised router */
/* Router as QuantizedLinear (gate: MaybeQuantized<Linear>, moe.rs:57,123;
 * QuantizedLinear::forward, layers/quantized.rs:356-373 ->
 * quantized_matmul, ops/quantization.rs:81-112).  The shipped Qwen3.6
 * checkpoints quantise mlp.gate and mlp.shared_expert_gate at 8 bits, group
 * 64 (tests/fixtures/qwen3_6_35b_a3b/config.json, applied by
 * qwen3_5/text/moe.rs:255-284).  With bf16 x and bf16 scales the result is
 * bf16.  Same lane order as lane_dot; the weight of element j is the f32
 * fmaf(code_j, scale, bias) of its group of 64; the f32 sum is rounded once
 * to bf16 (returned as its f32 value). */
static float lane_dot_q(const uint16_t* xrow, const uint32_t* wrow,
                        const uint16_t* srow, const uint16_t* brow, int64_t d,
                        int bits) {
  if (bits == 16) {
    /* a dense bf16 Linear ([E, d] bf16; Linear::forward, layers/linear.rs:
     * 91-95, in bf16): the same lane order over the bf16 weights, one
     * rounding of the sum */
    const uint16_t* w16 = (const uint16_t*)wrow;
    float* wf = (float*)malloc(sizeof(float) * (size_t)d);
    for (int64_t j = 0; j < d; ++j) wf[j] = orc_bf16_to_f32(w16[j]);
    const float v = lane_dot(xrow, wf, d);
    free(wf);
    return orc_bf16_to_f32(orc_f32_to_bf16(v));
  }
  const int per_word = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  float lane[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int64_t i = 0; 4 * l + 256 * i < d; ++i) {
      for (int c = 0; c < 4; ++c) {
        const int64_t j = 4 * l + 256 * i + c;
        if (j >= d) continue;
        const uint32_t code =
            (wrow[j / per_word] >> ((j % per_word) * bits)) & mask;
        const float w = fmaf((float)code, orc_bf16_to_f32(srow[j / 64]),
                             orc_bf16_to_f32(brow[j / 64]));
        acc = fmaf(orc_bf16_to_f32(xrow[j]), w, acc);
      }
    }
    lane[l] = acc;
  }
  for (int m = 32; m >= 1; m >>= 1) {
    float nxt[64];
    for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ m];
    memcpy(lane, nxt, sizeof(lane));
  }
  return orc_bf16_to_f32(orc_f32_to_bf16(lane[0]));
}

int orc_router_logits_q(const uint16_t* x, const uint32_t* wq,
                        const uint16_t* scales, const uint16_t* biases,
                        int bits, int64_t T, int64_t d, int64_t E,
                        float* logits) {
  if ((bits != 4 && bits != 8 && bits != 16) || d % 64) return -1;
  const int64_t wpr = d * bits / 32, gpr = bits == 16 ? 0 : d / 64;
  for (int64_t t = 0; t < T; ++t)
    for (int64_t e = 0; e < E; ++e)
      logits[t * E + e] = lane_dot_q(x + t * d, wq + e * wpr,
                                     scales ? scales + e * gpr : NULL,
                                     biases ? biases + e * gpr : NULL, d, bits);
  return 0;
}

/* lane_dot_q in the matrix-core order: the f32 weights (fmaf(code, scale,
 * bias), or the bf16 values of a dense Linear) through mfma_dot, then one
 * bf16 rounding. */
static float mfma_dot_q(const uint16_t* xrow, const uint32_t* wrow,
                        const uint16_t* srow, const uint16_t* brow, int64_t d,
                        int bits) {
  float* wf = (float*)malloc(sizeof(float) * (size_t)d);
  if (bits == 16) {
    const uint16_t* w16 = (const uint16_t*)wrow;
    for (int64_t j = 0; j < d; ++j) wf[j] = orc_bf16_to_f32(w16[j]);
  } else {
    const int per_word = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t j = 0; j < d; ++j) {
      const uint32_t code = (wrow[j / per_word] >> ((j % per_word) * bits)) & mask;
      wf[j] = fmaf((float)code, orc_bf16_to_f32(srow[j / 64]), orc_bf16_to_f32(brow[j / 64]));
    }
  }
  const float v = mfma_dot(xrow, wf, d);
  free(wf);
  return orc_bf16_to_f32(orc_f32_to_bf16(v));
}

int orc_router_logits_q_mfma(const uint16_t* x, const uint32_t* wq,
                             const uint16_t* scales, const uint16_t* biases,
                             int bits, int64_t T, int64_t d, int64_t E,
                             float* logits) {
  if ((bits != 4 && bits != 8 && bits != 16) || d % 64) return -1;
  const int64_t wpr = d * bits / 32, gpr = bits == 16 ? 0 : d / 64;
  for (int64_t t = 0; t < T; ++t)
    for (int64_t e = 0; e < E; ++e)
      logits[t * E + e] = mfma_dot_q(x + t * d, wq + e * wpr,
                                     scales ? scales + e * gpr : NULL,
                                     biases ? biases + e * gpr : NULL, d, bits);
  return 0;
}

/* softmax_axis(precise) keeps the input dtype (arithmetic.rs:1298-1311), so
 * bf16 logits give bf16 probabilities, and argpartition (sort.rs:211-226)
 * selects on those: distinct logits can tie.  Here m = max logit;
 * e_j = exp((double)l_j - m) in double; S = sum of e_j in double (lane l
 * holds experts l, l+64, ..., then the butterfly); p_j =
 * bf16((float)(e_j / S)).  Double keeps p independent of the exp and
 * summation details of either side.  Selection on p, descending, ties to
 * the lower id.  take_along_axis / sum / divide (moe.rs:136-138) in bf16:
 * denom = bf16(f32 sum of p_k in k order), w_k = bf16(p_k / denom) with an
 * f32 division. */
void orc_router_topk_bf16(const float* logits, int64_t T, int64_t E,
                          int64_t K, int32_t* idx, float* weights) {
  char* taken = (char*)malloc((size_t)E);
  float* p = (float*)malloc(sizeof(float) * (size_t)E);
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    float m = l[0];
    for (int64_t e = 1; e < E; ++e) m = l[e] > m ? l[e] : m;
    double lane[64];
    for (int ln = 0; ln < 64; ++ln) {
      double acc = 0.0;
      for (int64_t e = ln; e < E; e += 64) acc += exp((double)l[e] - (double)m);
      lane[ln] = acc;
    }
    for (int msk = 32; msk >= 1; msk >>= 1) {
      double nxt[64];
      for (int ln = 0; ln < 64; ++ln) nxt[ln] = lane[ln] + lane[ln ^ msk];
      memcpy(lane, nxt, sizeof(lane));
    }
    const double S = lane[0];
    for (int64_t e = 0; e < E; ++e)
      p[e] = orc_bf16_to_f32(
          orc_f32_to_bf16((float)(exp((double)l[e] - (double)m) / S)));
    memset(taken, 0, (size_t)E);
    float psum = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || p[e] > p[best]) best = e;
      }
      taken[best] = 1;
      idx[t * K + k] = (int32_t)best;
      psum += p[best];
    }
    const float denom = orc_bf16_to_f32(orc_f32_to_bf16(psum));
    for (int64_t k = 0; k < K; ++k)
      weights[t * K + k] =
          orc_bf16_to_f32(orc_f32_to_bf16(p[idx[t * K + k]] / denom));
  }
  free(p);
  free(taken);
}

/* ------------------------------------------------------------- dispatch */
/* gather_sort (switch.rs:499-512): order = argsort(flat ids) (stable),
 * inv = argsort(order).  Counting sort gives the same permutation. */
int orc_dispatch(const int32_t* ids, int64_t n, int64_t E, int32_t* counts,
                 int32_t* offsets, int32_t* sorted, int32_t* inv) {
  memset(counts, 0, sizeof(int32_t) * (size_t)E);
  for (int64_t i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] >= E) return -1;
    counts[ids[i]]++;
  }
  offsets[0] = 0;
  for (int64_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t* fill = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  memcpy(fill, offsets, sizeof(int32_t) * (size_t)E);
  for (int64_t i = 0; i < n; ++i) {
    int32_t pos = fill[ids[i]]++;
    sorted[pos] = (int32_t)i;
    inv[i] = pos;
  }
  free(fill);
  return 0;
}

/* ----------------------------------------------------------- gather_qmm */
/* gather_qmm has two numerics, as MLX's has (its matrix-vector kernels for
 * few rows per expert, its tiled matrix-matrix kernels for many):
 *   vector form  each weight is fmaf(code, scale, bias) in f32;
 *   tiled form   each weight is that value rounded to bf16 first -- the
 *                weight tile is dequantised into the activation dtype, and
 *                the product is gather_mm(x, dequantize(w)^T), which is how
 *                the reference's own test defines gather_qmm
 *                (quantization.rs:344-421).
 * Both accumulate in f32.  The GPU picks the form per GEMM from the rows per
 * expert (mlxr_moe_gather_qmm_tiled); the checks pass the same choice. */
/* One output element: x (already f32) . dequant(weight row), f32
 * accumulation in 8 interleaved partial sums. */
static float qdot(const float* xf, const uint32_t* wrow, const uint16_t* srow,
                  const uint16_t* brow, int64_t Kd, int gs, int bits,
                  int tiled) {
  if (bits == 16) {
    /* dense bf16 row (gather_mm): the same partial sums over the weights as
     * they are */
    const uint16_t* w16 = (const uint16_t*)wrow;
    float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t k = 0; k < Kd; ++k)
      part[k & 7] = fmaf(xf[k], orc_bf16_to_f32(w16[k]), part[k & 7]);
    return ((part[0] + part[1]) + (part[2] + part[3])) +
           ((part[4] + part[5]) + (part[6] + part[7]));
  }
  const int per_word = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t g = 0; g < Kd / gs; ++g) {
    const float s = orc_bf16_to_f32(srow[g]);
    const float b = orc_bf16_to_f32(brow[g]);
    const uint32_t* wg = wrow + g * gs / per_word;
    const float* xg = xf + g * gs;
    for (int wi = 0; wi < gs / per_word; ++wi) {
      uint32_t word = wg[wi];
      for (int k = 0; k < per_word; ++k) {
        float wv = fmaf((float)((word >> (k * bits)) & mask), s, b);
        if (tiled) wv = orc_bf16_to_f32(orc_f32_to_bf16(wv));
        part[k & 7] = fmaf(xg[wi * per_word + k], wv, part[k & 7]);
      }
    }
  }
  return ((part[0] + part[1]) + (part[2] + part[3])) +
         ((part[4] + part[5]) + (part[6] + part[7]));
}

/* y[n] = bf16(x . dequant(W[e, n])) for n in [0, N); bits 16: W is a
 * dense bf16 [E, N, Kd] tensor (no scales or biases) */
static void qmv(const float* xf, const orc_qlinear* q, int64_t e, int64_t N,
                int64_t Kd, int gs, int bits, int tiled, uint16_t* y) {
  const int64_t wpr = Kd * bits / 32, gpr = bits == 16 ? 0 : Kd / gs;
  for (int64_t n = 0; n < N; ++n) {
    const int64_t row = e * N + n;
    y[n] = orc_f32_to_bf16(qdot(xf, q->w + row * wpr,
                                q->scales ? q->scales + row * gpr : NULL,
                                q->biases ? q->biases + row * gpr : NULL, Kd,
                                gs, bits, tiled));
  }
}

int orc_gather_qmm(const uint16_t* x, int64_t x_batch, int64_t M, int64_t Kd,
                   const uint32_t* w, const uint16_t* scales,
                   const uint16_t* biases, int64_t E, int64_t N,
                   const int32_t* lhs, const int32_t* rhs, int64_t B,
                   int group_size, int bits, int tiled, uint16_t* out,
                   int nthreads) {
  if (!valid_gemm(group_size, bits) || Kd % group_size) return -1;
  if (!lhs && (x_batch <= 0 || B % x_batch)) return -1;
  for (int64_t b = 0; b < B; ++b) {
    if (rhs[b] < 0 || rhs[b] >= E) return -1;
    if (lhs && (lhs[b] < 0 || lhs[b] >= x_batch)) return -1;
  }
  orc_qlinear q = {w, scales, biases};
  const int64_t rep = lhs ? 1 : B / x_batch;
  if (nthreads <= 0) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (int64_t bm = 0; bm < B * M; ++bm) {
    const int64_t b = bm / M, m = bm % M;
    const int64_t xb = lhs ? lhs[b] : b / rep;
    float* xf = (float*)malloc(sizeof(float) * (size_t)Kd);
    for (int64_t j = 0; j < Kd; ++j)
      xf[j] = orc_bf16_to_f32(x[(xb * M + m) * Kd + j]);
    qmv(xf, &q, rhs[b], N, Kd, group_size, bits, tiled, out + bm * N);
    free(xf);
  }
  return 0;
}

/* gather_mm with the SwitchLinear layout (SwitchLinear::apply,
 * nn/switch.rs:84-93: gather_mm(x, swap_axes(weight, -1, -2), None,
 * indices), ops/arithmetic.rs:1577-1613): w bf16 [E, N, Kd] as stored,
 * out[b, m] = bf16(x[xb, m] . w[rhs[b], n]) with f32 accumulation -- the
 * tiled gather_qmm's sum over weights that need no dequantisation.  No bias:
 * every SwitchLinear on this path is built with bias = false (qwen3_5/text/
 * moe.rs:92-97, gemma4/text/text.rs:679). */
int orc_gather_mm(const uint16_t* x, int64_t x_batch, int64_t M, int64_t Kd,
                  const uint16_t* w, int64_t E, int64_t N, const int32_t* lhs,
                  const int32_t* rhs, int64_t B, uint16_t* out, int nthreads) {
  /* (no groups: any Kd) */
  return orc_gather_qmm(x, x_batch, M, Kd, (const uint32_t*)w, NULL, NULL, E,
                        N, lhs, rhs, B, 1, 16, 1, out, nthreads);
}

/* ------------------------------------------------------------- swiglu */
/* silu(g) * u (activations.rs:187-200) with silu = g * sigmoid(g)
 * (activation.rs:869-873).  MLX evaluates the compiled graph in the
 * arrays' dtype, so every op result is rounded to bf16. */
static inline float swiglu1(float g, float u) {
  const float sg = orc_bf16_to_f32(orc_f32_to_bf16(1.0f / (1.0f + expf(-g))));
  const float h = orc_bf16_to_f32(orc_f32_to_bf16(g * sg));
  return h * u;
}

void orc_swiglu(const uint16_t* g, const uint16_t* u, int64_t n,
                uint16_t* out) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = orc_f32_to_bf16(
        swiglu1(orc_bf16_to_f32(g[i]), orc_bf16_to_f32(u[i])));
}

/* geglu (activations.rs:223-259): gelu_approximate_in_dtype(g) * u, every
 * op in bf16 with the constants cast to bf16 first:
 * 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))). */
static inline float bfr(float v) { return orc_bf16_to_f32(orc_f32_to_bf16(v)); }
static inline float geglu1(float g, float u) {
  const float k = bfr(0.044715f), c = bfr(0.7978845608028654f);
  const float x3 = bfr(bfr(g * g) * g);
  const float inner = bfr(g + bfr(k * x3));
  const float t = bfr(tanhf(bfr(c * inner)));
  const float gl = bfr(bfr(0.5f * g) * bfr(1.0f + t));
  return gl * u;
}

void orc_geglu(const uint16_t* g, const uint16_t* u, int64_t n,
               uint16_t* out) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = orc_f32_to_bf16(
        geglu1(orc_bf16_to_f32(g[i]), orc_bf16_to_f32(u[i])));
}

/* ------------------------------------------------------------- combine */
/* combine_with_weights (switch.rs:223-234): (w * y) rounded to f32, then
 * summed over k in order.  Shared branch (moe.rs:117-120,145):
 * shared = y_s * sigmoid(sg); out = shared + routed. */
void orc_combine(const uint16_t* y, const float* w, int64_t T, int64_t K,
                 int64_t d, const uint16_t* shared_y, const float* shared_logit,
                 float* out) {
  for (int64_t t = 0; t < T; ++t) {
    float gate = 0.0f;
    if (shared_y) gate = 1.0f / (1.0f + expf(-shared_logit[t]));
    for (int64_t n = 0; n < d; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float prod = w[t * K + k] * orc_bf16_to_f32(y[(t * K + k) * d + n]);
        acc += prod;
      }
      if (shared_y) {
        const float sh = orc_bf16_to_f32(shared_y[t * d + n]) * gate;
        acc = sh + acc;
      }
      out[t * d + n] = acc;
    }
  }
}

/* The same with bf16 routing weights (a bf16 router, see
 * orc_router_topk_bf16): w * y is bf16, the sum over k is accumulated in
 * f32 in k order and rounded to bf16; shared = bf16(y_s *
 * bf16(sigmoid(sg))); out = bf16(shared + routed). */
void orc_combine_bf16(const uint16_t* y, const float* w, int64_t T, int64_t K,
                      int64_t d, const uint16_t* shared_y,
                      const float* shared_logit, uint16_t* out) {
  for (int64_t t = 0; t < T; ++t) {
    float gate = 0.0f;
    if (shared_y)
      gate = orc_bf16_to_f32(
          orc_f32_to_bf16(1.0f / (1.0f + expf(-shared_logit[t]))));
    for (int64_t n = 0; n < d; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k)
        acc += orc_bf16_to_f32(orc_f32_to_bf16(
            w[t * K + k] * orc_bf16_to_f32(y[(t * K + k) * d + n])));
      float r = orc_bf16_to_f32(orc_f32_to_bf16(acc));
      if (shared_y) {
        const float sh = orc_bf16_to_f32(
            orc_f32_to_bf16(orc_bf16_to_f32(shared_y[t * d + n]) * gate));
        r = sh + r;
      }
      out[t * d + n] = orc_f32_to_bf16(r);
    }
  }
}

/* ----------------------------------------------------- PackedSwitchFfn */
/* PackedSwitchFfn::forward_with_combine (switch.rs:290-335): per (t, k),
 * gate_up = gather_qmm over all 2H rows of expert idx, split_sections at H
 * (gate first), the activation (GeGLU for gemma4's GemmaSwitchGlu, or
 * SwiGLU), the down gather_qmm, then combine_with_weights: f32 weights give
 * an f32 out (orc_combine), bf16 weights a bf16 out (orc_combine_bf16). */
int orc_packed_switch_glu(const uint16_t* x, int64_t T, int64_t d, int64_t H,
                          int64_t E, const uint32_t* gu_w,
                          const uint16_t* gu_s, const uint16_t* gu_b,
                          const uint32_t* dn_w, const uint16_t* dn_s,
                          const uint16_t* dn_b, int bits, int act,
                          const int32_t* idx, const float* w, int w_bf16,
                          int64_t K, int tiled, void* out, uint16_t* y_out,
                          int nthreads) {
  if (!valid_gemm(64, bits) || d % 64 || H % 64 || (act != 0 && act != 1))
    return -1;
  for (int64_t i = 0; i < T * K; ++i)
    if (idx[i] < 0 || idx[i] >= E) return -1;
  if (nthreads <= 0) nthreads = 1;
  orc_qlinear gu = {gu_w, gu_s, gu_b}, dn = {dn_w, dn_s, dn_b};
  uint16_t* y = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * K * d));
#pragma omp parallel num_threads(nthreads)
  {
    float* xf = (float*)malloc(sizeof(float) * (size_t)d);
    float* af = (float*)malloc(sizeof(float) * (size_t)H);
    uint16_t* gub = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(2 * H));
#pragma omp for schedule(dynamic, 1)
    for (int64_t tk = 0; tk < T * K; ++tk) {
      const int64_t t = tk / K;
      for (int64_t j = 0; j < d; ++j) xf[j] = orc_bf16_to_f32(x[t * d + j]);
      qmv(xf, &gu, idx[tk], 2 * H, d, 64, bits, tiled, gub);
      for (int64_t n = 0; n < H; ++n) {
        const float g = orc_bf16_to_f32(gub[n]), u = orc_bf16_to_f32(gub[H + n]);
        af[n] = orc_bf16_to_f32(orc_f32_to_bf16(act ? geglu1(g, u) : swiglu1(g, u)));
      }
      qmv(af, &dn, idx[tk], d, H, 64, bits, tiled, y + tk * d);
    }
    free(xf);
    free(af);
    free(gub);
  }
  if (out) {
    if (w_bf16)
      orc_combine_bf16(y, w, T, K, d, NULL, NULL, (uint16_t*)out);
    else
      orc_combine(y, w, T, K, d, NULL, NULL, (float*)out);
  }
  if (y_out) memcpy(y_out, y, sizeof(uint16_t) * (size_t)(T * K * d));
  free(y);
  return 0;
}

/* ------------------------------------------------------- gemma4 router */
/* fast::rms_norm (gemma4 Router::forward, text.rs:640): out_j = bf16(w_j *
 * bf16(x_j * r)), r = 1 / sqrt(sum_j x_j^2 / d + eps), the sum of squares
 * in the router's lane order (lane l: fmaf over j = 4l + 256i + c; then
 * the butterfly). */
void orc_rms_norm(const uint16_t* x, int64_t T, int64_t d, const uint16_t* w,
                  float eps, uint16_t* out) {
  for (int64_t t = 0; t < T; ++t) {
    const uint16_t* xr = x + t * d;
    float lane[64];
    for (int l = 0; l < 64; ++l) {
      float acc = 0.0f;
      for (int64_t i = 0; 4 * l + 256 * i < d; ++i)
        for (int c = 0; c < 4; ++c) {
          const int64_t j = 4 * l + 256 * i + c;
          if (j < d) {
            const float v = orc_bf16_to_f32(xr[j]);
            acc = fmaf(v, v, acc);
          }
        }
      lane[l] = acc;
    }
    for (int m = 32; m >= 1; m >>= 1) {
      float nxt[64];
      for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ m];
      memcpy(lane, nxt, sizeof(lane));
    }
    const float r = 1.0f / sqrtf(lane[0] / (float)d + eps);
    for (int64_t j = 0; j < d; ++j)
      out[t * d + j] = orc_f32_to_bf16(
          orc_bf16_to_f32(w[j]) * bfr(orc_bf16_to_f32(xr[j]) * r));
  }
}

/* gemma4 Router::forward (text.rs:621-665): normed = rms_norm(x); scores =
 * bf16(normed . W_e) (a bf16 Linear, proj_bf16 [E, d], or a QuantizedLinear
 * (proj_q, bits, group 64) -- orc_router_logits' lane order); top-K on the
 * scores (descending, ties to the lower id); router_post
 * (activations.rs:309-331): softmax of the K selected scores in bf16
 * (d_k = bf16(s_k - m), e_k = bf16(exp(d_k)) with exp in double,
 * S = bf16(sum_k e_k in f32, k in order), p_k = bf16(e_k / S)) times
 * per_expert_scale[id_k], rounded to bf16.  weights_out [T, K] bf16. */
int orc_gemma_router(const uint16_t* x, int64_t T, int64_t d, int64_t E,
                     int64_t K, const uint16_t* norm_w, float eps,
                     const uint16_t* proj_bf16, const orc_qlinear* proj_q,
                     int bits, const uint16_t* pes, int32_t* idx,
                     uint16_t* weights_out, int mfma) {
  if (K < 1 || K > E || (!proj_bf16 && !proj_q)) return -1;
  if (mfma && d % 64) return -1;
  if (proj_q && ((bits != 4 && bits != 8) || d % 64)) return -1;
  uint16_t* normed = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * d));
  float* wrow = (float*)malloc(sizeof(float) * (size_t)d);
  float* sc = (float*)malloc(sizeof(float) * (size_t)E);
  char* taken = (char*)malloc((size_t)E);
  orc_rms_norm(x, T, d, norm_w, eps, normed);
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t e = 0; e < E; ++e) {
      if (proj_q) {
        sc[e] = (mfma ? mfma_dot_q : lane_dot_q)(normed + t * d, proj_q->w + e * (d * bits / 32),
                                                 proj_q->scales + e * (d / 64),
                                                 proj_q->biases + e * (d / 64), d, bits);
      } else {
        for (int64_t j = 0; j < d; ++j) wrow[j] = orc_bf16_to_f32(proj_bf16[e * d + j]);
        sc[e] = bfr(mfma ? mfma_dot(normed + t * d, wrow, d) : lane_dot(normed + t * d, wrow, d));
      }
    }
    memset(taken, 0, (size_t)E);
    float sel[64];
    for (int64_t k = 0; k < K; ++k) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || sc[e] > sc[best]) best = e;
      }
      taken[best] = 1;
      idx[t * K + k] = (int32_t)best;
      sel[k] = sc[best];
    }
    const float m = sel[0];
    float ek[64], S = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      ek[k] = bfr((float)exp((double)bfr(sel[k] - m)));
      S += ek[k];
    }
    S = bfr(S);
    for (int64_t k = 0; k < K; ++k) {
      const float p = bfr(ek[k] / S);
      weights_out[t * K + k] =
          orc_f32_to_bf16(p * orc_bf16_to_f32(pes[idx[t * K + k]]));
    }
  }
  free(normed);
  free(wrow);
  free(sc);
  free(taken);
  return 0;
}

/* --------------------------------------------------------------- block */
/* One expert FFN on one token: y = down(swiglu(gate(x), up(x))). */
static void expert_ffn(const float* xf, const orc_qlinear* g,
                       const orc_qlinear* u, const orc_qlinear* dn, int64_t e,
                       int64_t d, int64_t f, int gs, int bits, int tiled,
                       uint16_t* y, uint16_t* gb, uint16_t* ub, float* af) {
  qmv(xf, g, e, f, d, gs, bits, tiled, gb);
  qmv(xf, u, e, f, d, gs, bits, tiled, ub);
  for (int64_t n = 0; n < f; ++n) {
    uint16_t a = orc_f32_to_bf16(
        swiglu1(orc_bf16_to_f32(gb[n]), orc_bf16_to_f32(ub[n])));
    af[n] = orc_bf16_to_f32(a);
  }
  qmv(af, dn, e, d, f, gs, bits, tiled, y);
}

int orc_block_forward(const orc_block* blk, const uint16_t* x, int64_t T,
                      void* out, int32_t* idx_out, float* w_out,
                      int nthreads) {
  const int64_t d = blk->hidden, E = blk->num_experts, K = blk->top_k;
  const int64_t f = blk->intermediate, fs = blk->shared_intermediate;
  const int gs = blk->group_size, bits = blk->bits;
  if (!valid_gemm(gs, bits) || d % gs || f % gs || (fs && fs % gs) ||
      K < 1 || K > E || K > 64)
    return -1;
  if (nthreads <= 0) nthreads = 1;

  const int qr = blk->router_q.w != NULL;
  if (qr && ((blk->router_bits != 4 && blk->router_bits != 8 &&
              blk->router_bits != 16) ||
             (fs && !blk->shared_gate_q.w)))
    return -1;
  float* logits = (float*)malloc(sizeof(float) * (size_t)(T * E));
  int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)(T * K));
  float* wts = (float*)malloc(sizeof(float) * (size_t)(T * K));
  uint16_t* y = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * K * d));
  uint16_t* sy = fs ? (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * d)) : NULL;
  float* sg = fs ? (float*)malloc(sizeof(float) * (size_t)T) : NULL;

  /* router: f32 Linear (f32 logits), or a QuantizedLinear or bf16 Linear
   * (router_bits 16; bf16 logits) */
  const int rb = blk->router_bits;
  /* the router in the matrix-core order (mfma_dot / mfma_dot_q) when asked */
  const int mf = blk->router_mfma && d % 64 == 0;
#pragma omp parallel for schedule(static) num_threads(nthreads)
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t e = 0; e < E; ++e) {
      float v;
      if (qr) {
        const int64_t gr = rb == 16 ? 0 : d / 64;  /* bf16 Linear: none */
        v = (mf ? mfma_dot_q : lane_dot_q)(x + t * d, blk->router_q.w + e * (d * rb / 32),
                                           rb == 16 ? NULL : blk->router_q.scales + e * gr,
                                           rb == 16 ? NULL : blk->router_q.biases + e * gr,
                                           d, rb);
      } else {
        v = mf ? mfma_dot(x + t * d, blk->router_w + e * d, d)
               : lane_dot(x + t * d, blk->router_w + e * d, d);
        if (blk->router_b) v += blk->router_b[e];
      }
      logits[t * E + e] = v;
    }
    if (fs)
      sg[t] = qr ? (mf ? mfma_dot_q : lane_dot_q)(x + t * d, blk->shared_gate_q.w,
                                                  blk->shared_gate_q.scales,
                                                  blk->shared_gate_q.biases, d, rb)
            : mf ? mfma_dot(x + t * d, blk->shared_gate_w, d)
                 : lane_dot(x + t * d, blk->shared_gate_w, d);
  }
  if (qr)
    orc_router_topk_bf16(logits, T, E, K, idx, wts);
  else
    orc_router_topk(logits, T, E, K, idx, wts);

  /* routed experts, one (token, k) pair at a time (gather_qmm's
   * unsorted path; the sorted path gives identical rows) */
  const int64_t fmax = fs > f ? fs : f;
#pragma omp parallel num_threads(nthreads)
  {
    float* xf = (float*)malloc(sizeof(float) * (size_t)d);
    float* af = (float*)malloc(sizeof(float) * (size_t)fmax);
    uint16_t* gb = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)fmax);
    uint16_t* ub = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)fmax);
    int64_t last_t = -1;
#pragma omp for schedule(dynamic, 1)
    for (int64_t tk = 0; tk < T * K; ++tk) {
      const int64_t t = tk / K;
      if (t != last_t) {
        for (int64_t j = 0; j < d; ++j) xf[j] = orc_bf16_to_f32(x[t * d + j]);
        last_t = t;
      }
      expert_ffn(xf, &blk->gate_proj, &blk->up_proj, &blk->down_proj,
                 idx[tk], d, f, gs, bits, blk->switch_tiled, y + tk * d, gb,
                 ub, af);
    }
    if (fs) {
#pragma omp for schedule(dynamic, 1)
      for (int64_t t = 0; t < T; ++t) {
        for (int64_t j = 0; j < d; ++j) xf[j] = orc_bf16_to_f32(x[t * d + j]);
        expert_ffn(xf, &blk->shared_gate, &blk->shared_up, &blk->shared_down,
                   0, d, fs, gs, bits, blk->shared_tiled, sy + t * d, gb, ub,
                   af);
      }
    }
    free(xf);
    free(af);
    free(gb);
    free(ub);
  }

  if (qr)
    orc_combine_bf16(y, wts, T, K, d, sy, sg, (uint16_t*)out);
  else
    orc_combine(y, wts, T, K, d, sy, sg, (float*)out);
  if (idx_out) memcpy(idx_out, idx, sizeof(int32_t) * (size_t)(T * K));
  if (w_out) memcpy(w_out, wts, sizeof(float) * (size_t)(T * K));
  free(logits);
  free(idx);
  free(wts);
  free(y);
  free(sy);
  free(sg);
  return 0;
}

/* The MoE half of a Qwen3.5 decoder layer (DecoderLayer::forward,
 * crates/mlxr-lm/src/qwen3_5/text/layer.rs:134-138):
 *   out = h + block(post_attention_layernorm(h))
 * with the norm fast::rms_norm (orc_rms_norm) and the add in the block
 * output's dtype: f32 = f32(h) + mlp_out, or bf16(h + mlp_out) with a bf16
 * router. */
int orc_block_forward_residual(const orc_block* blk, const uint16_t* norm_w,
                               float eps, const uint16_t* h, int64_t T,
                               void* out, int32_t* idx_out, float* w_out,
                               int nthreads) {
  const int64_t d = blk->hidden;
  const int bf16 = blk->router_q.w != NULL;
  uint16_t* normed = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * d));
  void* m = malloc((bf16 ? 2 : 4) * (size_t)(T * d));
  orc_rms_norm(h, T, d, norm_w, eps, normed);
  const int rc = orc_block_forward(blk, normed, T, m, idx_out, w_out, nthreads);
  if (rc == 0) {
    for (int64_t i = 0; i < T * d; ++i) {
      const float hv = orc_bf16_to_f32(h[i]);
      if (bf16)
        ((uint16_t*)out)[i] =
            orc_f32_to_bf16(hv + orc_bf16_to_f32(((const uint16_t*)m)[i]));
      else
        ((float*)out)[i] = hv + ((const float*)m)[i];
    }
  }
  free(normed);
  free(m);
  return rc;
}
