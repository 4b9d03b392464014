/*
 * q35_oracle.h -- CPU restatement of the Qwen3.5 hybrid-attention cores.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the HIP path is compared
 * against and the CPU baseline the benchmark times beside it; no product
 * code links it.  It restates, in plain C99, the semantics of
 *   src/attn_qwen.c  gqa_body          :235-397  (full-GQA core)
 *   src/attn_qwen.c  lin_body          :434-764  (gated delta-rule core,
 *                                                  scalar branch :657-717)
 *   src/attn_qwen.c  ds4f_attn_gqa_chunk    :1222-1231 (serial prefill body loop)
 *   src/attn_qwen.c  ds4f_attn_linear_chunk :1088-1109 (serial prefill body loop)
 * with the projections (MLX-4bit matvecs) removed: the callers hand in the
 * post-projection activations, exactly what the reference's bodies receive;
 * and the whole layer steps around them,
 *   src/attn_qwen.c  gqa_step          :87-225   (input norm, projections,
 *                                                  body, o_proj, residual)
 *   src/attn_qwen.c  linear_step       :837-968  (the same for a delta-rule
 *                                                  layer, with lin_body's
 *                                                  a / b and out projections)
 * on the MLX 4-bit matvec of src/kernels.c :118-219.
 * It is compiled with gcc -std=c99 -O2 (no -mfma), which on x86-64 gives the
 * same unfused float evaluation the reference's ISO-C scalar build has.
 */
#ifndef Q35_ORACLE_H
#define Q35_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 bits -> float (src/attn_qwen.c:42-47). */
float orc_bf16_f(uint16_t h);

/* In-place RMSNorm, double sum of squares, eps 1e-6 on the mean, x/r*w
 * (src/attn_qwen.c:50-55). */
void orc_rmsnorm(const uint16_t *w, int dim, float *x);

/* RoPE cos/sin of one position: rd/2 entries each, computed in double and
 * cast (src/attn_qwen.c:297-307; theta fixed at 1e7 there). */
void orc_rope_table(int token, int rd, double theta, float *cos_t, float *sin_t);

/* Full-GQA body for one token (src/attn_qwen.c:235-397).
 *   kv_layer : this layer's fp32 cache, [max_tokens][2*kv_heads*kh]
 *              (k rows first, then v rows; src/attn_qwen.c:329-331)
 *   q        : [heads][2*kh]  (q | gate per head), read only
 *   k        : [kv_heads][kh] normed + rotated IN PLACE (as the reference)
 *   v        : [kv_heads][kh]
 *   attn_out : [heads][kh]
 * Returns 0, or -1 on a geometry error.  token outside [0, max_tokens) is a
 * silent skip (returns 0 and writes nothing), as src/attn_qwen.c:256. */
int orc_gqa_body(int heads, int kv_heads, int kh, int max_tokens,
                 float *kv_layer, int token, const float *q, float *k,
                 const float *v, const uint16_t *qn_w, const uint16_t *kn_w,
                 float *attn_out);

/* Gated delta-rule body for one token, projections excluded
 * (src/attn_qwen.c:470-764, scalar branch).
 *   conv_ring : this layer's ring [4][qkv_rows], slot = token % 4
 *   S         : this layer's state [v_heads][kd][vd] (row i = key dim)
 *   qkv       : [qkv_rows] raw projection in; post-conv, normed values out
 *               (the reference mutates it in place: :503, :535)
 *   z         : [v_heads*vd]; a, b: [v_heads] (the in_proj_a / in_proj_b
 *               outputs the reference computes at :462-468)
 *   out       : [v_heads*vd] gated, normed readout (the o_proj input)
 * qkv_rows = 2*k_heads*kd + v_heads*vd; value head h uses key head h/2
 * (src/attn_qwen.c:658), so v_heads must equal 2*k_heads. */
int orc_lin_body(int k_heads, int v_heads, int kd, int vd, int token,
                 float *conv_ring, float *S, float *qkv, const float *z,
                 const float *a, const float *b, const uint16_t *conv_w,
                 const float *A_log, const uint16_t *dt_bias,
                 const uint16_t *norm_w, float *out);

/* The cache row gqa_body writes for `token` without the attention: k normed
 * (k_norm) and rotated in place (src/attn_qwen.c:292-293, :297-325), then
 * [k | v] copied to row_out [2*kv_heads*kh].  Lets a test build a long
 * cache cheaply and run orc_gqa_body only at sampled tokens. */
void orc_gqa_cache_row(int kv_heads, int kh, int token, float *k, const float *v,
                       const uint16_t *kn_w, float *row_out);

/* Serial prefill: orc_gqa_body for t = t0 .. t0+B-1 in order
 * (src/attn_qwen.c:1222-1231).  q: [B][heads*2*kh], k (in place), v:
 * [B][kv_heads*kh], attn_out: [B][heads*kh]. */
int orc_gqa_prefill(int heads, int kv_heads, int kh, int max_tokens,
                    float *kv_layer, int t0, int B, const float *q, float *k,
                    const float *v, const uint16_t *qn_w,
                    const uint16_t *kn_w, float *attn_out);

/* Serial prefill: orc_lin_body for t = t0 .. t0+B-1 in order
 * (src/attn_qwen.c:1088-1109).  qkv: [B][qkv_rows] (in place), z/out:
 * [B][v_heads*vd], a/b: [B][v_heads]. */
int orc_lin_prefill(int k_heads, int v_heads, int kd, int vd, int t0, int B,
                    float *conv_ring, float *S, float *qkv, const float *z,
                    const float *a, const float *b, const uint16_t *conv_w,
                    const float *A_log, const uint16_t *dt_bias,
                    const uint16_t *norm_w, float *out);

/* MLX 4-bit affine weights (src/kernels.c:104-136): U32 words of 8
 * nibbles, low nibble first, element k = (v[k/8] >> 4(k%8)) & 15 of the
 * row-major [R x C] matrix; BF16 scale and bias per 64 elements, group
 * g = k / 64 over the flattened index; w = q * scale + bias (no offset).
 * biases may be NULL (bias 0). */
void orc_mlx4_decode(const uint32_t *vals, const uint16_t *scales,
                     const uint16_t *biases, int n, float *out);

/* y[r] = sum_c w(r, c) x[c], the scalar path of ds4f_mlx4_matvec
 * (src/kernels.c:196-219): per-group LUT q * s + b, fp32 accumulation in
 * ascending c. */
void orc_mlx4_matvec(const uint32_t *vals, const uint16_t *scales,
                     const uint16_t *biases, int R, int C, const float *x, float *y);

/* One MLX 4-bit weight as mlx4_proj hands it to ds4f_mlx4_matvec
 * (src/attn_qwen.c:59-70): decoded shape rows x cols. */
typedef struct OrcMlx4 {
    const uint32_t *vals;
    const uint16_t *scales, *biases;
    int rows, cols;
} OrcMlx4;

/* Full-GQA layer step (gqa_step, src/attn_qwen.c:87-225) on the hidden
 * state [hidden], in place: xin = input_layernorm(state) (:142-157; in_norm
 * NULL: xin = state), q|gate, k, v = W xin (:160-165), the body (:172),
 * o = W_o attn_out (:196), state += o (:222).  The residual adds to the raw
 * state, the projections read the normed copy.  token outside
 * [0, max_tokens) is the silent skip of :117 (state untouched). */
int orc_gqa_step(int heads, int kv_heads, int kh, int max_tokens, float *kv_layer,
                 int token, int hidden, float *state, const uint16_t *in_norm,
                 const OrcMlx4 *wq, const OrcMlx4 *wk, const OrcMlx4 *wv,
                 const OrcMlx4 *wo, const uint16_t *qn_w, const uint16_t *kn_w);

/* Gated delta-rule layer step (linear_step, src/attn_qwen.c:837-968, with
 * lin_body's a / b projections :459-469 and out_proj + residual :771-776,
 * :832-833): xin = input_layernorm(state) (:913-928), qkv and z = W xin
 * (:932-948), a and b = W xin, the body, state += W_out out.  token
 * outside [0, max_tokens) is the silent skip of :882. */
int orc_lin_step(int k_heads, int v_heads, int kd, int vd, int max_tokens, int token,
                 int hidden, float *conv_ring, float *S, float *state,
                 const uint16_t *in_norm, const OrcMlx4 *wqkv, const OrcMlx4 *wz,
                 const OrcMlx4 *wa, const OrcMlx4 *wb, const OrcMlx4 *wout,
                 const uint16_t *conv_w, const float *A_log, const uint16_t *dt_bias,
                 const uint16_t *norm_w);

/* Prefill chunks on the residual stream: ds4f_attn_gqa_chunk
 * (src/attn_qwen.c:1145-1252) and ds4f_attn_linear_chunk (:977-1135).  The
 * reference batches the tokens' projections and output projections
 * (ds4f_mlx4_matvec_batch, the same per-row sums) and runs the bodies
 * serially in token order, so a chunk equals the layer steps of tokens
 * t0 .. t0+B-1 in order, each on its own state: states [B][hidden]. */
int orc_gqa_chunk(int heads, int kv_heads, int kh, int max_tokens, float *kv_layer, int t0,
                  int B, int hidden, float *states, const uint16_t *in_norm, const OrcMlx4 *wq,
                  const OrcMlx4 *wk, const OrcMlx4 *wv, const OrcMlx4 *wo,
                  const uint16_t *qn_w, const uint16_t *kn_w);
int orc_lin_chunk(int k_heads, int v_heads, int kd, int vd, int max_tokens, int t0, int B,
                  int hidden, float *conv_ring, float *S, float *states,
                  const uint16_t *in_norm, const OrcMlx4 *wqkv, const OrcMlx4 *wz,
                  const OrcMlx4 *wa, const OrcMlx4 *wb, const OrcMlx4 *wout,
                  const uint16_t *conv_w, const float *A_log, const uint16_t *dt_bias,
                  const uint16_t *norm_w);

#ifdef __cplusplus
}
#endif

#endif /* Q35_ORACLE_H */
