/*
 * q35_oracle.c -- CPU restatement of the Qwen3.5 hybrid-attention cores.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
 * baseline.  Nothing in the shipped library links or calls this file.
 *
 * Every floating-point expression keeps the reference's operand order and
 * types (float arithmetic, double sums of squares, division by r rather
 * than multiplication by 1/r, no fused multiply-add), because the point of
 * the restatement is to produce the numbers src/attn_qwen.c produces on an
 * x86-64 ISO-C build.  The control flow, buffers and names are this file's
 * own: the reference's shared scratch arena, getenv probes and debug dumps
 * are not part of the arithmetic and are left out.
 */
#include "q35_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define RING 4               /* conv taps, src/attn_qwen.c:424 (Q3_CONV_K) */
#define ROPE_THETA 10000000.0 /* src/attn_qwen.c:299 */

float orc_bf16_f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* sqrtf(mean(x^2) + 1e-6) with the square sum in double
 * (src/attn_qwen.c:51-53, :528-531, :729-732). */
static float rms_of(const float *x, int n) {
    double acc = 0.0;
    for (int i = 0; i < n; i++) acc += (double)x[i] * x[i];
    return sqrtf((float)(acc / (double)n) + 1e-6f);
}

void orc_rmsnorm(const uint16_t *w, int dim, float *x) {
    float r = rms_of(x, dim);
    for (int i = 0; i < dim; i++) x[i] = x[i] / r * orc_bf16_f(w[i]);
}

void orc_rope_table(int token, int rd, double theta, float *cos_t,
                    float *sin_t) {
    int half = rd / 2;
    for (int i = 0; i < half; i++) {
        double inv = 1.0 / pow(theta, (double)(2 * i) / (double)rd);
        double ang = (double)token * inv;
        cos_t[i] = (float)cos(ang);
        sin_t[i] = (float)sin(ang);
    }
}

/* Half-split rotation of dims (i, i+rd/2), i < rd/2 (src/attn_qwen.c:308-325). */
static void rope_rotate(float *x, int rd, const float *cos_t,
                        const float *sin_t) {
    int half = rd / 2;
    for (int i = 0; i < half; i++) {
        float lo = x[i], hi = x[i + half];
        float c = cos_t[i], s = sin_t[i];
        x[i] = lo * c - hi * s;
        x[i + half] = lo * s + hi * c;
    }
}

static float sigmoidf_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

int orc_gqa_body(int heads, int kv_heads, int kh, int max_tokens,
                 float *kv_layer, int token, const float *q, float *k,
                 const float *v, const uint16_t *qn_w, const uint16_t *kn_w,
                 float *attn_out) {
    if (heads < 1 || kv_heads < 1 || kh < 1 || heads % kv_heads != 0)
        return -1;
    if (token < 0 || !kv_layer || token >= max_tokens) return 0;
    int row = 2 * kv_heads * kh;          /* k rows then v rows per token */
    int group = heads / kv_heads;         /* q heads per kv head */
    int rd = (int)(kh * 0.25f);           /* src/attn_qwen.c:298 */
    int npos = token + 1;

    float *qn = (float *)malloc((size_t)heads * kh * sizeof(float));
    float *cs = (float *)malloc((size_t)(rd > 0 ? rd : 1) * sizeof(float));
    float *sc = (float *)malloc((size_t)npos * sizeof(float));
    float *wt = (float *)malloc((size_t)npos * sizeof(float));
    if (!qn || !cs || !sc || !wt) {
        free(qn); free(cs); free(sc); free(wt);
        return -1;
    }
    float *cos_t = cs, *sin_t = cs + rd / 2;

    /* q half of each head, normed (gate stays in q) */
    for (int h = 0; h < heads; h++) {
        memcpy(qn + (size_t)h * kh, q + (size_t)h * 2 * kh,
               (size_t)kh * sizeof(float));
        orc_rmsnorm(qn_w, kh, qn + (size_t)h * kh);
    }
    for (int g = 0; g < kv_heads; g++) orc_rmsnorm(kn_w, kh, k + (size_t)g * kh);

    orc_rope_table(token, rd, ROPE_THETA, cos_t, sin_t);
    for (int h = 0; h < heads; h++)
        rope_rotate(qn + (size_t)h * kh, rd, cos_t, sin_t);
    for (int g = 0; g < kv_heads; g++)
        rope_rotate(k + (size_t)g * kh, rd, cos_t, sin_t);

    float *dst = kv_layer + (size_t)token * row;
    memcpy(dst, k, (size_t)kv_heads * kh * sizeof(float));
    memcpy(dst + (size_t)kv_heads * kh, v, (size_t)kv_heads * kh * sizeof(float));

    float scale = 1.0f / sqrtf((float)kh);
    memset(attn_out, 0, (size_t)heads * kh * sizeof(float));
    for (int h = 0; h < heads; h++) {
        const float *qv = qn + (size_t)h * kh;
        int g = h / group;
        float mx = -1e30f;
        for (int p = 0; p < npos; p++) {
            const float *kp = kv_layer + (size_t)p * row + (size_t)g * kh;
            float dot = 0.0f;
            for (int i = 0; i < kh; i++) dot += qv[i] * kp[i];
            sc[p] = dot * scale;
            if (sc[p] > mx) mx = sc[p];
        }
        float den = 0.0f;
        for (int p = 0; p < npos; p++) {
            wt[p] = expf(sc[p] - mx);
            den += wt[p];
        }
        for (int p = 0; p < npos; p++) wt[p] /= den;
        float *o = attn_out + (size_t)h * kh;
        for (int p = 0; p < npos; p++) {
            const float *vp = kv_layer + (size_t)p * row +
                              (size_t)kv_heads * kh + (size_t)g * kh;
            float w = wt[p];
            for (int i = 0; i < kh; i++) o[i] += w * vp[i];
        }
    }
    /* output gate: the second kh of each q head (src/attn_qwen.c:387-395) */
    for (int h = 0; h < heads; h++) {
        const float *gt = q + (size_t)h * 2 * kh + kh;
        float *o = attn_out + (size_t)h * kh;
        for (int i = 0; i < kh; i++) o[i] *= sigmoidf_ref(gt[i]);
    }
    free(qn); free(cs); free(sc); free(wt);
    return 0;
}

int orc_lin_body(int k_heads, int v_heads, int kd, int vd, int token,
                 float *conv_ring, float *S, float *qkv, const float *z,
                 const float *a, const float *b, const uint16_t *conv_w,
                 const float *A_log, const uint16_t *dt_bias,
                 const uint16_t *norm_w, float *out) {
    if (k_heads < 1 || kd < 1 || vd < 1 || v_heads != 2 * k_heads) return -1;
    if (token < 0) return 0;
    int rows = 2 * k_heads * kd + v_heads * vd;

    /* 1. ring write of the raw row, then causal depthwise conv + SiLU;
     *    tap k = 0 is the oldest, taps before position 0 are skipped
     *    (src/attn_qwen.c:479-504). */
    memcpy(conv_ring + (size_t)(token % RING) * rows, qkv,
           (size_t)rows * sizeof(float));
    for (int c = 0; c < rows; c++) {
        float acc = 0.0f;
        for (int tap = 0; tap < RING; tap++) {
            int tp = token - (RING - 1 - tap);
            if (tp < 0) continue;
            acc += conv_ring[(size_t)(tp % RING) * rows + c] *
                   orc_bf16_f(conv_w[(size_t)c * RING + tap]);
        }
        qkv[c] = acc * sigmoidf_ref(acc);
    }

    /* 2. q/k RMS-normalisation per key head, q scaled 1/kd, k 1/sqrt(kd)
     *    (src/attn_qwen.c:522-538). */
    float qscale = 1.0f / (float)kd;
    float kscale = 1.0f / sqrtf((float)kd);
    for (int h = 0; h < k_heads; h++) {
        float *qv = qkv + (size_t)h * kd;
        float *kv = qkv + (size_t)k_heads * kd + (size_t)h * kd;
        float rq = rms_of(qv, kd);
        for (int i = 0; i < kd; i++) qv[i] = qv[i] / rq * qscale;
        float rk = rms_of(kv, kd);
        for (int i = 0; i < kd; i++) kv[i] = kv[i] / rk * kscale;
    }

    float *delta = (float *)malloc((size_t)vd * sizeof(float));
    if (!delta) return -1;
    for (int h = 0; h < v_heads; h++) {
        /* 3. log-decay g = -exp(A_log) * softplus(a + dt_bias), branch form
         *    of src/attn_qwen.c:545-551; beta = sigmoid(b) (:664). */
        float x = a[h] + orc_bf16_f(dt_bias[h]);
        float sp = x > 0 ? x + log1pf(expf(-x)) : log1pf(expf(x));
        float g = -expf(A_log[h]) * sp;
        float beta = sigmoidf_ref(b[h]);
        float decay = expf(g);

        const float *qh = qkv + (size_t)(h / 2) * kd;
        const float *kk = qkv + (size_t)k_heads * kd + (size_t)(h / 2) * kd;
        const float *vv = qkv + (size_t)2 * k_heads * kd + (size_t)h * vd;
        float *Sh = S + (size_t)h * kd * vd;

        /* 4. gated delta rule (src/attn_qwen.c:666-690), i ascending */
        for (int e = 0; e < kd * vd; e++) Sh[e] *= decay;
        for (int j = 0; j < vd; j++) {
            float mem = 0.0f;
            for (int i = 0; i < kd; i++) mem += Sh[(size_t)i * vd + j] * kk[i];
            delta[j] = (vv[j] - mem) * beta;
        }
        for (int i = 0; i < kd; i++) {
            float ki = kk[i];
            float *Srow = Sh + (size_t)i * vd;
            for (int j = 0; j < vd; j++) Srow[j] += ki * delta[j];
        }
        float *oh = out + (size_t)h * vd;
        for (int j = 0; j < vd; j++) {
            float acc = 0.0f;
            for (int i = 0; i < kd; i++) acc += Sh[(size_t)i * vd + j] * qh[i];
            oh[j] = acc;
        }
    }
    free(delta);

    /* 5. RMSNormGated, one weight vector shared by every head
     *    (src/attn_qwen.c:726-749): o/r * w * (z*sigmoid(z)). */
    for (int h = 0; h < v_heads; h++) {
        float *oh = out + (size_t)h * vd;
        const float *zh = z + (size_t)h * vd;
        float r = rms_of(oh, vd);
        for (int j = 0; j < vd; j++) {
            float zv = zh[j];
            float sg = sigmoidf_ref(zv);
            oh[j] = oh[j] / r * orc_bf16_f(norm_w[j]) * (zv * sg);
        }
    }
    return 0;
}

void orc_gqa_cache_row(int kv_heads, int kh, int token, float *k, const float *v,
                       const uint16_t *kn_w, float *row_out) {
    int rd = (int)(kh * 0.25f);
    float cs[128];
    float *cos_t = cs, *sin_t = cs + 64;
    for (int g = 0; g < kv_heads; g++) orc_rmsnorm(kn_w, kh, k + (size_t)g * kh);
    orc_rope_table(token, rd, ROPE_THETA, cos_t, sin_t);
    for (int g = 0; g < kv_heads; g++) rope_rotate(k + (size_t)g * kh, rd, cos_t, sin_t);
    memcpy(row_out, k, (size_t)kv_heads * kh * sizeof(float));
    memcpy(row_out + (size_t)kv_heads * kh, v, (size_t)kv_heads * kh * sizeof(float));
}

int orc_gqa_prefill(int heads, int kv_heads, int kh, int max_tokens,
                    float *kv_layer, int t0, int B, const float *q, float *k,
                    const float *v, const uint16_t *qn_w,
                    const uint16_t *kn_w, float *attn_out) {
    size_t qs = (size_t)heads * 2 * kh, ks = (size_t)kv_heads * kh;
    size_t os = (size_t)heads * kh;
    for (int t = 0; t < B; t++) {
        int rc = orc_gqa_body(heads, kv_heads, kh, max_tokens, kv_layer, t0 + t,
                              q + t * qs, k + t * ks, v + t * ks, qn_w, kn_w,
                              attn_out + t * os);
        if (rc != 0) return rc;
    }
    return 0;
}

int orc_lin_prefill(int k_heads, int v_heads, int kd, int vd, int t0, int B,
                    float *conv_ring, float *S, float *qkv, const float *z,
                    const float *a, const float *b, const uint16_t *conv_w,
                    const float *A_log, const uint16_t *dt_bias,
                    const uint16_t *norm_w, float *out) {
    size_t rows = (size_t)2 * k_heads * kd + (size_t)v_heads * vd;
    size_t zs = (size_t)v_heads * vd;
    for (int t = 0; t < B; t++) {
        int rc = orc_lin_body(k_heads, v_heads, kd, vd, t0 + t, conv_ring, S,
                              qkv + t * rows, z + t * zs, a + (size_t)t * v_heads,
                              b + (size_t)t * v_heads, conv_w, A_log, dt_bias,
                              norm_w, out + t * zs);
        if (rc != 0) return rc;
    }
    return 0;
}

/* ---- MLX 4-bit affine matvec (src/kernels.c:118-136, :196-219) ---- */

static void mlx4_lut(const uint16_t *scales, const uint16_t *biases, long g, float lut[16]) {
    const float sc = orc_bf16_f(scales[g]);
    const float bi = biases ? orc_bf16_f(biases[g]) : 0.0f;
    for (int q = 0; q < 16; q++) lut[q] = (float)q * sc + bi;
}

void orc_mlx4_decode(const uint32_t *vals, const uint16_t *scales,
                     const uint16_t *biases, int n, float *out) {
    float lut[16];
    long gcur = -1;
    for (int k = 0; k < n; k++) {
        const long g = k / 64;
        if (g != gcur) {
            gcur = g;
            mlx4_lut(scales, biases, g, lut);
        }
        out[k] = lut[(vals[k >> 3] >> (4 * (k & 7))) & 0xFu];
    }
}

void orc_mlx4_matvec(const uint32_t *vals, const uint16_t *scales,
                     const uint16_t *biases, int R, int C, const float *x, float *y) {
    float lut[16];
    long gcur = -1;
    for (int r = 0; r < R; r++) {
        float acc = 0.0f;
        for (int c = 0; c < C; c++) {
            const long k = (long)r * C + c, g = k / 64;
            if (g != gcur) {
                gcur = g;
                mlx4_lut(scales, biases, g, lut);
            }
            acc += lut[(vals[k >> 3] >> (4 * (int)(k & 7))) & 0xFu] * x[c];
        }
        y[r] = acc;
    }
}

/* mlx4_proj (src/attn_qwen.c:59-70): y = W x, W rows x cols */
static void mlx4_proj(const OrcMlx4 *w, const float *x, float *y) {
    orc_mlx4_matvec(w->vals, w->scales, w->biases, w->rows, w->cols, x, y);
}

/* xin = input_layernorm(state), or a copy without a norm weight
 * (src/attn_qwen.c:142-159, :913-930) */
static void input_norm(const float *state, const uint16_t *in_norm, int hidden, float *xin) {
    memcpy(xin, state, (size_t)hidden * sizeof(float));
    if (in_norm) orc_rmsnorm(in_norm, hidden, xin);
}

int orc_gqa_step(int heads, int kv_heads, int kh, int max_tokens, float *kv_layer,
                 int token, int hidden, float *state, const uint16_t *in_norm,
                 const OrcMlx4 *wq, const OrcMlx4 *wk, const OrcMlx4 *wv,
                 const OrcMlx4 *wo, const uint16_t *qn_w, const uint16_t *kn_w) {
    if (wq->rows != heads * 2 * kh || wk->rows != kv_heads * kh || wv->rows != kv_heads * kh ||
        wq->cols != hidden || wk->cols != hidden || wv->cols != hidden ||
        wo->cols != heads * kh || wo->rows != hidden)
        return -1;                                   /* :108-115 */
    if (token < 0 || token >= max_tokens) return 0;  /* :117 */
    float *xin = malloc((size_t)hidden * sizeof(float));
    float *q = malloc((size_t)wq->rows * sizeof(float));
    float *k = malloc((size_t)wk->rows * sizeof(float));
    float *v = malloc((size_t)wv->rows * sizeof(float));
    float *ao = malloc((size_t)heads * kh * sizeof(float));
    float *o = malloc((size_t)hidden * sizeof(float));
    int rc = -1;
    if (xin && q && k && v && ao && o) {
        input_norm(state, in_norm, hidden, xin);
        mlx4_proj(wq, xin, q);                       /* :160-165 */
        mlx4_proj(wk, xin, k);
        mlx4_proj(wv, xin, v);
        rc = orc_gqa_body(heads, kv_heads, kh, max_tokens, kv_layer, token, q, k, v, qn_w, kn_w, ao);
        if (rc == 0) {
            mlx4_proj(wo, ao, o);                    /* :196 */
            for (int i = 0; i < hidden; i++) state[i] += o[i];   /* :222 */
        }
    }
    free(xin);
    free(q);
    free(k);
    free(v);
    free(ao);
    free(o);
    return rc;
}

int orc_lin_step(int k_heads, int v_heads, int kd, int vd, int max_tokens, int token,
                 int hidden, float *conv_ring, float *S, float *state,
                 const uint16_t *in_norm, const OrcMlx4 *wqkv, const OrcMlx4 *wz,
                 const OrcMlx4 *wa, const OrcMlx4 *wb, const OrcMlx4 *wout,
                 const uint16_t *conv_w, const float *A_log, const uint16_t *dt_bias,
                 const uint16_t *norm_w) {
    const int qkv_rows = 2 * k_heads * kd + v_heads * vd;
    if (wqkv->rows != qkv_rows || wz->rows != v_heads * vd || wout->rows != hidden ||
        wa->rows != v_heads || wb->rows != v_heads || wqkv->cols != hidden ||
        wz->cols != hidden || wa->cols != hidden || wb->cols != hidden ||
        wout->cols != v_heads * vd)
        return -1;                                   /* :870-879 */
    if (token < 0 || token >= max_tokens) return 0;  /* :882 */
    float *xin = malloc((size_t)hidden * sizeof(float));
    float *qkv = malloc((size_t)qkv_rows * sizeof(float));
    float *z = malloc((size_t)v_heads * vd * sizeof(float));
    float *a = malloc((size_t)v_heads * sizeof(float));
    float *b = malloc((size_t)v_heads * sizeof(float));
    float *out = malloc((size_t)v_heads * vd * sizeof(float));
    float *o = malloc((size_t)hidden * sizeof(float));
    int rc = -1;
    if (xin && qkv && z && a && b && out && o) {
        input_norm(state, in_norm, hidden, xin);
        mlx4_proj(wqkv, xin, qkv);                   /* :932-948 */
        mlx4_proj(wz, xin, z);
        mlx4_proj(wa, xin, a);                       /* :459-469 */
        mlx4_proj(wb, xin, b);
        rc = orc_lin_body(k_heads, v_heads, kd, vd, token, conv_ring, S, qkv, z, a, b, conv_w,
                          A_log, dt_bias, norm_w, out);
        if (rc == 0) {
            mlx4_proj(wout, out, o);                 /* :771-776 */
            for (int i = 0; i < hidden; i++) state[i] += o[i];   /* :832-833 */
        }
    }
    free(xin);
    free(qkv);
    free(z);
    free(a);
    free(b);
    free(out);
    free(o);
    return rc;
}

int orc_gqa_chunk(int heads, int kv_heads, int kh, int max_tokens, float *kv_layer, int t0,
                  int B, int hidden, float *states, const uint16_t *in_norm, const OrcMlx4 *wq,
                  const OrcMlx4 *wk, const OrcMlx4 *wv, const OrcMlx4 *wo,
                  const uint16_t *qn_w, const uint16_t *kn_w) {
    if (B < 1 || t0 < 0) return -1;                  /* :1162-1163 */
    for (int b = 0; b < B; b++) {
        const int rc = orc_gqa_step(heads, kv_heads, kh, max_tokens, kv_layer, t0 + b, hidden,
                                    states + (size_t)b * hidden, in_norm, wq, wk, wv, wo, qn_w,
                                    kn_w);
        if (rc != 0) return rc;
    }
    return 0;
}

int orc_lin_chunk(int k_heads, int v_heads, int kd, int vd, int max_tokens, int t0, int B,
                  int hidden, float *conv_ring, float *S, float *states,
                  const uint16_t *in_norm, const OrcMlx4 *wqkv, const OrcMlx4 *wz,
                  const OrcMlx4 *wa, const OrcMlx4 *wb, const OrcMlx4 *wout,
                  const uint16_t *conv_w, const float *A_log, const uint16_t *dt_bias,
                  const uint16_t *norm_w) {
    if (B < 1 || t0 < 0) return -1;
    for (int b = 0; b < B; b++) {                    /* token order, :1088-1109 */
        const int rc = orc_lin_step(k_heads, v_heads, kd, vd, max_tokens, t0 + b, hidden,
                                    conv_ring, S, states + (size_t)b * hidden, in_norm, wqkv, wz,
                                    wa, wb, wout, conv_w, A_log, dt_bias, norm_w);
        if (rc != 0) return rc;
    }
    return 0;
}

