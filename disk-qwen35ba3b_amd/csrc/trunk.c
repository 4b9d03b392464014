/*
 * trunk.c -- a layer's attention weights from the engine's packed trunk.
 *
 * The engine keeps one tensor list per layer, parsed from trunk.json by
 * ds4f_trunk_layout_load (src/moe.c:162-520) into Ds4fTrunkTensor entries
 * (include/ds4f/moe.h:49-56: name, dtype code, dims, rank, byte offset in
 * the layer payload, size), and the layer payload itself, the layer's bytes
 * of trunk.bin (written by tools/build-trunk-mlx.py:95-160: tensors sorted
 * by name, 8-byte aligned).  The functions here take that list and payload
 * as they are and resolve the roles the attention steps read, by the same
 * name suffixes as the reference (first match wins, src/moe.c:425-490),
 * into a Ds4fGpuLayerW for ds4f_gpu_attn_weights.  A layer that lacks a
 * role its step requires is skipped by every later step and chunk, as
 * gqa_step / linear_step skip it (src/attn_qwen.c:96-97, :849-856).
 *
 * MLX 4-bit weights are U32 tensors of shape [rows, cols / 8]: the decoded
 * column count is dims[1] * 8 (src/attn_qwen.c:103-105), with BF16 scales
 * and biases of 64-element groups.
 */
#include "ds4f_gpu_attn.h"

#include <stdio.h>
#include <string.h>

/* the reference's dtype codes (src/moe.c:36-42) */
enum { DT_F32 = 0, DT_BF16 = 4, DT_U32 = 5 };

/* the plugin's error text and its incomplete-layer mark (gpu_hip.c) */
void ds4f_plugin_set_err(const char *msg) __attribute__((visibility("hidden")));
int ds4f_plugin_layer_skip(int L) __attribute__((visibility("hidden")));

static int ends_with(const char *s, const char *suffix) {
    const size_t cap = sizeof(((Ds4fGpuTrunkTensor *)0)->name);
    const char *z = (const char *)memchr(s, 0, cap);
    const size_t n = z ? (size_t)(z - s) : cap, m = strlen(suffix);
    return n >= m && memcmp(s + n - m, suffix, m) == 0;
}

/* role suffixes: an MLX triplet is ".weight", ".scales", ".biases" */
typedef struct { const char *suffix; int *slot; } RoleName;

int ds4f_gpu_trunk_roles(const Ds4fGpuTrunkTensor *t, int n, Ds4fGpuTrunkRoles *r) {
    if (!r || n < 0 || (n > 0 && !t)) return -1;
    int *all = (int *)r;
    for (size_t i = 0; i < sizeof *r / sizeof(int); i++) all[i] = -1;
    const RoleName names[] = {
        {".attn_norm.weight", &r->in_norm}, {".input_layernorm.weight", &r->in_norm},
        {".self_attn.q_proj.weight", &r->q[0]}, {".self_attn.q_proj.scales", &r->q[1]},
        {".self_attn.q_proj.biases", &r->q[2]},
        {".self_attn.k_proj.weight", &r->k[0]}, {".self_attn.k_proj.scales", &r->k[1]},
        {".self_attn.k_proj.biases", &r->k[2]},
        {".self_attn.v_proj.weight", &r->v[0]}, {".self_attn.v_proj.scales", &r->v[1]},
        {".self_attn.v_proj.biases", &r->v[2]},
        {".self_attn.o_proj.weight", &r->o[0]}, {".self_attn.o_proj.scales", &r->o[1]},
        {".self_attn.o_proj.biases", &r->o[2]},
        {".self_attn.q_norm.weight", &r->q_norm}, {".self_attn.k_norm.weight", &r->k_norm},
        {".linear_attn.conv1d.weight", &r->conv}, {".linear_attn.A_log", &r->A_log},
        {".linear_attn.dt_bias", &r->dt_bias},
        {".linear_attn.in_proj_qkv.weight", &r->qkv[0]},
        {".linear_attn.in_proj_qkv.scales", &r->qkv[1]},
        {".linear_attn.in_proj_qkv.biases", &r->qkv[2]},
        {".linear_attn.in_proj_z.weight", &r->z[0]}, {".linear_attn.in_proj_z.scales", &r->z[1]},
        {".linear_attn.in_proj_z.biases", &r->z[2]},
        {".linear_attn.in_proj_a.weight", &r->a[0]}, {".linear_attn.in_proj_a.scales", &r->a[1]},
        {".linear_attn.in_proj_a.biases", &r->a[2]},
        {".linear_attn.in_proj_b.weight", &r->b[0]}, {".linear_attn.in_proj_b.scales", &r->b[1]},
        {".linear_attn.in_proj_b.biases", &r->b[2]},
        {".linear_attn.out_proj.weight", &r->out[0]},
        {".linear_attn.out_proj.scales", &r->out[1]},
        {".linear_attn.out_proj.biases", &r->out[2]},
        {".linear_attn.norm.weight", &r->norm},
    };
    for (int i = 0; i < n; i++)
        for (size_t j = 0; j < sizeof names / sizeof names[0]; j++)
            if (ends_with(t[i].name, names[j].suffix)) {
                if (*names[j].slot < 0) *names[j].slot = i;
                break;
            }
    /* the layer dispatch of ds4f_attn_qwen_step (src/attn_qwen.c:1259-1263) */
    if (r->q[0] >= 0) return DS4F_LAYER_GQA;
    if (r->conv >= 0 || r->qkv[0] >= 0) return DS4F_LAYER_LINEAR;
    return DS4F_LAYER_NONE;
}

static char trunk_err[256];

/* a role's payload holds at least `bytes` (what the upload copies) */
static int holds(const Ds4fGpuTrunkTensor *t, int i, long bytes, const char *what) {
    if (t[i].nbytes < bytes) {
        snprintf(trunk_err, sizeof trunk_err, "trunk: role %s holds %ld bytes, needs %ld", what,
                 t[i].nbytes, bytes);
        return 0;
    }
    return 1;
}

static int need(const Ds4fGpuTrunkTensor *t, int i, int dtype, int rank, const char *what) {
    if (i < 0) {
        snprintf(trunk_err, sizeof trunk_err, "trunk: role %s missing", what);
        return 0;
    }
    if (t[i].dtype != dtype || (rank > 0 && t[i].rank < rank) || t[i].off < 0 ||
        (dtype == DT_F32 && (t[i].off & 3)) || ((dtype == DT_BF16 || dtype == DT_U32) && (t[i].off & 1))) {
        snprintf(trunk_err, sizeof trunk_err, "trunk: role %s (%s) has dtype %d rank %d off %ld",
                 what, t[i].name, t[i].dtype, t[i].rank, t[i].off);
        return 0;
    }
    return 1;
}

/* an MLX triplet: U32 [rows, cols / 8] words, BF16 scales, optional biases */
static int mlx4(const Ds4fGpuTrunkTensor *t, const int *ix, const uint8_t *tr, Ds4fGpuMlx4W *w,
                const char *what) {
    if (!need(t, ix[0], DT_U32, 2, what) || !need(t, ix[1], DT_BF16, 1, what)) return 0;
    if (ix[2] >= 0 && !need(t, ix[2], DT_BF16, 1, what)) return 0;
    w->vals = (const uint32_t *)(const void *)(tr + t[ix[0]].off);
    w->scales = (const uint16_t *)(const void *)(tr + t[ix[1]].off);
    w->biases = ix[2] >= 0 ? (const uint16_t *)(const void *)(tr + t[ix[2]].off) : NULL;
    w->rows = (int)t[ix[0]].dims[0];
    w->cols = (int)t[ix[0]].dims[1] * 8;
    const long groups = ((long)w->rows * w->cols + 63) / 64;
    if (t[ix[0]].nbytes < (long)w->rows * w->cols / 2 || t[ix[1]].nbytes < 2 * groups ||
        (ix[2] >= 0 && t[ix[2]].nbytes < 2 * groups)) {
        snprintf(trunk_err, sizeof trunk_err, "trunk: role %s sizes do not match its shape", what);
        return 0;
    }
    return 1;
}

int ds4f_gpu_attn_weights_trunk(int L, const Ds4fGpuTrunkTensor *t, int n, const uint8_t *tr) {
    Ds4fGpuTrunkRoles r;
    const int kind = ds4f_gpu_trunk_roles(t, n, &r);
    if (kind < 0 || !tr) return -1;
    if (kind == DS4F_LAYER_NONE) return 0;           /* no attention roles: nothing to upload */
    /* the roles whose absence makes gqa_step / linear_step skip the layer
     * (src/attn_qwen.c:96-97, :849-856: "incomplete graph: skip") */
    const int complete = kind == DS4F_LAYER_GQA
        ? r.q[0] >= 0 && r.k[0] >= 0 && r.v[0] >= 0 && r.o[0] >= 0 && r.q_norm >= 0 && r.k_norm >= 0
        : r.qkv[0] >= 0 && r.z[0] >= 0 && r.a[0] >= 0 && r.b[0] >= 0 && r.conv >= 0 &&
              r.out[0] >= 0 && r.norm >= 0 && r.A_log >= 0 && r.dt_bias >= 0;
    if (!complete) return ds4f_plugin_layer_skip(L);
    Ds4fGpuLayerW w;
    memset(&w, 0, sizeof w);
    trunk_err[0] = 0;
    int ok = 1;
    if (kind == DS4F_LAYER_GQA) {
        /* q_norm / k_norm: one head of the plugin's head dim (256) */
        ok = mlx4(t, r.q, tr, &w.q, "q_proj") && mlx4(t, r.k, tr, &w.k, "k_proj") &&
             mlx4(t, r.v, tr, &w.v, "v_proj") && mlx4(t, r.o, tr, &w.o, "o_proj") &&
             need(t, r.q_norm, DT_BF16, 1, "q_norm") && need(t, r.k_norm, DT_BF16, 1, "k_norm") &&
             holds(t, r.q_norm, 2L * 256, "q_norm") && holds(t, r.k_norm, 2L * 256, "k_norm");
        if (ok) {
            w.q_norm = (const uint16_t *)(const void *)(tr + t[r.q_norm].off);
            w.k_norm = (const uint16_t *)(const void *)(tr + t[r.k_norm].off);
        }
    } else {
        ok = mlx4(t, r.qkv, tr, &w.qkv, "in_proj_qkv") && mlx4(t, r.z, tr, &w.z, "in_proj_z") &&
             mlx4(t, r.a, tr, &w.a, "in_proj_a") && mlx4(t, r.b, tr, &w.b, "in_proj_b") &&
             mlx4(t, r.out, tr, &w.out, "out_proj") && need(t, r.conv, DT_BF16, 2, "conv1d") &&
             need(t, r.A_log, DT_F32, 1, "A_log") && need(t, r.dt_bias, DT_BF16, 1, "dt_bias") &&
             need(t, r.norm, DT_BF16, 1, "norm") && w.a.rows > 0 &&
             holds(t, r.conv, 2L * 4 * w.qkv.rows, "conv1d") &&
             holds(t, r.A_log, 4L * w.a.rows, "A_log") && holds(t, r.dt_bias, 2L * w.a.rows, "dt_bias") &&
             holds(t, r.norm, 2L * w.z.rows / w.a.rows, "norm");
        if (ok) {
            w.conv_w = (const uint16_t *)(const void *)(tr + t[r.conv].off);
            w.A_log = (const float *)(const void *)(tr + t[r.A_log].off);
            w.dt_bias = (const uint16_t *)(const void *)(tr + t[r.dt_bias].off);
            w.norm_w = (const uint16_t *)(const void *)(tr + t[r.norm].off);
        }
    }
    if (ok && r.in_norm >= 0) {
        const int hidden = kind == DS4F_LAYER_GQA ? w.q.cols : w.qkv.cols;
        ok = need(t, r.in_norm, DT_BF16, 1, "input_layernorm") &&
             holds(t, r.in_norm, 2L * hidden, "input_layernorm");
        if (ok) w.in_norm = (const uint16_t *)(const void *)(tr + t[r.in_norm].off);
    }
    if (!ok) {
        char msg[300];
        snprintf(msg, sizeof msg, "layer %d: %s", L, trunk_err);
        ds4f_plugin_set_err(msg);
        return -1;
    }
    return ds4f_gpu_attn_weights(L, &w);
}
