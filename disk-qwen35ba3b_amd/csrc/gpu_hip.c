/*
 * gpu_hip.c -- the HIP attention plugin: a C99 sibling of the reference's
 * src/gpu_stub.c and src/gpu_metal.mm, exporting include/ds4f_gpu_attn.h.
 *
 * It owns the device mirrors of the engine's attention state (the
 * Ds4fKvCache arrays of include/ds4f/attn.h:26-42), one HIP stream, and the
 * staging buffers of the host-pointer entry points, and it applies the
 * plugin conventions of include/ds4f/gpu.h:20-21 and src/head.c:271-283:
 * lazy init, 0 = done, -1 = fall back to the CPU, sticky disable after the
 * first failure with the device state written back to the bound host
 * arrays first so the CPU path continues from exactly the same state.
 *
 * Kernels live in the .hip files next to this one (q35_launch.h).
 */
#include "ds4f_gpu_attn.h"
#include "q35_launch.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define GQA_D 256
#define GQA_GROUP 8
#define ROPE_DIMS 64
#define ROPE_THETA 10000000.0 /* src/attn_qwen.c:299 */
#define KV_CHUNK_ROWS 4096    /* host<->device KV staging granularity */

static struct Plugin {
    int tried, ok, disabled;
    hipStream_t stream;
    char err[256];
    int fail_countdown;        /* DS4F_GPU_FAIL_AFTER: forced failure */

    int bound;
    Ds4fGpuAttnGeom g;
    int *kind, *slot;
    int n_gqa, n_lin;
    int t_pad, t_tiles;
    int rows, vh, kd, vd;
    size_t kv_elems;           /* per GQA layer, per K or V plane */
    uint16_t *d_k, *d_v;
    float *d_lin, *d_conv, *d_rope;
    float *d_part_o, *d_part_ml;
    float *host_kv, *host_lin, *host_conv;

    void *d_stage, *h_stage;
    size_t d_stage_cap, h_stage_cap;
    void *d_ws;                /* prefill workspaces (grow-only) */
    size_t ws_cap;

    /* whole-layer steps: per-layer device weights, the activations between
     * their launches, a device copy of the host state */
    int hidden;
    struct LayerW *lw;         /* [n_layers] */
    float *d_act, *d_state;
    /* whole-layer chunks: X operands and projection outputs */
    void *d_chunk;
    int chunk_cap;             /* token rows (a multiple of the GEMM's M tile) */
    float *h_states;           /* pinned staging of the host chunk entry */
    size_t h_states_cap;
    int scratch_rc;            /* q35_lin_scratch_init's result at init */
    int *d_status, *h_status;  /* the prefill kernels' status words (Q35_STATUS_*): [0] the
                                  device-pointer callers', [HOST_WORD] the host entries' */
    int *d_status_cur;         /* the word the next prefill launch sets */
    float *d_backup;           /* a delta-rule layer's state and ring before a chunk */
} P;

static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(P.err, sizeof P.err, fmt, ap);
    va_end(ap);
}

const char *ds4f_gpu_last_error(void) { return P.err; }

/* for the plugin's other translation units (trunk.c) */
__attribute__((visibility("hidden"))) void ds4f_plugin_set_err(const char *msg) {
    set_err("%s", msg);
}

static void mlx4_free(void);
static void layers_free(void);

#define HIPCHK(call)                                                              \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess) {                                                   \
            set_err("%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__,     \
                    __LINE__);                                                    \
            return -1;                                                            \
        }                                                                         \
    } while (0)

int ds4f_gpu_init(void) {
    if (P.tried) return P.ok ? 0 : -1;
    P.tried = 1;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        set_err("no HIP device");
        return -1;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) {
        set_err("hipGetDeviceProperties failed");
        return -1;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_err("device is %s, kernels are built for gfx950", prop.gcnArchName);
        return -1;
    }
    if (hipSetDevice(0) != hipSuccess ||
        hipStreamCreateWithFlags(&P.stream, hipStreamNonBlocking) != hipSuccess) {
        set_err("stream creation failed");
        return -1;
    }
    const char *f = getenv("DS4F_GPU_FAIL_AFTER");
    P.fail_countdown = f ? atoi(f) : -1;
    /* the device address of the no-allocation entry's static workspace, on
     * this device; a failure here only disables that entry */
    P.scratch_rc = (int)q35_lin_scratch_init();
    if (hipMalloc((void **)&P.d_status, 256) != hipSuccess ||
        hipHostMalloc((void **)&P.h_status, 256, hipHostMallocDefault) != hipSuccess ||
        hipMemset(P.d_status, 0, 256) != hipSuccess) {
        set_err("status word allocation failed");
        return -1;
    }
    P.d_status_cur = P.d_status;
    P.ok = 1;
    return 0;
}

static void free_binding(void) {
    layers_free();
    if (P.d_k) hipFree(P.d_k);
    if (P.d_v) hipFree(P.d_v);
    if (P.d_lin) hipFree(P.d_lin);
    if (P.d_conv) hipFree(P.d_conv);
    if (P.d_rope) hipFree(P.d_rope);
    if (P.d_part_o) hipFree(P.d_part_o);
    if (P.d_part_ml) hipFree(P.d_part_ml);
    if (P.d_backup) hipFree(P.d_backup);
    free(P.kind);
    free(P.slot);
    P.d_backup = NULL;
    P.d_k = P.d_v = NULL;
    P.d_lin = P.d_conv = P.d_rope = P.d_part_o = P.d_part_ml = NULL;
    P.kind = P.slot = NULL;
    P.bound = 0;
}

void ds4f_gpu_free(void) {
    if (!P.ok) return;
    hipStreamSynchronize(P.stream);
    free_binding();
    if (P.d_stage) hipFree(P.d_stage);
    if (P.h_stage) hipHostFree(P.h_stage);
    if (P.d_ws) hipFree(P.d_ws);
    if (P.d_status) hipFree(P.d_status);
    if (P.h_status) hipHostFree(P.h_status);
    mlx4_free();
    hipStreamDestroy(P.stream);
    memset(&P, 0, sizeof P);
}

int ds4f_gpu_attn_unbind(void) {
    if (!P.ok) return -1;
    hipStreamSynchronize(P.stream);
    free_binding();
    return 0;
}

static int ensure_stage(size_t dbytes, size_t hbytes) {
    if (dbytes > P.d_stage_cap) {
        if (P.d_stage) hipFree(P.d_stage);
        P.d_stage = NULL;
        P.d_stage_cap = 0;
        HIPCHK(hipMalloc(&P.d_stage, dbytes));
        P.d_stage_cap = dbytes;
    }
    if (hbytes > P.h_stage_cap) {
        if (P.h_stage) hipHostFree(P.h_stage);
        P.h_stage = NULL;
        P.h_stage_cap = 0;
        HIPCHK(hipHostMalloc(&P.h_stage, hbytes, 0));
        P.h_stage_cap = hbytes;
    }
    return 0;
}

/* the prefill workspace: grow-only, by at least half its size, so a
 * sequence of growing requests reallocates a few times, not every call */
static int ensure_ws(size_t bytes) {
    if (bytes <= P.ws_cap) return 0;
    const size_t want = bytes > P.ws_cap + P.ws_cap / 2 ? bytes : P.ws_cap + P.ws_cap / 2;
    if (P.d_ws) {
        HIPCHK(hipStreamSynchronize(P.stream));
        hipFree(P.d_ws);
    }
    P.d_ws = NULL;
    P.ws_cap = 0;
    HIPCHK(hipMalloc(&P.d_ws, want));
    P.ws_cap = want;
    return 0;
}

static size_t kv_row_floats(void) { return (size_t)2 * P.g.n_kv_heads * P.g.head_dim; }
static size_t lin_floats(void) { return (size_t)P.vh * P.kd * P.vd; }
static size_t conv_floats(void) { return (size_t)4 * P.rows; }

static uint16_t *layer_k(int s) { return P.d_k + (size_t)s * P.kv_elems; }
static uint16_t *layer_v(int s) { return P.d_v + (size_t)s * P.kv_elems; }
static float *layer_lin(int s) { return P.d_lin + (size_t)s * lin_floats(); }
static float *layer_conv(int s) { return P.d_conv + (size_t)s * conv_floats(); }

/* One layer, one direction, synchronous. */
static int sync_layer(int L, int dir, int n_tokens) {
    int s = P.slot[L];
    if (P.kind[L] == DS4F_LAYER_GQA && P.host_kv) {
        size_t rf = kv_row_floats();
        if (n_tokens > P.g.max_tokens) n_tokens = P.g.max_tokens;
        if (ensure_stage((size_t)KV_CHUNK_ROWS * rf * sizeof(float), 0) != 0) return -1;
        float *host = P.host_kv + (size_t)L * P.g.max_tokens * rf;
        for (int p0 = 0; p0 < n_tokens; p0 += KV_CHUNK_ROWS) {
            int n = n_tokens - p0 < KV_CHUNK_ROWS ? n_tokens - p0 : KV_CHUNK_ROWS;
            size_t bytes = (size_t)n * rf * sizeof(float);
            if (dir == DS4F_SYNC_TO_DEVICE) {
                HIPCHK(hipMemcpyAsync(P.d_stage, host + (size_t)p0 * rf, bytes,
                                      hipMemcpyHostToDevice, P.stream));
                HIPCHK(q35_kv_import((const float *)P.d_stage, p0, n, layer_k(s), layer_v(s),
                                     P.t_tiles, P.g.n_kv_heads, P.stream));
            } else {
                HIPCHK(q35_kv_export((float *)P.d_stage, p0, n, layer_k(s), layer_v(s),
                                     P.t_tiles, P.g.n_kv_heads, P.stream));
                HIPCHK(hipMemcpyAsync(host + (size_t)p0 * rf, P.d_stage, bytes,
                                      hipMemcpyDeviceToHost, P.stream));
            }
            HIPCHK(hipStreamSynchronize(P.stream));
        }
    } else if (P.kind[L] == DS4F_LAYER_LINEAR) {
        if (P.host_lin) {
            size_t bytes = lin_floats() * sizeof(float);
            if (ensure_stage(bytes, 0) != 0) return -1;
            float *host = P.host_lin + (size_t)L * lin_floats();
            if (dir == DS4F_SYNC_TO_DEVICE) {
                HIPCHK(hipMemcpyAsync(P.d_stage, host, bytes, hipMemcpyHostToDevice, P.stream));
                HIPCHK(q35_state_transpose((const float *)P.d_stage, layer_lin(s), P.vh, P.kd,
                                           P.vd, P.stream));
            } else {
                HIPCHK(q35_state_transpose(layer_lin(s), (float *)P.d_stage, P.vh, P.vd, P.kd,
                                           P.stream));
                HIPCHK(hipMemcpyAsync(host, P.d_stage, bytes, hipMemcpyDeviceToHost, P.stream));
            }
            HIPCHK(hipStreamSynchronize(P.stream));
        }
        if (P.host_conv) {
            size_t bytes = conv_floats() * sizeof(float);
            float *host = P.host_conv + (size_t)L * conv_floats();
            if (dir == DS4F_SYNC_TO_DEVICE)
                HIPCHK(hipMemcpyAsync(layer_conv(s), host, bytes, hipMemcpyHostToDevice,
                                      P.stream));
            else
                HIPCHK(hipMemcpyAsync(host, layer_conv(s), bytes, hipMemcpyDeviceToHost,
                                      P.stream));
            HIPCHK(hipStreamSynchronize(P.stream));
        }
    }
    return 0;
}

int ds4f_gpu_attn_sync(int L, int dir, int n_kv_tokens) {
    if (!P.ok || !P.bound) {
        set_err("plugin not bound");
        return -1;
    }
    if (L >= P.g.n_layers) {
        set_err("sync: layer %d outside [0, %d)", L, P.g.n_layers);
        return -1;
    }
    int lo = L < 0 ? 0 : L, hi = L < 0 ? P.g.n_layers : L + 1;
    for (int l = lo; l < hi; l++)
        if (sync_layer(l, dir, n_kv_tokens) != 0) return -1;
    return 0;
}

/* Sticky fallback: write the device state back, then disable. */
static int fail_over(int n_kv_tokens) {
    char saved[256];
    memcpy(saved, P.err, sizeof saved);
    if (P.ok && P.bound) {
        hipStreamSynchronize(P.stream);
        for (int l = 0; l < P.g.n_layers; l++) sync_layer(l, DS4F_SYNC_TO_HOST, n_kv_tokens);
    }
    memcpy(P.err, saved, sizeof saved);
    P.disabled = 1;
    fprintf(stderr, "ds4f gpu: attention plugin disabled, CPU fallback (%s)\n", P.err);
    return -1;
}

/* Failure injection for tests of the fallback path: DS4F_GPU_FAIL_AFTER=n
 * makes the (n+1)-th entry-point call fail before it launches anything. */
static int forced_failure(void) {
    if (P.fail_countdown < 0) return 0;
    if (P.fail_countdown == 0) {
        set_err("forced failure (DS4F_GPU_FAIL_AFTER)");
        return 1;
    }
    P.fail_countdown--;
    return 0;
}

int ds4f_gpu_attn_bind(const Ds4fGpuAttnGeom *geom, const int *layer_kind, float *host_kv,
                       float *host_lin, float *host_conv, int n_kv_tokens) {
    if (ds4f_gpu_init() != 0 || P.disabled) return -1;
    if (!geom || !layer_kind) return -1;
    const Ds4fGpuAttnGeom g = *geom;
    if (g.n_layers < 1 || g.max_tokens < 1 || g.head_dim != GQA_D || g.n_kv_heads < 1 ||
        g.n_heads != GQA_GROUP * g.n_kv_heads || g.lin_kd != 128 || g.lin_vd != 128) {
        set_err("unsupported geometry (head_dim %d heads %d kv_heads %d kd %d vd %d)",
                g.head_dim, g.n_heads, g.n_kv_heads, g.lin_kd, g.lin_vd);
        return -1;
    }
    hipStreamSynchronize(P.stream);
    free_binding();
    P.g = g;
    P.kind = (int *)calloc((size_t)g.n_layers, sizeof(int));
    P.slot = (int *)calloc((size_t)g.n_layers, sizeof(int));
    if (!P.kind || !P.slot) return -1;
    P.n_gqa = P.n_lin = 0;
    for (int l = 0; l < g.n_layers; l++) {
        P.kind[l] = layer_kind[l];
        if (layer_kind[l] == DS4F_LAYER_GQA)
            P.slot[l] = P.n_gqa++;
        else if (layer_kind[l] == DS4F_LAYER_LINEAR)
            P.slot[l] = P.n_lin++;
        else
            P.slot[l] = -1;
    }
    P.kd = g.lin_kd;
    P.vd = g.lin_vd;
    P.vh = 16 * g.n_kv_heads;                           /* src/attn_qwen.c:453 */
    P.rows = 2 * g.n_heads * P.kd + P.vh * P.vd;        /* src/attn_qwen.c:866 */
    P.t_pad = (g.max_tokens + 63) / 64 * 64;
    P.t_tiles = P.t_pad / 16;
    P.kv_elems = (size_t)g.n_kv_heads * P.t_pad * GQA_D;
    P.host_kv = host_kv;
    P.host_lin = host_lin;
    P.host_conv = host_conv;

    if (P.n_gqa) {
        size_t b = (size_t)P.n_gqa * P.kv_elems * sizeof(uint16_t);
        HIPCHK(hipMalloc((void **)&P.d_k, b));
        HIPCHK(hipMalloc((void **)&P.d_v, b));
        HIPCHK(hipMemsetAsync(P.d_k, 0, b, P.stream));
        HIPCHK(hipMemsetAsync(P.d_v, 0, b, P.stream));
        size_t pb = (size_t)g.n_kv_heads * q35_gqa_max_chunks() * GQA_GROUP;
        HIPCHK(hipMalloc((void **)&P.d_part_o, pb * GQA_D * sizeof(float)));
        HIPCHK(hipMalloc((void **)&P.d_part_ml, pb * 2 * sizeof(float)));
        /* RoPE table: double -> float per position, as src/attn_qwen.c:302-307 */
        size_t nr = (size_t)g.max_tokens * ROPE_DIMS;
        float *tab = (float *)malloc(nr * sizeof(float));
        if (!tab) return -1;
        double inv[ROPE_DIMS / 2];
        for (int i = 0; i < ROPE_DIMS / 2; i++)
            inv[i] = 1.0 / pow(ROPE_THETA, (double)(2 * i) / (double)ROPE_DIMS);
        for (int t = 0; t < g.max_tokens; t++) {
            float *row = tab + (size_t)t * ROPE_DIMS;
            for (int i = 0; i < ROPE_DIMS / 2; i++) {
                double f = (double)t * inv[i];
                row[i] = (float)cos(f);
                row[ROPE_DIMS / 2 + i] = (float)sin(f);
            }
        }
        if (hipMalloc((void **)&P.d_rope, nr * sizeof(float)) != hipSuccess ||
            hipMemcpy(P.d_rope, tab, nr * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
            free(tab);
            set_err("rope table upload failed");
            return -1;
        }
        free(tab);
    }
    if (P.n_lin) {
        size_t b = (size_t)P.n_lin * lin_floats() * sizeof(float);
        size_t c = (size_t)P.n_lin * conv_floats() * sizeof(float);
        HIPCHK(hipMalloc((void **)&P.d_lin, b));
        HIPCHK(hipMalloc((void **)&P.d_conv, c));
        HIPCHK(hipMemsetAsync(P.d_lin, 0, b, P.stream));
        HIPCHK(hipMemsetAsync(P.d_conv, 0, c, P.stream));
    }
    HIPCHK(hipStreamSynchronize(P.stream));
    P.bound = 1;
    for (int l = 0; l < g.n_layers; l++)
        if (sync_layer(l, DS4F_SYNC_TO_DEVICE, n_kv_tokens) != 0) {
            P.bound = 0;
            return -1;
        }
    return 0;
}

static hipStream_t pick(void *stream) { return stream ? (hipStream_t)stream : P.stream; }

static int check_layer(int L, int kind) {
    if (!P.ok || P.disabled || !P.bound) {
        set_err("plugin not bound or disabled");
        return -1;
    }
    if (L < 0 || L >= P.g.n_layers || P.kind[L] != kind) {
        set_err("layer %d is not bound as kind %d", L, kind);
        return -1;
    }
    return 0;
}

/* ---- device-pointer entry points --------------------------------------- */

int ds4f_hip_gqa_decode_async(int L, int token, const float *q_gate, const float *k,
                              const float *v, const uint16_t *qn_w, const uint16_t *kn_w,
                              float *attn_out, float *k_post, void *stream) {
    if (check_layer(L, DS4F_LAYER_GQA) != 0) return -1;
    if (token < 0 || token >= P.g.max_tokens) return 0;     /* src/attn_qwen.c:256 */
    Q35GqaDecode p;
    memset(&p, 0, sizeof p);
    p.q_gate = q_gate;
    p.k_new = k;
    p.v_new = v;
    p.qn_w = qn_w;
    p.kn_w = kn_w;
    p.rope = P.d_rope + (size_t)token * ROPE_DIMS;
    p.kt = layer_k(P.slot[L]);
    p.vt = layer_v(P.slot[L]);
    p.part_o = P.d_part_o;
    p.part_ml = P.d_part_ml;
    p.attn_out = attn_out;
    p.k_post = k_post;
    p.token = token;
    p.t_tiles = P.t_tiles;
    p.heads = P.g.n_heads;
    p.kv_heads = P.g.n_kv_heads;
    q35_gqa_split(token, &p.chunk, &p.n_chunks);
    HIPCHK(q35_gqa_decode(&p, pick(stream)));
    return 0;
}

int ds4f_hip_gqa_prefill_async(int L, int t0, int B, const float *q_gate, const float *k,
                               const float *v, const uint16_t *qn_w, const uint16_t *kn_w,
                               float *attn_out, float *k_post, void *stream) {
    if (check_layer(L, DS4F_LAYER_GQA) != 0) return -1;
    if (t0 < 0 || B < 1 || t0 >= P.g.max_tokens) return 0;   /* src/attn_qwen.c:256 */
    if (B > P.g.max_tokens - t0) B = P.g.max_tokens - t0;
    /* the first call reserves the fp16 K / V workspace of the whole cache
     * (t0 + B = max_tokens), so the later chunks of a chunked prefill, whose
     * workspace grows with t0 + B, neither reallocate nor invalidate a HIP
     * graph captured after the first */
    size_t kb, vb, kr, vr;
    q35_gqa_prefill_ws_bytes(t0, B, P.g.n_kv_heads, &kb, &vb);
    q35_gqa_prefill_ws_bytes(0, P.g.max_tokens, P.g.n_kv_heads, &kr, &vr);
    if (ensure_ws(kr + vr) != 0) return -1;
    Q35GqaPrefill p;
    memset(&p, 0, sizeof p);
    p.q_gate = q_gate;
    p.k_in = k;
    p.v_in = v;
    p.qn_w = qn_w;
    p.kn_w = kn_w;
    p.rope = P.d_rope;
    p.kt = layer_k(P.slot[L]);
    p.vt = layer_v(P.slot[L]);
    p.kw = (uint16_t *)P.d_ws;
    p.vw = (uint16_t *)((char *)P.d_ws + kb);
    p.attn_out = attn_out;
    p.k_post = k_post;
    p.t0 = t0;
    p.B = B;
    p.t_tiles = P.t_tiles;
    p.heads = P.g.n_heads;
    p.kv_heads = P.g.n_kv_heads;
    p.status = P.d_status_cur;
    HIPCHK(q35_gqa_prefill(&p, pick(stream)));
    return 0;
}

int ds4f_hip_lin_decode_async(int L, int token, const float *qkv, const float *z, const float *a,
                              const float *b, const uint16_t *conv_w, const float *A_log,
                              const uint16_t *dt_bias, const uint16_t *norm_w, float *out,
                              float *qkv_post, void *stream) {
    if (check_layer(L, DS4F_LAYER_LINEAR) != 0) return -1;
    if (token < 0 || token >= P.g.max_tokens) return 0;     /* src/attn_qwen.c:882 */
    Q35LinDecode p;
    memset(&p, 0, sizeof p);
    p.qkv = qkv;
    p.z = z;
    p.a = a;
    p.b = b;
    p.conv_w = conv_w;
    p.A_log = A_log;
    p.dt_bias = dt_bias;
    p.norm_w = norm_w;
    p.ring = layer_conv(P.slot[L]);
    p.state = layer_lin(P.slot[L]);
    p.out = out;
    p.qkv_post = qkv_post;
    p.token = token;
    p.k_heads = P.g.n_heads;
    p.v_heads = P.vh;
    HIPCHK(q35_lin_decode(&p, pick(stream)));
    return 0;
}

/* the delta-rule prefill; xw non-NULL: the gated norm writes the chunk
 * GEMM's X operand (xw, xsum over mpad rows) instead of out */
static int lin_prefill_launch(int L, int t0, int B, const float *qkv, const float *z,
                              const float *a, const float *b, const uint16_t *conv_w,
                              const float *A_log, const uint16_t *dt_bias, const uint16_t *norm_w,
                              float *out, float *qkv_post, uint16_t *xw, float *xsum, int mpad,
                              void *ws, size_t ws_cap, void *stream) {
    if (check_layer(L, DS4F_LAYER_LINEAR) != 0) return -1;
    if (t0 < 0 || B < 1 || t0 >= P.g.max_tokens) return 0;   /* src/attn_qwen.c:882 */
    if (B > P.g.max_tokens - t0) B = P.g.max_tokens - t0;
    if (xw && (mpad < B || mpad % q35_mlx4_gemm_mtile() != 0 || !xsum)) {
        set_err("lin prefill: X operand of %d rows for %d tokens", mpad, B);
        return -1;
    }
    size_t bytes;
    q35_lin_prefill_ws_bytes(B, P.g.n_heads, P.vh, qkv_post == NULL, &bytes);
    if (!ws) {
        if (ensure_ws(bytes) != 0) return -1;
        ws = P.d_ws;
    } else if (bytes > ws_cap) {
        set_err("lin prefill: %d tokens need %zu workspace bytes, the static workspace holds %zu",
                B, bytes, ws_cap);
        return -1;
    }
    Q35LinPrefill p;
    memset(&p, 0, sizeof p);
    p.qkv = qkv;
    p.z = z;
    p.a = a;
    p.b = b;
    p.conv_w = conv_w;
    p.A_log = A_log;
    p.dt_bias = dt_bias;
    p.norm_w = norm_w;
    p.ring = layer_conv(P.slot[L]);
    p.state = layer_lin(P.slot[L]);
    p.out = out;
    p.t0 = t0;
    p.B = B;
    p.n_chunks = (B + 63) / 64;
    p.k_heads = P.g.n_heads;
    p.v_heads = P.vh;
    /* carve the workspace, each piece 256-byte aligned */
    const size_t nc = (size_t)p.n_chunks, vh = (size_t)P.vh;
    char *w = (char *)ws;
#define CARVE(dst, nfloats)                                   \
    do {                                                      \
        (dst) = (float *)w;                                   \
        w += (((size_t)(nfloats) * sizeof(float)) + 255) & ~(size_t)255; \
    } while (0)
    if (qkv_post)
        p.post = qkv_post;
    else
        CARVE(p.post, (size_t)B * P.rows);
    CARVE(p.gates, (size_t)B * vh * 2);
    CARVE(p.T, nc * vh * 64 * 64);
    CARVE(p.Pm, nc * vh * 64 * 64);
    CARVE(p.gvec, nc * vh * Q35_LIN_GVEC);
#undef CARVE
    p.xw = xw;
    p.xsum = xsum;
    p.mpad = mpad;
    p.status = P.d_status_cur;
    HIPCHK(q35_lin_prefill(&p, pick(stream)));
    return 0;
}

int ds4f_hip_lin_prefill_async(int L, int t0, int B, const float *qkv, const float *z,
                               const float *a, const float *b, const uint16_t *conv_w,
                               const float *A_log, const uint16_t *dt_bias,
                               const uint16_t *norm_w, float *out, float *qkv_post,
                               void *stream) {
    return lin_prefill_launch(L, t0, B, qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, out, qkv_post,
                              NULL, NULL, 0, NULL, 0, stream);
}

int ds4f_hip_lin_prefill_noalloc(int L, int t0, int B, const float *qkv, const float *z,
                                 const float *a, const float *b, const uint16_t *conv_w,
                                 const float *A_log, const uint16_t *dt_bias,
                                 const uint16_t *norm_w, float *out, float *qkv_post,
                                 void *stream) {
    if (check_layer(L, DS4F_LAYER_LINEAR) != 0) return -1;
    if (t0 >= 0 && t0 < P.g.max_tokens && B > Q35_LIN_NOALLOC_MAX_B &&
        (B < P.g.max_tokens - t0 ? B : P.g.max_tokens - t0) > Q35_LIN_NOALLOC_MAX_B) {
        set_err("lin prefill (no allocation): %d tokens exceed the maximum of %d", B,
                Q35_LIN_NOALLOC_MAX_B);
        return -1;
    }
    void *ws = q35_lin_scratch();
    if (P.scratch_rc != (int)hipSuccess || !ws) {
        set_err("lin prefill (no allocation): static workspace address unavailable (%s)",
                hipGetErrorString((hipError_t)P.scratch_rc));
        return -1;
    }
    return lin_prefill_launch(L, t0, B, qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, out, qkv_post,
                              NULL, NULL, 0, ws, Q35_LIN_SCRATCH_BYTES, stream);
}

/* ---- host-pointer entry points ----------------------------------------- */

/* Pack host arrays into the pinned stage, one H2D copy; returns device
 * pointers of each piece (256-byte aligned). */
typedef struct { const void *src; size_t bytes; void **dev; } Piece;

static int upload(Piece *pc, int n, size_t out_bytes, void **d_out) {
    size_t off = 0, offs[16];
    for (int i = 0; i < n; i++) {
        offs[i] = off;
        off += (pc[i].bytes + 255) & ~(size_t)255;
    }
    size_t out_off = off;
    off += (out_bytes + 255) & ~(size_t)255;
    if (ensure_stage(off, off) != 0) return -1;
    for (int i = 0; i < n; i++) {
        memcpy((char *)P.h_stage + offs[i], pc[i].src, pc[i].bytes);
        *pc[i].dev = (char *)P.d_stage + offs[i];
    }
    HIPCHK(hipMemcpyAsync(P.d_stage, P.h_stage, out_off, hipMemcpyHostToDevice, P.stream));
    *d_out = (char *)P.d_stage + out_off;
    return 0;
}

static int download(void *d_src, size_t bytes) {
    HIPCHK(hipMemcpyAsync(P.h_stage, d_src, bytes, hipMemcpyDeviceToHost, P.stream));
    HIPCHK(hipStreamSynchronize(P.stream));
    return 0;
}

/* The status words.  Word 0 is the device-pointer callers' (read and
 * cleared by ds4f_hip_f16_status); the host entries switch the launches to
 * their own word HOST_WORD for the duration of a call (host_status_begin
 * clears it, host_status_end reads it and switches back), so a bit a
 * device-pointer call left in word 0 is neither cleared nor reported by
 * them. */
enum { HOST_WORD = 16 };   /* 64 bytes past word 0 */
static int status_clear(const int *word, hipStream_t st) {
    HIPCHK(hipMemsetAsync((void *)word, 0, sizeof(int), st));
    return 0;
}
static int status_read(const int *word, hipStream_t st, int *bits) {
    HIPCHK(hipMemcpyAsync(P.h_status, word, sizeof(int), hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    *bits = *P.h_status;
    return 0;
}
static int host_status_begin(void) {
    P.d_status_cur = P.d_status + HOST_WORD;
    if (status_clear(P.d_status_cur, P.stream) != 0) {
        P.d_status_cur = P.d_status;
        return -1;
    }
    return 0;
}
/* reads the host word (when bits is not NULL) and switches back to word 0 */
static int host_status_end(int *bits) {
    int rc = bits ? status_read(P.d_status + HOST_WORD, P.stream, bits) : 0;
    P.d_status_cur = P.d_status;
    return rc;
}

int ds4f_hip_f16_status(void *stream, int clear) {
    if (!P.ok) {
        set_err("plugin not initialised (ds4f_gpu_init)");
        return -1;
    }
    hipStream_t st = pick(stream);
    int bits = 0;
    if (status_read(P.d_status, st, &bits) != 0) return -1;
    if (clear && bits && (status_clear(P.d_status, st) != 0 || hipStreamSynchronize(st) != hipSuccess))
        return -1;
    return bits;
}

int ds4f_gpu_gqa_decode(int L, int token, const float *q_gate, float *k, const float *v,
                        const uint16_t *qn_w, const uint16_t *kn_w, float *attn_out) {
    if (check_layer(L, DS4F_LAYER_GQA) != 0) return -1;
    if (token < 0 || token >= P.g.max_tokens) return 0;
    if (forced_failure()) return fail_over(token);
    const int H = P.g.n_heads, KVH = P.g.n_kv_heads, D = GQA_D;
    void *dq, *dk, *dv, *dqn, *dkn, *dout;
    Piece pc[5] = {{q_gate, (size_t)H * 2 * D * 4, &dq},
                   {k, (size_t)KVH * D * 4, &dk},
                   {v, (size_t)KVH * D * 4, &dv},
                   {qn_w, (size_t)D * 2, &dqn},
                   {kn_w, (size_t)D * 2, &dkn}};
    size_t ob = (size_t)(H + KVH) * D * 4;   /* attn_out then k_post */
    if (upload(pc, 5, ob, &dout) != 0) return fail_over(token);
    float *d_attn = (float *)dout, *d_kpost = d_attn + (size_t)H * D;
    if (ds4f_hip_gqa_decode_async(L, token, (const float *)dq, (const float *)dk,
                                  (const float *)dv, (const uint16_t *)dqn,
                                  (const uint16_t *)dkn, d_attn, d_kpost, NULL) != 0 ||
        download(dout, ob) != 0)
        return fail_over(token);
    memcpy(attn_out, P.h_stage, (size_t)H * D * 4);
    memcpy(k, (char *)P.h_stage + (size_t)H * D * 4, (size_t)KVH * D * 4);
    return 0;
}

int ds4f_gpu_lin_decode(int L, int token, float *qkv, const float *z, const float *a,
                        const float *b, const uint16_t *conv_w, const float *A_log,
                        const uint16_t *dt_bias, const uint16_t *norm_w, float *out) {
    if (check_layer(L, DS4F_LAYER_LINEAR) != 0) return -1;
    if (token < 0 || token >= P.g.max_tokens) return 0;
    if (forced_failure()) return fail_over(token);
    const int rows = P.rows, VH = P.vh, VD = P.vd;
    void *dqkv, *dz, *da, *db, *dcw, *dal, *ddt, *dnw, *dout;
    Piece pc[8] = {{qkv, (size_t)rows * 4, &dqkv},
                   {z, (size_t)VH * VD * 4, &dz},
                   {a, (size_t)VH * 4, &da},
                   {b, (size_t)VH * 4, &db},
                   {conv_w, (size_t)rows * 4 * 2, &dcw},
                   {A_log, (size_t)VH * 4, &dal},
                   {dt_bias, (size_t)VH * 2, &ddt},
                   {norm_w, (size_t)VD * 2, &dnw}};
    size_t ob = ((size_t)VH * VD + rows) * 4;   /* out then qkv_post */
    if (upload(pc, 8, ob, &dout) != 0) return fail_over(token);
    float *d_out = (float *)dout, *d_post = d_out + (size_t)VH * VD;
    if (ds4f_hip_lin_decode_async(L, token, (const float *)dqkv, (const float *)dz,
                                  (const float *)da, (const float *)db, (const uint16_t *)dcw,
                                  (const float *)dal, (const uint16_t *)ddt,
                                  (const uint16_t *)dnw, d_out, d_post, NULL) != 0 ||
        download(dout, ob) != 0)
        return fail_over(token);
    memcpy(out, P.h_stage, (size_t)VH * VD * 4);
    memcpy(qkv, (char *)P.h_stage + (size_t)VH * VD * 4, (size_t)rows * 4);
    return 0;
}

/* Prefill over B tokens (src/attn_qwen.c:1222-1231 / :1088-1109 semantics). */
int ds4f_gpu_gqa_prefill(int L, int t0, int B, const float *q_gate, float *k, const float *v,
                         const uint16_t *qn_w, const uint16_t *kn_w, float *attn_out) {
    if (check_layer(L, DS4F_LAYER_GQA) != 0) return -1;
    if (t0 < 0 || B < 1 || t0 >= P.g.max_tokens) return 0;
    if (B > P.g.max_tokens - t0) B = P.g.max_tokens - t0;   /* later tokens: silent skip */
    if (forced_failure()) return fail_over(t0);
    const int H = P.g.n_heads, KVH = P.g.n_kv_heads, D = GQA_D;
    void *dq, *dk, *dv, *dqn, *dkn, *dout;
    Piece pc[5] = {{q_gate, (size_t)B * H * 2 * D * 4, &dq},
                   {k, (size_t)B * KVH * D * 4, &dk},
                   {v, (size_t)B * KVH * D * 4, &dv},
                   {qn_w, (size_t)D * 2, &dqn},
                   {kn_w, (size_t)D * 2, &dkn}};
    const size_t ob = (size_t)B * H * D * 4, kb = (size_t)B * KVH * D * 4;
    if (upload(pc, 5, ob + kb, &dout) != 0) return fail_over(t0);
    float *d_attn = (float *)dout, *d_kpost = (float *)((char *)dout + ob);
    int bits = 0;
    if (host_status_begin() != 0) return fail_over(t0 + B);
    if (ds4f_hip_gqa_prefill_async(L, t0, B, (const float *)dq, (const float *)dk,
                                   (const float *)dv, (const uint16_t *)dqn,
                                   (const uint16_t *)dkn, d_attn, d_kpost, NULL) != 0) {
        host_status_end(NULL);
        return fail_over(t0 + B);
    }
    if (host_status_end(&bits) != 0) return fail_over(t0 + B);
    if (bits & Q35_STATUS_GQA_F16) {
        /* an operand beyond fp16 range: the tokens again on the decode
         * kernels (bf16 cache, fp32 q and weights), in order; the prefill
         * already wrote their cache rows, which each decode step rewrites
         * with the same values before attending */
        for (int b = 0; b < B; b++)
            if (ds4f_hip_gqa_decode_async(L, t0 + b, (const float *)dq + (size_t)b * H * 2 * D,
                                          (const float *)dk + (size_t)b * KVH * D,
                                          (const float *)dv + (size_t)b * KVH * D,
                                          (const uint16_t *)dqn, (const uint16_t *)dkn,
                                          d_attn + (size_t)b * H * D,
                                          d_kpost + (size_t)b * KVH * D, NULL) != 0)
                return fail_over(t0 + B);
    }
    if (download(dout, ob + kb) != 0) return fail_over(t0 + B);
    memcpy(attn_out, P.h_stage, ob);
    memcpy(k, (char *)P.h_stage + ob, kb);
    return 0;
}

int ds4f_gpu_lin_prefill(int L, int t0, int B, float *qkv, const float *z, const float *a,
                         const float *b, const uint16_t *conv_w, const float *A_log,
                         const uint16_t *dt_bias, const uint16_t *norm_w, float *out) {
    if (check_layer(L, DS4F_LAYER_LINEAR) != 0) return -1;
    if (t0 < 0 || B < 1 || t0 >= P.g.max_tokens) return 0;
    if (B > P.g.max_tokens - t0) B = P.g.max_tokens - t0;   /* later tokens: silent skip */
    if (forced_failure()) return fail_over(t0);
    const int rows = P.rows, VH = P.vh, VD = P.vd;
    void *dqkv, *dz, *da, *db, *dcw, *dal, *ddt, *dnw, *dout;
    Piece pc[8] = {{qkv, (size_t)B * rows * 4, &dqkv},
                   {z, (size_t)B * VH * VD * 4, &dz},
                   {a, (size_t)B * VH * 4, &da},
                   {b, (size_t)B * VH * 4, &db},
                   {conv_w, (size_t)rows * 4 * 2, &dcw},
                   {A_log, (size_t)VH * 4, &dal},
                   {dt_bias, (size_t)VH * 2, &ddt},
                   {norm_w, (size_t)VD * 2, &dnw}};
    const size_t ob = (size_t)B * VH * VD * 4, pb = (size_t)B * rows * 4;
    if (upload(pc, 8, ob + pb, &dout) != 0) return fail_over(t0);
    float *d_out = (float *)dout, *d_post = (float *)((char *)dout + ob);
    if (ds4f_hip_lin_prefill_async(L, t0, B, (const float *)dqkv, (const float *)dz,
                                   (const float *)da, (const float *)db, (const uint16_t *)dcw,
                                   (const float *)dal, (const uint16_t *)ddt,
                                   (const uint16_t *)dnw, d_out, d_post, NULL) != 0 ||
        download(dout, ob + pb) != 0)
        return fail_over(t0 + B);
    memcpy(out, P.h_stage, ob);
    memcpy(qkv, (char *)P.h_stage + ob, pb);
    return 0;
}

/* ---- synthetic state ---------------------------------------------------- */

int ds4f_hip_launch_floor(int n, int grid, int block, void *stream) {
    if (ds4f_gpu_init() != 0) return -1;
    HIPCHK(q35_empty_kernels(n, grid, block, pick(stream)));
    return 0;
}

int ds4f_hip_synth(void *dst, int64_t n, int dtype, int dist, double p0, double p1,
                   uint64_t seed, uint64_t tid, void *stream) {
    if (ds4f_gpu_init() != 0) return -1;
    HIPCHK(q35_synth(dst, n, dtype, dist, p0, p1, seed, tid, pick(stream)));
    return 0;
}

int ds4f_hip_synth_gqa_cache(int L, int n_past, uint64_t seed, uint64_t tid_k, uint64_t tid_v,
                             void *stream) {
    if (check_layer(L, DS4F_LAYER_GQA) != 0) return -1;
    if (n_past < 0 || n_past > P.g.max_tokens) return -1;
    HIPCHK(q35_synth_kv(layer_k(P.slot[L]), layer_v(P.slot[L]), n_past, P.t_tiles,
                        P.g.n_kv_heads, seed, tid_k, tid_v, pick(stream)));
    return 0;
}

int ds4f_hip_synth_lin_state(int L, double sigma, uint64_t seed, uint64_t tid, void *stream) {
    if (check_layer(L, DS4F_LAYER_LINEAR) != 0) return -1;
    HIPCHK(q35_synth_state(layer_lin(P.slot[L]), P.vh, P.kd, P.vd, sigma, seed, tid,
                           pick(stream)));
    return 0;
}

int ds4f_hip_synth_conv_history(int L, int token, uint64_t seed, uint64_t tid, void *stream) {
    if (check_layer(L, DS4F_LAYER_LINEAR) != 0) return -1;
    HIPCHK(q35_synth_conv(layer_conv(P.slot[L]), P.rows, token, seed, tid, pick(stream)));
    return 0;
}

/* ---- MLX 4-bit matvecs (include/ds4f/gpu.h:29-54) ---------------------- */

/* one device copy of an MLX 4-bit weight: nibble words, scales, biases */
typedef struct {
    const void *key;
    int R, C, has_b;
    void *d;                   /* vals | scales | biases, one allocation */
} Mlx4W;

static struct {
    Mlx4W head;                /* ds4f_gpu_mlx4_matvec's weight */
    Mlx4W *slot;               /* ds4f_gpu_mlx4_batch's weights, by id */
    int n_slot, cap_slot;
    float *d_x, *d_y, *h_x, *h_y;
    size_t x_cap, y_cap;       /* floats */
    Q35Mlx4Job *d_jobs, *h_jobs;
    int jobs_cap;
} M;

static size_t mlx4_vbytes(int R, int C) { return (size_t)R * C / 2; }
static size_t mlx4_sbytes(int R, int C) { return ((size_t)R * C + 63) / 64 * 2; }
static const uint32_t *mlx4_v(const Mlx4W *w) { return (const uint32_t *)w->d; }
static const uint16_t *mlx4_s(const Mlx4W *w) {
    return (const uint16_t *)((const char *)w->d + mlx4_vbytes(w->R, w->C));
}
static const uint16_t *mlx4_b(const Mlx4W *w) {
    return w->has_b ? (const uint16_t *)((const char *)w->d + mlx4_vbytes(w->R, w->C) +
                                         mlx4_sbytes(w->R, w->C))
                    : NULL;
}

/* (re)fill a device weight from host arrays when its key or shape changed */
static int mlx4_upload(Mlx4W *w, const void *key, const uint32_t *vals, const uint16_t *scales,
                       const uint16_t *biases, int R, int C) {
    const int has_b = biases != NULL;
    if (w->d && w->key == key && w->R == R && w->C == C && w->has_b == has_b) return 0;
    if (w->d) hipFree(w->d);
    w->d = NULL;
    const size_t vb = mlx4_vbytes(R, C), sb = mlx4_sbytes(R, C);
    HIPCHK(hipMalloc(&w->d, vb + sb * (has_b ? 2 : 1)));
    HIPCHK(hipMemcpy(w->d, vals, vb, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy((char *)w->d + vb, scales, sb, hipMemcpyHostToDevice));
    if (has_b) HIPCHK(hipMemcpy((char *)w->d + vb + sb, biases, sb, hipMemcpyHostToDevice));
    w->key = key;
    w->R = R;
    w->C = C;
    w->has_b = has_b;
    return 0;
}

/* pinned host and device staging for njobs x / y vectors */
static int mlx4_stage(size_t xf, size_t yf, int njobs) {
    if (xf > M.x_cap) {
        if (M.d_x) hipFree(M.d_x);
        if (M.h_x) hipHostFree(M.h_x);
        M.d_x = M.h_x = NULL;
        M.x_cap = 0;
        HIPCHK(hipMalloc((void **)&M.d_x, xf * sizeof(float)));
        HIPCHK(hipHostMalloc((void **)&M.h_x, xf * sizeof(float), hipHostMallocDefault));
        M.x_cap = xf;
    }
    if (yf > M.y_cap) {
        if (M.d_y) hipFree(M.d_y);
        if (M.h_y) hipHostFree(M.h_y);
        M.d_y = M.h_y = NULL;
        M.y_cap = 0;
        HIPCHK(hipMalloc((void **)&M.d_y, yf * sizeof(float)));
        HIPCHK(hipHostMalloc((void **)&M.h_y, yf * sizeof(float), hipHostMallocDefault));
        M.y_cap = yf;
    }
    if (njobs > M.jobs_cap) {
        if (M.d_jobs) hipFree(M.d_jobs);
        if (M.h_jobs) hipHostFree(M.h_jobs);
        M.d_jobs = M.h_jobs = NULL;
        M.jobs_cap = 0;
        HIPCHK(hipMalloc((void **)&M.d_jobs, (size_t)njobs * sizeof(Q35Mlx4Job)));
        HIPCHK(hipHostMalloc((void **)&M.h_jobs, (size_t)njobs * sizeof(Q35Mlx4Job),
                             hipHostMallocDefault));
        M.jobs_cap = njobs;
    }
    return 0;
}

static int mlx4_ready(int R, int C) {
    if (!P.ok) {
        set_err("plugin not initialised (ds4f_gpu_init)");
        return -1;
    }
    if (!q35_mlx4_supported(R, C)) {
        set_err("mlx4 matvec: unsupported shape R %d C %d (needs C %% 32 == 0, 32..8192)", R, C);
        return -1;
    }
    return 0;
}

static void mlx4_free(void) {
    if (M.head.d) hipFree(M.head.d);
    for (int i = 0; i < M.n_slot; i++)
        if (M.slot[i].d) hipFree(M.slot[i].d);
    free(M.slot);
    if (M.d_x) hipFree(M.d_x);
    if (M.d_y) hipFree(M.d_y);
    if (M.d_jobs) hipFree(M.d_jobs);
    if (M.h_x) hipHostFree(M.h_x);
    if (M.h_y) hipHostFree(M.h_y);
    if (M.h_jobs) hipHostFree(M.h_jobs);
    memset(&M, 0, sizeof M);
}

int ds4f_gpu_mlx4_matvec(const uint32_t *vals, const uint16_t *scales, const uint16_t *biases,
                         int R, int C, const float *x, float *y) {
    if (mlx4_ready(R, C) != 0) return -1;
    /* the weight stays on the device between calls (the output head); a
     * new pointer or shape replaces it */
    if (mlx4_upload(&M.head, vals, vals, scales, biases, R, C) != 0) return -1;
    if (mlx4_stage((size_t)C, (size_t)R, 0) != 0) return -1;
    memcpy(M.h_x, x, (size_t)C * sizeof(float));
    HIPCHK(hipMemcpyAsync(M.d_x, M.h_x, (size_t)C * sizeof(float), hipMemcpyHostToDevice, P.stream));
    Q35Mlx4 p = {mlx4_v(&M.head), mlx4_s(&M.head), mlx4_b(&M.head), M.d_x, M.d_y, NULL, R, C, NULL, 0};
    HIPCHK(q35_mlx4_matvec(&p, 1, P.stream));
    HIPCHK(hipMemcpyAsync(M.h_y, M.d_y, (size_t)R * sizeof(float), hipMemcpyDeviceToHost, P.stream));
    HIPCHK(hipStreamSynchronize(P.stream));
    memcpy(y, M.h_y, (size_t)R * sizeof(float));
    return 0;
}

int ds4f_gpu_mlx4_batch(const uint32_t *const *vals, const uint16_t *const *scales,
                        const uint16_t *const *biases, const float *const *xs, float *const *ys,
                        const void *const *ids, int R, int C, int njobs) {
    if (njobs < 1) return 0;
    if (mlx4_ready(R, C) != 0) return -1;
    if (mlx4_stage((size_t)njobs * C, (size_t)njobs * R, njobs) != 0) return -1;
    for (int j = 0; j < njobs; j++) {
        /* weights are cached per stable id (gpu.h:36-43): the first sight
         * uploads, later calls reuse the device copy */
        int i = 0;
        while (i < M.n_slot && M.slot[i].key != ids[j]) i++;
        if (i == M.n_slot) {
            if (M.n_slot == M.cap_slot) {
                const int cap = M.cap_slot ? 2 * M.cap_slot : 64;
                Mlx4W *ns = (Mlx4W *)realloc(M.slot, (size_t)cap * sizeof(Mlx4W));
                if (!ns) {
                    set_err("mlx4 batch: out of host memory");
                    return -1;
                }
                memset(ns + M.cap_slot, 0, (size_t)(cap - M.cap_slot) * sizeof(Mlx4W));
                M.slot = ns;
                M.cap_slot = cap;
            }
            M.n_slot++;
        }
        if (mlx4_upload(&M.slot[i], ids[j], vals[j], scales[j], biases ? biases[j] : NULL, R, C) != 0)
            return -1;
        memcpy(M.h_x + (size_t)j * C, xs[j], (size_t)C * sizeof(float));
        const Q35Mlx4Job jb = {mlx4_v(&M.slot[i]), mlx4_s(&M.slot[i]), mlx4_b(&M.slot[i]),
                               M.d_x + (size_t)j * C, M.d_y + (size_t)j * R, R};
        M.h_jobs[j] = jb;
    }
    HIPCHK(hipMemcpyAsync(M.d_x, M.h_x, (size_t)njobs * C * sizeof(float), hipMemcpyHostToDevice,
                          P.stream));
    HIPCHK(hipMemcpyAsync(M.d_jobs, M.h_jobs, (size_t)njobs * sizeof(Q35Mlx4Job),
                          hipMemcpyHostToDevice, P.stream));
    Q35Mlx4 p = {NULL, NULL, NULL, NULL, NULL, M.d_jobs, R, C, NULL, 0};
    HIPCHK(q35_mlx4_matvec(&p, njobs, P.stream));
    HIPCHK(hipMemcpyAsync(M.h_y, M.d_y, (size_t)njobs * R * sizeof(float), hipMemcpyDeviceToHost,
                          P.stream));
    HIPCHK(hipStreamSynchronize(P.stream));
    for (int j = 0; j < njobs; j++) memcpy(ys[j], M.h_y + (size_t)j * R, (size_t)R * sizeof(float));
    return 0;
}

int ds4f_hip_mlx4_matvec_async(const uint32_t *vals, const uint16_t *scales,
                               const uint16_t *biases, int R, int C, const float *x, float *y,
                               void *stream) {
    if (mlx4_ready(R, C) != 0) return -1;
    Q35Mlx4 p = {vals, scales, biases, x, y, NULL, R, C, NULL, 0};
    HIPCHK(q35_mlx4_matvec(&p, 1, pick(stream)));
    return 0;
}

/* ---- whole attention layers (src/attn_qwen.c:87-225, :837-968) ---------- */

typedef struct LayerW {
    void *d;                   /* one allocation holding every tensor below */
    const uint16_t *in_norm;   /* input_layernorm, or NULL */
    Q35Mlx4Job *jobs;          /* projections of xin (x NULL: the launch's x) */
    int njobs, rmax;
    Q35Mlx4 out;               /* output projection: x, y set per call */
    const uint16_t *qn, *kn, *conv_w, *dt_bias, *norm_w;
    const float *A_log;
    Q35Mlx4GemmJob gj[5];      /* the chunk GEMMs' projections, then the output (y set per call) */
    int skip;                  /* incomplete in the trunk: every step and chunk is a silent skip */
} LayerW;

/* activations between the launches of one layer step, floats */
enum { ACT_Q, ACT_K, ACT_V, ACT_AO, ACT_QKV, ACT_Z, ACT_A, ACT_B, ACT_LO, ACT_N };

static size_t act_len(int i) {
    const size_t H = (size_t)P.g.n_heads, KVH = (size_t)P.g.n_kv_heads;
    switch (i) {
    case ACT_Q: return H * 2 * GQA_D;
    case ACT_K: case ACT_V: return KVH * GQA_D;
    case ACT_AO: return H * GQA_D;
    case ACT_QKV: return (size_t)P.rows;
    case ACT_Z: case ACT_LO: return (size_t)P.vh * P.vd;
    default: return (size_t)P.vh;          /* a, b */
    }
}

static float *act(int i) {
    size_t off = 0;
    for (int j = 0; j < i; j++) off += (act_len(j) + 63) & ~(size_t)63;
    return P.d_act + off;
}

static void layers_free(void) {
    if (P.lw) {
        for (int l = 0; l < P.g.n_layers; l++)
            if (P.lw[l].d) hipFree(P.lw[l].d);
        free(P.lw);
    }
    if (P.d_act) hipFree(P.d_act);
    if (P.d_state) hipFree(P.d_state);
    if (P.d_chunk) hipFree(P.d_chunk);
    if (P.h_states) hipHostFree(P.h_states);
    P.lw = NULL;
    P.d_act = P.d_state = NULL;
    P.d_chunk = NULL;
    P.h_states = NULL;
    P.chunk_cap = 0;
    P.h_states_cap = 0;
    P.hidden = 0;
}

/* Layer L's trunk lacks a role that gqa_step / linear_step require
 * (src/attn_qwen.c:96-97, :849-856, "incomplete graph: skip"): its weights
 * are dropped and every step and chunk of it returns 0 with the state
 * unchanged, as the reference's do.  Called by the trunk loader. */
__attribute__((visibility("hidden"))) int ds4f_plugin_layer_skip(int L) {
    if (!P.ok || P.disabled || !P.bound) {
        set_err("plugin not bound or disabled");
        return -1;
    }
    if (L < 0 || L >= P.g.n_layers) {
        set_err("layer %d outside [0, %d)", L, P.g.n_layers);
        return -1;
    }
    if (!P.lw) {
        P.lw = (LayerW *)calloc((size_t)P.g.n_layers, sizeof(LayerW));
        if (!P.lw) {
            set_err("layer table allocation failed");
            return -1;
        }
    }
    LayerW *lw = &P.lw[L];
    if (lw->d) {
        HIPCHK(hipStreamSynchronize(P.stream));
        hipFree(lw->d);
    }
    memset(lw, 0, sizeof *lw);
    lw->skip = 1;
    return 0;
}

/* a layer the trunk loader marked incomplete */
static int layer_skipped(int L) { return P.lw && P.lw[L].skip; }

static int mlx4_shape_ok(const Ds4fGpuMlx4W *m, int rows, int cols, const char *name) {
    if (!m->vals || !m->scales || m->rows != rows || m->cols != cols ||
        !q35_mlx4_supported(rows, cols)) {
        set_err("layer weights: %s is %dx%d, expected %dx%d", name, m->rows, m->cols, rows, cols);
        return 0;
    }
    return 1;
}

/* tensors of a layer in one allocation: every part with bytes > 0 gets a
 * 256-byte aligned slot (its device address in *dst, else NULL) and is
 * copied when it has a host source */
typedef struct { const void *src; size_t bytes; const void **dst; } Part;

static int upload_parts(LayerW *lw, Part *pt, int n) {
    size_t total = 0;
    for (int i = 0; i < n; i++) total += (pt[i].bytes + 255) & ~(size_t)255;
    HIPCHK(hipMalloc(&lw->d, total));
    size_t off = 0;
    for (int i = 0; i < n; i++) {
        char *d = (char *)lw->d + off;
        *pt[i].dst = pt[i].bytes ? d : NULL;
        if (pt[i].src && pt[i].bytes) HIPCHK(hipMemcpy(d, pt[i].src, pt[i].bytes, hipMemcpyHostToDevice));
        off += (pt[i].bytes + 255) & ~(size_t)255;
    }
    return 0;
}

/* the parts of one MLX 4-bit weight: vals, scales, biases */
static int mlx4_parts(Part *pt, const Ds4fGpuMlx4W *m, const void **v, const void **sc,
                      const void **b) {
    const size_t n = (size_t)m->rows * m->cols, ng = (n + 63) / 64;
    pt[0] = (Part){m->vals, n / 2, v};
    pt[1] = (Part){m->scales, ng * 2, sc};
    pt[2] = (Part){m->biases, m->biases ? ng * 2 : 0, b};
    return 3;
}

int ds4f_gpu_attn_weights(int L, const Ds4fGpuLayerW *w) {
    if (!P.ok || P.disabled || !P.bound) {
        set_err("plugin not bound or disabled");
        return -1;
    }
    if (L < 0 || L >= P.g.n_layers || !w) {
        set_err("layer weights: layer %d outside [0, %d) or no weights", L, P.g.n_layers);
        return -1;
    }
    const int kind = P.kind[L];
    if (kind != DS4F_LAYER_GQA && kind != DS4F_LAYER_LINEAR) {
        set_err("layer %d has no attention kind", L);
        return -1;
    }
    const int hidden = kind == DS4F_LAYER_GQA ? w->q.cols : w->qkv.cols;
    if (P.hidden && hidden != P.hidden) {
        set_err("layer weights: hidden %d differs from %d", hidden, P.hidden);
        return -1;
    }
    const int H = P.g.n_heads, KVH = P.g.n_kv_heads;
    if (kind == DS4F_LAYER_GQA) {
        if (!mlx4_shape_ok(&w->q, H * 2 * GQA_D, hidden, "q_proj") ||
            !mlx4_shape_ok(&w->k, KVH * GQA_D, hidden, "k_proj") ||
            !mlx4_shape_ok(&w->v, KVH * GQA_D, hidden, "v_proj") ||
            !mlx4_shape_ok(&w->o, hidden, H * GQA_D, "o_proj") || !w->q_norm || !w->k_norm)
            return -1;
    } else {
        if (!mlx4_shape_ok(&w->qkv, P.rows, hidden, "in_proj_qkv") ||
            !mlx4_shape_ok(&w->z, P.vh * P.vd, hidden, "in_proj_z") ||
            !mlx4_shape_ok(&w->a, P.vh, hidden, "in_proj_a") ||
            !mlx4_shape_ok(&w->b, P.vh, hidden, "in_proj_b") ||
            !mlx4_shape_ok(&w->out, hidden, P.vh * P.vd, "out_proj") || !w->conv_w ||
            !w->A_log || !w->dt_bias || !w->norm_w)
            return -1;
    }
    if (!P.lw) {
        P.lw = (LayerW *)calloc((size_t)P.g.n_layers, sizeof(LayerW));
        if (!P.lw) return -1;
    }
    if (!P.d_act) {
        size_t n = 0;
        for (int i = 0; i < ACT_N; i++) n += (act_len(i) + 63) & ~(size_t)63;
        HIPCHK(hipMalloc((void **)&P.d_act, n * sizeof(float)));
        HIPCHK(hipMalloc((void **)&P.d_state, (size_t)hidden * sizeof(float)));
    }
    P.hidden = hidden;
    LayerW *lw = &P.lw[L];
    if (lw->d) {
        HIPCHK(hipStreamSynchronize(P.stream));
        hipFree(lw->d);
    }
    memset(lw, 0, sizeof *lw);

    const Ds4fGpuMlx4W *proj[4], *outw;
    int np = 0, yact[4];
    if (kind == DS4F_LAYER_GQA) {
        proj[0] = &w->q, proj[1] = &w->k, proj[2] = &w->v;
        yact[0] = ACT_Q, yact[1] = ACT_K, yact[2] = ACT_V;
        np = 3;
        outw = &w->o;
    } else {
        proj[0] = &w->qkv, proj[1] = &w->z, proj[2] = &w->a, proj[3] = &w->b;
        yact[0] = ACT_QKV, yact[1] = ACT_Z, yact[2] = ACT_A, yact[3] = ACT_B;
        np = 4;
        outw = &w->out;
    }
    Part pt[40];
    const void *pv[5], *ps[5], *pb[5], *psb[5], *pwt[5], *in_norm, *jobs, *t0, *t1, *t2, *t3;
    int n = 0;
    for (int i = 0; i < np; i++) n += mlx4_parts(pt + n, proj[i], &pv[i], &ps[i], &pb[i]);
    n += mlx4_parts(pt + n, outw, &pv[4], &ps[4], &pb[4]);
    /* (16 s, b - 16 s) per row and 64-column group of each weight, for the
     * chunk GEMMs (filled on the device below) */
    for (int i = 0; i < 5; i++) {
        const Ds4fGpuMlx4W *m = i < 4 ? (i < np ? proj[i] : NULL) : outw;
        pt[n++] = (Part){NULL,
                         m ? (size_t)q35_mlx4_sb_npad(m->rows) * (m->cols / 64) * sizeof(Q35Mlx4SB) : 0,
                         &psb[i]};
        /* the words again, re-laid out for the GEMM's staging */
        pt[n++] = (Part){NULL, m ? (size_t)q35_mlx4_sb_npad(m->rows) * m->cols / 2 : 0, &pwt[i]};
    }
    pt[n++] = (Part){w->in_norm, w->in_norm ? (size_t)hidden * 2 : 0, &in_norm};
    pt[n++] = (Part){NULL, (size_t)np * sizeof(Q35Mlx4Job), &jobs};   /* filled below */
    if (kind == DS4F_LAYER_GQA) {
        pt[n++] = (Part){w->q_norm, GQA_D * 2, &t0};
        pt[n++] = (Part){w->k_norm, GQA_D * 2, &t1};
    } else {
        pt[n++] = (Part){w->conv_w, (size_t)P.rows * 4 * 2, &t0};
        pt[n++] = (Part){w->A_log, (size_t)P.vh * 4, &t1};
        pt[n++] = (Part){w->dt_bias, (size_t)P.vh * 2, &t2};
        pt[n++] = (Part){w->norm_w, (size_t)P.vd * 2, &t3};
    }
    if (upload_parts(lw, pt, n) != 0) {
        if (lw->d) hipFree(lw->d);
        memset(lw, 0, sizeof *lw);
        return -1;
    }
    /* the projections' job table, pointing at the weights just placed */
    Q35Mlx4Job hj[4];
    lw->rmax = 0;
    for (int i = 0; i < np; i++) {
        hj[i] = (Q35Mlx4Job){(const uint32_t *)pv[i], (const uint16_t *)ps[i],
                             (const uint16_t *)pb[i], NULL, act(yact[i]), proj[i]->rows};
        if (proj[i]->rows > lw->rmax) lw->rmax = proj[i]->rows;
    }
    if (hipMemcpy((void *)jobs, hj, (size_t)np * sizeof(Q35Mlx4Job), hipMemcpyHostToDevice) !=
        hipSuccess) {
        set_err("layer weights: job table upload failed");
        hipFree(lw->d);
        memset(lw, 0, sizeof *lw);
        return -1;
    }
    lw->jobs = (Q35Mlx4Job *)jobs;
    lw->njobs = np;
    /* the chunk GEMMs' jobs: the np projections, then the output */
    int ng = 0;
    for (int i = 0; i < 5; i++) {
        const Ds4fGpuMlx4W *m = i < 4 ? (i < np ? proj[i] : NULL) : outw;
        if (!m) continue;
        if (q35_mlx4_sb((const uint16_t *)ps[i], (const uint16_t *)pb[i], (Q35Mlx4SB *)psb[i],
                        m->rows, m->cols / 64, P.stream) != hipSuccess ||
            q35_mlx4_wt((const uint32_t *)pv[i], (uint32_t *)pwt[i], m->rows, m->cols, P.stream) !=
                hipSuccess ||
            hipStreamSynchronize(P.stream) != hipSuccess) {
            set_err("layer weights: scale table failed");
            hipFree(lw->d);
            memset(lw, 0, sizeof *lw);
            return -1;
        }
        lw->gj[ng++] = (Q35Mlx4GemmJob){(const uint32_t *)pwt[i], (const Q35Mlx4SB *)psb[i], NULL,
                                        m->rows, 0};
    }
    lw->in_norm = (const uint16_t *)in_norm;
    memset(&lw->out, 0, sizeof lw->out);
    lw->out.vals = (const uint32_t *)pv[4];
    lw->out.scales = (const uint16_t *)ps[4];
    lw->out.biases = (const uint16_t *)pb[4];
    lw->out.R = outw->rows;
    lw->out.C = outw->cols;
    lw->out.accumulate = 1;
    if (kind == DS4F_LAYER_GQA) {
        lw->qn = (const uint16_t *)t0;
        lw->kn = (const uint16_t *)t1;
    } else {
        lw->conv_w = (const uint16_t *)t0;
        lw->A_log = (const float *)t1;
        lw->dt_bias = (const uint16_t *)t2;
        lw->norm_w = (const uint16_t *)t3;
    }
    return 0;
}

int ds4f_hip_attn_step_async(int L, int token, float *state, void *stream) {
    if (!P.ok || P.disabled || !P.bound) {
        set_err("plugin not bound or disabled");
        return -1;
    }
    if (L < 0 || L >= P.g.n_layers) {
        set_err("layer step: layer %d outside [0, %d)", L, P.g.n_layers);
        return -1;
    }
    const int kind = P.kind[L];
    if (kind == DS4F_LAYER_NONE || layer_skipped(L)) return 0;   /* src/attn_qwen.c:1264, :96-97, :849-856 */
    if (!P.lw || !P.lw[L].d) {
        set_err("layer %d has no weights on the device (ds4f_gpu_attn_weights)", L);
        return -1;
    }
    if (token < 0 || token >= P.g.max_tokens) return 0;    /* :117, :882 */
    const LayerW *lw = &P.lw[L];
    hipStream_t st = pick(stream);
    Q35Mlx4 pr;
    memset(&pr, 0, sizeof pr);
    pr.jobs = lw->jobs;
    pr.R = lw->rmax;
    pr.C = P.hidden;
    pr.x = state;
    pr.x_norm = lw->in_norm;
    HIPCHK(q35_mlx4_matvec(&pr, lw->njobs, st));
    Q35Mlx4 po = lw->out;
    po.y = state;
    if (kind == DS4F_LAYER_GQA) {
        if (ds4f_hip_gqa_decode_async(L, token, act(ACT_Q), act(ACT_K), act(ACT_V), lw->qn,
                                      lw->kn, act(ACT_AO), NULL, st) != 0)
            return -1;
        po.x = act(ACT_AO);
    } else {
        if (ds4f_hip_lin_decode_async(L, token, act(ACT_QKV), act(ACT_Z), act(ACT_A),
                                      act(ACT_B), lw->conv_w, lw->A_log, lw->dt_bias, lw->norm_w,
                                      act(ACT_LO), NULL, st) != 0)
            return -1;
        po.x = act(ACT_LO);
    }
    HIPCHK(q35_mlx4_matvec(&po, 1, st));
    return 0;
}

int ds4f_gpu_attn_step(int L, int token, float *state) {
    if (!P.ok || P.disabled || !P.bound) {
        set_err("plugin not bound or disabled");
        return -1;
    }
    if (L < 0 || L >= P.g.n_layers) {
        set_err("layer step: layer %d outside [0, %d)", L, P.g.n_layers);
        return -1;
    }
    if (P.kind[L] == DS4F_LAYER_NONE || layer_skipped(L) || token < 0 || token >= P.g.max_tokens)
        return 0;
    if (!P.lw || !P.lw[L].d) {
        set_err("layer %d has no weights on the device (ds4f_gpu_attn_weights)", L);
        return -1;
    }
    if (forced_failure()) return fail_over(token);
    const size_t bytes = (size_t)P.hidden * sizeof(float);
    if (ensure_stage(0, bytes) != 0) return fail_over(token);
    memcpy(P.h_stage, state, bytes);
    if (hipMemcpyAsync(P.d_state, P.h_stage, bytes, hipMemcpyHostToDevice, P.stream) !=
            hipSuccess ||
        ds4f_hip_attn_step_async(L, token, P.d_state, NULL) != 0 ||
        download(P.d_state, bytes) != 0)
        return fail_over(token);
    memcpy(state, P.h_stage, bytes);
    return 0;
}


/* ---- whole-layer chunks (ds4f_attn_gqa_chunk :1145-1252,
 * ds4f_attn_linear_chunk :977-1135) ------------------------------------- */

/* chunk workspace of mpad token rows: X operands (hi, lo, group sums) for
 * K up to 4096, the projection outputs of either layer kind, the core's
 * output; grow-only */
enum { CH_Q, CH_K, CH_V, CH_AO, CH_QKV, CH_Z, CH_A, CH_B, CH_LO, CH_N };

static size_t ch_width(int i) {
    switch (i) {
    case CH_Q: return (size_t)P.g.n_heads * 2 * GQA_D;
    case CH_K: case CH_V: return (size_t)P.g.n_kv_heads * GQA_D;
    case CH_AO: return (size_t)P.g.n_heads * GQA_D;
    case CH_QKV: return (size_t)P.rows;
    case CH_Z: case CH_LO: return (size_t)P.vh * P.vd;
    default: return (size_t)P.vh;
    }
}

static size_t ch_kmax(void) {
    size_t k = (size_t)P.hidden;
    if (ch_width(CH_AO) > k) k = ch_width(CH_AO);
    if (ch_width(CH_LO) > k) k = ch_width(CH_LO);
    return k;
}

typedef struct { uint16_t *xw; float *xsum; float *out[CH_N]; } ChunkWs;

/* byte offsets of the workspace parts for mpad rows; the total when ws is
 * NULL, else ws filled with pointers into P.d_chunk */
static size_t chunk_layout(int mpad, ChunkWs *ws) {
    const size_t K = ch_kmax();
    size_t sizes[2 + CH_N], off[2 + CH_N], total = 0;
    sizes[0] = (size_t)mpad * K * 4;            /* fp16 hi and lo */
    sizes[1] = (K / 64) * (size_t)mpad * 4;
    for (int i = 0; i < CH_N; i++) sizes[2 + i] = (size_t)mpad * ch_width(i) * 4;
    for (int i = 0; i < 2 + CH_N; i++) {
        off[i] = total;
        total += (sizes[i] + 255) & ~(size_t)255;
    }
    if (ws) {
        char *b = (char *)P.d_chunk;
        ws->xw = (uint16_t *)(b + off[0]);
        ws->xsum = (float *)(b + off[1]);
        for (int i = 0; i < CH_N; i++) ws->out[i] = (float *)(b + off[2 + i]);
    }
    return total;
}

/* The workspace grows to hold mpad = B rounded up to the GEMM's M tile;
 * the parts' base pointers follow the capacity, and a call lays its X
 * operand, group sums and outputs over its own mpad rows inside them.
 * Growth frees the old buffer: a HIP graph captured over it must be
 * captured again (a caller that captures prefill chunks makes its largest
 * chunk first, outside the capture). */
static int ensure_chunk(int B, ChunkWs *ws, int *mpad_out) {
    const int mt = q35_mlx4_gemm_mtile();
    const int mpad = (B + mt - 1) / mt * mt;
    *mpad_out = mpad;
    if (mpad > P.chunk_cap) {
        /* grow-only, by at least half, in whole token tiles */
        int cap = P.chunk_cap + P.chunk_cap / 2;
        cap = (cap + mt - 1) / mt * mt;
        if (cap < mpad) cap = mpad;
        if (P.d_chunk) {
            HIPCHK(hipStreamSynchronize(P.stream));
            hipFree(P.d_chunk);
        }
        P.d_chunk = NULL;
        P.chunk_cap = 0;
        HIPCHK(hipMalloc(&P.d_chunk, chunk_layout(cap, NULL)));
        P.chunk_cap = cap;
    }
    chunk_layout(P.chunk_cap, ws);
    return 0;
}

/* X = [norm](x rows) (x NULL: the workspace already holds X over mpad
 * rows), then y = X W^T for the njobs GEMM jobs, job j writing ys[j]
 * [B][lds[j]] */
static int chunk_gemm(const float *x, int ldx, const uint16_t *norm_w, int K, int B, int mpad,
                      const Q35Mlx4GemmJob *jobs, int njobs, float *const *ys, const int *lds,
                      int accumulate, const ChunkWs *ws, hipStream_t st) {
    if (x) {
        Q35Mlx4Xprep xp = {x, norm_w, ws->xw, ws->xsum, B, mpad, K, ldx, P.d_status_cur};
        HIPCHK(q35_mlx4_xprep(&xp, st));
    }
    Q35Mlx4Gemm g;
    memset(&g, 0, sizeof g);
    g.xw = ws->xw;
    g.xsum = ws->xsum;
    for (int j = 0; j < njobs; j++) {
        g.jobs[j] = jobs[j];
        g.jobs[j].y = ys[j];
        g.jobs[j].ldy = lds[j];
    }
    g.njobs = njobs;
    g.M = B;
    g.Mpad = mpad;
    g.K = K;
    g.accumulate = accumulate;
    HIPCHK(q35_mlx4_gemm(&g, st));
    return 0;
}

int ds4f_hip_attn_chunk_async(int L, int t0, int B, float *states, void *stream) {
    if (!P.ok || P.disabled || !P.bound) {
        set_err("plugin not bound or disabled");
        return -1;
    }
    if (L < 0 || L >= P.g.n_layers) {
        set_err("layer chunk: layer %d outside [0, %d)", L, P.g.n_layers);
        return -1;
    }
    const int kind = P.kind[L];
    if (kind == DS4F_LAYER_NONE || layer_skipped(L) || B < 1) return 0;
    if (!P.lw || !P.lw[L].d) {
        set_err("layer %d has no weights on the device (ds4f_gpu_attn_weights)", L);
        return -1;
    }
    if (t0 < 0 || t0 >= P.g.max_tokens) return 0;           /* :117, :882 */
    if (B > P.g.max_tokens - t0) B = P.g.max_tokens - t0;
    if (P.hidden % 64 != 0 || ch_kmax() % 64 != 0) {
        set_err("chunk GEMM needs widths that are multiples of 64");
        return -1;
    }
    const LayerW *lw = &P.lw[L];
    hipStream_t st = pick(stream);
    ChunkWs ws;
    int mpad;
    if (ensure_chunk(B, &ws, &mpad) != 0) return -1;
    const int H = P.hidden;
    /* the projections of the B normed rows */
    const int outs[4] = {kind == DS4F_LAYER_GQA ? CH_Q : CH_QKV, kind == DS4F_LAYER_GQA ? CH_K : CH_Z,
                         kind == DS4F_LAYER_GQA ? CH_V : CH_A, CH_B};
    float *ys[4];
    int lds[4];
    for (int j = 0; j < lw->njobs; j++) {
        ys[j] = ws.out[outs[j]];
        lds[j] = (int)ch_width(outs[j]);
    }
    if (chunk_gemm(states, H, lw->in_norm, H, B, mpad, lw->gj, lw->njobs, ys, lds, 0, &ws, st) != 0)
        return -1;
    /* the core over the chunk */
    int core_out;
    if (kind == DS4F_LAYER_GQA) {
        if (ds4f_hip_gqa_prefill_async(L, t0, B, ws.out[CH_Q], ws.out[CH_K], ws.out[CH_V], lw->qn,
                                       lw->kn, ws.out[CH_AO], NULL, st) != 0)
            return -1;
        core_out = CH_AO;
    } else {
        /* the gated norm writes the output GEMM's X operand directly */
        if (lin_prefill_launch(L, t0, B, ws.out[CH_QKV], ws.out[CH_Z], ws.out[CH_A], ws.out[CH_B],
                               lw->conv_w, lw->A_log, lw->dt_bias, lw->norm_w, ws.out[CH_LO], NULL,
                               ws.xw, ws.xsum, mpad, NULL, 0, st) != 0)
            return -1;
        core_out = -1;
    }
    /* the output projection, added to the rows' states */
    float *yo[1] = {states};
    const int ldo[1] = {H};
    const int K = (int)ch_width(kind == DS4F_LAYER_GQA ? CH_AO : CH_LO);
    return chunk_gemm(core_out >= 0 ? ws.out[core_out] : NULL, K, NULL, K, B, mpad,
                      lw->gj + lw->njobs, 1, yo, ldo, 1, &ws, st);
}

int ds4f_gpu_attn_chunk(int L, int t0, int B, float *const *states) {
    if (!P.ok || P.disabled || !P.bound) {
        set_err("plugin not bound or disabled");
        return -1;
    }
    if (L < 0 || L >= P.g.n_layers) {
        set_err("layer chunk: layer %d outside [0, %d)", L, P.g.n_layers);
        return -1;
    }
    if (P.kind[L] == DS4F_LAYER_NONE || layer_skipped(L) || B < 1 || t0 < 0 ||
        t0 >= P.g.max_tokens)
        return 0;
    if (!P.lw || !P.lw[L].d) {
        set_err("layer %d has no weights on the device (ds4f_gpu_attn_weights)", L);
        return -1;
    }
    if (forced_failure()) return fail_over(t0);
    if (B > P.g.max_tokens - t0) B = P.g.max_tokens - t0;
    const size_t row = (size_t)P.hidden * sizeof(float), bytes = (size_t)B * row;
    if (bytes > P.h_states_cap) {
        if (P.h_states) hipHostFree(P.h_states);
        P.h_states = NULL;
        P.h_states_cap = 0;
        if (hipHostMalloc((void **)&P.h_states, bytes, hipHostMallocDefault) != hipSuccess) {
            set_err("chunk: pinned staging failed");
            return fail_over(t0);
        }
        P.h_states_cap = bytes;
    }
    if (ensure_stage(bytes, 0) != 0) return fail_over(t0);
    const int lin = P.kind[L] == DS4F_LAYER_LINEAR;
    const size_t sb = lin_floats() * sizeof(float), cb = conv_floats() * sizeof(float);
    if (lin && !P.d_backup && hipMalloc((void **)&P.d_backup, sb + cb) != hipSuccess) {
        set_err("chunk: state backup allocation failed");
        return fail_over(t0);
    }
    for (int b = 0; b < B; b++) memcpy((char *)P.h_states + b * row, states[b], row);
    float *d_states = (float *)P.d_stage;
    int bits = 0;
    /* a delta-rule layer's state and ring are kept until the chunk is known
     * to be good: a recomputation starts from them */
    if ((lin && (hipMemcpyAsync(P.d_backup, layer_lin(P.slot[L]), sb, hipMemcpyDeviceToDevice,
                                P.stream) != hipSuccess ||
                 hipMemcpyAsync((char *)P.d_backup + sb, layer_conv(P.slot[L]), cb,
                                hipMemcpyDeviceToDevice, P.stream) != hipSuccess)) ||
        hipMemcpyAsync(d_states, P.h_states, bytes, hipMemcpyHostToDevice, P.stream) != hipSuccess ||
        host_status_begin() != 0)
        return fail_over(t0);
    if (ds4f_hip_attn_chunk_async(L, t0, B, d_states, NULL) != 0) {
        host_status_end(NULL);
        return fail_over(t0);
    }
    if (host_status_end(&bits) != 0) return fail_over(t0);
    if (bits) {
        /* a GEMM or attention operand beyond fp16 range: the chunk again as
         * B layer steps on the decode kernels (fp32 activations, bf16 cache),
         * from the states and the layer state the chunk started from */
        if ((lin && (hipMemcpyAsync(layer_lin(P.slot[L]), P.d_backup, sb, hipMemcpyDeviceToDevice,
                                    P.stream) != hipSuccess ||
                     hipMemcpyAsync(layer_conv(P.slot[L]), (char *)P.d_backup + sb, cb,
                                    hipMemcpyDeviceToDevice, P.stream) != hipSuccess)) ||
            hipMemcpyAsync(d_states, P.h_states, bytes, hipMemcpyHostToDevice, P.stream) !=
                hipSuccess)
            return fail_over(t0);
        for (int b = 0; b < B; b++)
            if (ds4f_hip_attn_step_async(L, t0 + b, d_states + (size_t)b * P.hidden, NULL) != 0)
                return fail_over(t0);
    }
    if (hipMemcpyAsync(P.h_states, d_states, bytes, hipMemcpyDeviceToHost, P.stream) != hipSuccess ||
        hipStreamSynchronize(P.stream) != hipSuccess)
        return fail_over(t0);
    for (int b = 0; b < B; b++) memcpy(states[b], (char *)P.h_states + b * row, row);
    return 0;
}
