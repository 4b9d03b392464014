/*
 * q35_launch.h -- launchers of the gfx950 kernels, callable from the C99
 * shim (gpu_hip.c).  Every pointer is a device pointer; every launcher only
 * enqueues on `stream` and returns the launch status.
 *
 * Device layouts (all chosen for the MFMA operand shapes of gfx950):
 *   K cache  bf16, per kv head, 16-token x 32-dim blocks:
 *            [kvh][T/16][D/32][16 tok][32 dim]  -- one block is exactly one
 *            16x16x32 MFMA operand (1 KiB, contiguous)
 *   V cache  bf16, per kv head, 16-token tiles stored dim-major:
 *            [kvh][T/16][D][16 tok]             -- 16 dims of a tile are one
 *            16x16x16 MFMA operand (512 B, contiguous)
 *   delta state  fp32, value-major per head: [vh][vd][kd]; one value column
 *            is 512 B contiguous
 *   conv ring    fp32 [4][rows], slot = token % 4 (the reference's ring)
 * T is the padded token capacity (a multiple of 64).
 */
#ifndef Q35_LAUNCH_H
#define Q35_LAUNCH_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bits of the status word the prefill kernels set (q35_f16_guard): a value
 * out of fp16 range met by the GQA prefill's operand conversion, or by the
 * chunk GEMM's X operand (its X prep or the delta-rule gated norm). */
#define Q35_STATUS_GQA_F16  1
#define Q35_STATUS_GEMM_F16 2

/* ---- gated delta-rule decode (kd = vd = 128) ---- */
typedef struct Q35LinDecode {
    const float *qkv, *z, *a, *b;
    const uint16_t *conv_w, *dt_bias, *norm_w;
    const float *A_log;
    float *ring;       /* [4][rows] */
    float *state;      /* [vh][vd][kd] */
    float *out;        /* [vh*vd] */
    float *qkv_post;   /* optional [rows] */
    int token, k_heads, v_heads;
} Q35LinDecode;
hipError_t q35_lin_decode(const Q35LinDecode *p, hipStream_t stream);

/* ---- gated delta-rule prefill, chunked (chunk 64, kd = vd = 128) ---- *
 * Workspaces (fp32), nc = ceil(B/64), VH value heads:
 *   post  [B][rows]          post-conv, normed q | k | v (the caller's
 *                            qkv_post, or a workspace)
 *   gates [B][VH][2]         (log-decay g, beta)
 *   T, Pm [nc][VH][64][64]   (I + A)^-1 and the masked decayed Q K^T
 *   gvec  [nc][VH][Q35_LIN_GVEC]  exp(G_t) | exp(G_C - G_t) | beta_t | exp(G_C) */
#define Q35_LIN_GVEC 256
typedef struct Q35LinPrefill {
    const float *qkv, *z, *a, *b;  /* [B][rows], [B][VH*VD], [B][VH], [B][VH] */
    const uint16_t *conv_w, *dt_bias, *norm_w;
    const float *A_log;
    float *ring;                   /* [4][rows] */
    float *state;                  /* [vh][vd][kd] */
    float *out;                    /* [B][VH*VD] */
    float *post, *gates, *T, *Pm, *gvec;
    int t0, B, n_chunks, k_heads, v_heads;
    /* xw non-NULL: the gated norm writes its rows as the chunk GEMM's X
     * operand (xw, xsum over mpad rows, mlx4_gemm.hip) instead of into out,
     * which then only carries the scan's rows */
    uint16_t *xw;
    float *xsum;
    int mpad;
    int *status;                   /* Q35_STATUS_GEMM_F16 (xw path), or NULL */
} Q35LinPrefill;
/* workspace bytes, post included when with_post != 0 */
void q35_lin_prefill_ws_bytes(int B, int k_heads, int v_heads, int with_post, size_t *bytes);
hipError_t q35_lin_prefill(const Q35LinPrefill *p, hipStream_t stream);
/* The static device workspace of the no-allocation prefill entry: 8 MiB,
 * one per GPU, for chunks of at most Q35_LIN_NOALLOC_MAX_B tokens (6.1 MiB
 * at 16 key / 32 value heads with the post rows in the workspace).
 * q35_lin_scratch_init takes its device address on the current device
 * (once per device); q35_lin_scratch returns it for the current device
 * (NULL before the init). */
#define Q35_LIN_SCRATCH_BYTES ((size_t)8 << 20)
#define Q35_LIN_NOALLOC_MAX_B 128
hipError_t q35_lin_scratch_init(void);
void *q35_lin_scratch(void);

/* ---- GQA split-K decode (head_dim 256, 8 q heads per kv head) ---- */
typedef struct Q35GqaDecode {
    const float *q_gate;           /* [H][2D] */
    const float *k_new, *v_new;    /* [KVH][D] */
    const uint16_t *qn_w, *kn_w;
    const float *rope;             /* this position: cos[rd/2] then sin[rd/2] */
    uint16_t *kt, *vt;             /* this layer's K / V tiles */
    float *part_o;                 /* [KVH][P][8][D] */
    float *part_ml;                /* [KVH][P][8][2] */
    float *attn_out;               /* [H][D] */
    float *k_post;                 /* optional [KVH][D] */
    int token;                     /* position; cache rows [0, token) are past */
    int t_tiles;                   /* T/16 of this layer's tiles */
    int heads, kv_heads;
    int chunk, n_chunks;           /* positions per workgroup, P */
} Q35GqaDecode;
hipError_t q35_gqa_decode(const Q35GqaDecode *p, hipStream_t stream);
/* P and chunk for a step with n_past cached rows. */
void q35_gqa_split(int n_past, int *chunk, int *n_chunks);
int q35_gqa_max_chunks(void);

/* ---- GQA prefill: causal flash attention over B new tokens ---- *
 * Workspaces (fp16 bits, filled by the prep kernels; q is read from q_gate
 * by the attention kernel itself):
 *   kw  [KVH][kbt][32 keys][D]                kbt = ceil((t0+B)/32)
 *   vw  [KVH][kbt][D][32 keys, MFMA order]
 * q35_gqa_prefill_ws_bytes() gives the two sizes. */
typedef struct Q35GqaPrefill {
    const float *q_gate;           /* [B][H][2D] */
    const float *k_in, *v_in;      /* [B][KVH][D] */
    const uint16_t *qn_w, *kn_w;
    const float *rope;             /* table [max_tokens][rd]: cos then sin */
    uint16_t *kt, *vt;             /* this layer's K / V cache tiles */
    uint16_t *kw, *vw;             /* fp16 workspaces */
    float *attn_out;               /* [B][H][D] */
    float *k_post;                 /* optional [B][KVH][D] */
    int t0, B, t_tiles, heads, kv_heads;
    int nqb, kbt;
    int *status;                   /* Q35_STATUS_GQA_F16, or NULL */
} Q35GqaPrefill;
void q35_gqa_prefill_ws_bytes(int t0, int B, int kv_heads, size_t *kw, size_t *vw);
hipError_t q35_gqa_prefill(const Q35GqaPrefill *p, hipStream_t stream);

/* ---- state movement between host row layouts and device layouts ---- */
/* rows [p0, p0+n) of a host-layout fp32 block [n][2*KVH*D] <-> tiles */
hipError_t q35_kv_import(const float *rows, int p0, int n, uint16_t *kt, uint16_t *vt,
                         int t_tiles, int kv_heads, hipStream_t stream);
hipError_t q35_kv_export(float *rows, int p0, int n, const uint16_t *kt,
                         const uint16_t *vt, int t_tiles, int kv_heads, hipStream_t stream);
/* [vh][kd][vd] <-> [vh][vd][kd] */
hipError_t q35_state_transpose(const float *src, float *dst, int heads, int rows, int cols,
                               hipStream_t stream);

/* ---- synthetic streams ---- */
hipError_t q35_synth(void *dst, int64_t n, int dtype, int dist, double p0, double p1,
                     uint64_t seed, uint64_t tid, hipStream_t stream);
hipError_t q35_synth_kv(uint16_t *kt, uint16_t *vt, int n_past, int t_tiles, int kv_heads,
                        uint64_t seed, uint64_t tid_k, uint64_t tid_v, hipStream_t stream);
hipError_t q35_synth_state(float *state, int heads, int kd, int vd, double sigma,
                           uint64_t seed, uint64_t tid, hipStream_t stream);
hipError_t q35_synth_conv(float *ring, int rows, int token, uint64_t seed, uint64_t tid,
                          hipStream_t stream);

/* n launches of an empty kernel of `grid` workgroups of `block` threads */
hipError_t q35_empty_kernels(int n, int grid, int block, hipStream_t stream);

/* ---- MLX 4-bit affine matvec (src/kernels.c:104-219) ---- *
 * y[R] = W[R x C] x, W as U32 nibble words + BF16 scale / bias per 64
 * elements (biases may be NULL).  One job: the inline pointers, jobs NULL.
 * Batched: jobs points to njobs device descriptors sharing C; a job's R
 * is its own when non-zero, else the launch's R (R is the largest), and a
 * job's x is its own when non-NULL, else the launch's x.
 * x_norm: when non-NULL, every job reads RMSNorm(x) with these BF16
 * weights (the input_layernorm of src/attn_qwen.c:142-157: double sum of
 * squares, eps 1e-6 on the mean, x / r * w) instead of x.  accumulate:
 * y += W x (the residual add of :222, :833) instead of y = W x. */
typedef struct Q35Mlx4Job {
    const uint32_t *vals;
    const uint16_t *scales, *biases;
    const float *x;
    float *y;
    int R;
} Q35Mlx4Job;
typedef struct Q35Mlx4 {
    const uint32_t *vals;
    const uint16_t *scales, *biases;
    const float *x;
    float *y;
    const Q35Mlx4Job *jobs;        /* device array, or NULL for the inline job */
    int R, C;
    const uint16_t *x_norm;
    int accumulate;
} Q35Mlx4;
/* 1 if the kernel takes this shape: C % 32 == 0, 32 <= C <= 8192 */
int q35_mlx4_supported(int R, int C);
hipError_t q35_mlx4_matvec(const Q35Mlx4 *p, int njobs, hipStream_t stream);

/* ---- MLX 4-bit projections of a prefill chunk on MFMA (mlx4_gemm.hip) ----
 * Y[M][N] = X[M][K] W^T for [N x K] 4-bit weights, K % 64 == 0.  X goes
 * through q35_mlx4_xprep first (optional RMSNorm, fp16 hi / lo in word
 * order, tiled per 64 rows and group; group sums); the weight's scales /
 * biases through q35_mlx4_sb once ((16 s, b - 16 s) per group and row). */
typedef struct Q35Mlx4Xprep {
    const float *x;                /* [M][ldx] */
    const uint16_t *norm_w;        /* [K] or NULL */
    uint16_t *xw;                  /* Mpad * K * 2 halfs: hi / lo blocks per (64-row tile, group) */
    float *xsum;                   /* [K/64][Mpad] */
    int M, Mpad, K, ldx;
    int *status;                   /* Q35_STATUS_GEMM_F16, or NULL */
} Q35Mlx4Xprep;
typedef struct Q35Mlx4SB {
    float s, b;                    /* 16 scale, bias - 16 scale */
} Q35Mlx4SB;
#define Q35_GEMM_MAX_JOBS 4
typedef struct Q35Mlx4GemmJob {
    const uint32_t *vals;          /* the words re-laid out by q35_mlx4_wt */
    const Q35Mlx4SB *sb;           /* [K/64][q35_mlx4_sb_npad(N)] */
    float *y;                      /* [M][ldy] */
    int N, ldy;
} Q35Mlx4GemmJob;
/* the jobs ride in the kernel arguments; one launch covers every job's
 * 256-feature tiles */
typedef struct Q35Mlx4Gemm {
    const uint16_t *xw;
    const float *xsum;
    Q35Mlx4GemmJob jobs[Q35_GEMM_MAX_JOBS];
    int njobs, M, Mpad, K, accumulate;   /* accumulate: y += instead of y = */
} Q35Mlx4Gemm;
/* the (s, b') table of an N-row weight with G groups a row: G x npad(N) */
int q35_mlx4_sb_npad(int N);
hipError_t q35_mlx4_sb(const uint16_t *scales, const uint16_t *biases, Q35Mlx4SB *sb, int N, int G,
                       hipStream_t stream);
/* the weight words [N][K/8] re-laid out for the GEMM's staging:
 * npad(N) * K / 2 bytes */
hipError_t q35_mlx4_wt(const uint32_t *vals, uint32_t *wt, int N, int K, hipStream_t stream);
hipError_t q35_mlx4_xprep(const Q35Mlx4Xprep *p, hipStream_t stream);
hipError_t q35_mlx4_gemm(const Q35Mlx4Gemm *p, hipStream_t stream);
int q35_mlx4_gemm_mtile(void);      /* Mpad must be a multiple of this */

#ifdef __cplusplus
}
#endif


#endif /* Q35_LAUNCH_H */
