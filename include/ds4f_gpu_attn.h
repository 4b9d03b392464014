/*
 * ds4f_gpu_attn.h -- HIP (gfx950) attention plugin for the Qwen3.5 hybrid
 * stack: the C ABI a sibling of src/gpu_stub.c / src/gpu_metal.mm exports.
 *
 * Conventions are the ones include/ds4f/gpu.h fixes for the engine's GPU
 * plugin (gpu.h:6-8, :20-21):
 *   - plain C, extern "C", caller-owned plain pointers and sizes;
 *   - return 0 when the work was done, -1 when the GPU is unavailable or
 *     the call failed -- the caller then runs its CPU path;
 *   - after the first failure the plugin stays disabled (the sticky
 *     fallback of src/head.c:283) and device state has been written back
 *     to the bound host arrays, so the CPU path continues exactly.
 *
 * The reference has no attention entry points in gpu.h; the ones below are
 * the call sites inside src/attn_qwen.c they replace:
 *   ds4f_gpu_gqa_decode   <- gqa_body :279-396 (norms, RoPE, cache write,
 *                            softmax attention, sigmoid gate)
 *   ds4f_gpu_lin_decode   <- lin_body :470-764 (conv1d+SiLU, q/k norm,
 *                            gates, gated delta rule, RMSNormGated)
 *   ds4f_gpu_gqa_prefill  <- the serial gqa_body loop of
 *                            ds4f_attn_gqa_chunk :1222-1231
 *   ds4f_gpu_lin_prefill  <- the serial lin_body loop of
 *                            ds4f_attn_linear_chunk :1088-1109
 * and the state container they act on is the engine's Ds4fKvCache
 * (include/ds4f/attn.h:26-42), bound once with ds4f_gpu_attn_bind.
 *
 * Activations cross the host ABI as float (the reference's float*), weights
 * as the raw trunk bits (bf16 as uint16_t, A_log as float).  The device keeps
 * the KV cache in bf16 (GQA layers only), the delta-rule state in fp32 and
 * the conv ring in fp32; host arrays are stale until ds4f_gpu_attn_sync.
 *
 * Threading: single caller, one HIP stream, static device state (as
 * src/gpu_metal.mm:16-23).  Calls that overlap race.
 */
#ifndef DS4F_GPU_ATTN_H
#define DS4F_GPU_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- lifecycle (include/ds4f/gpu.h:22-23) ------------------------------ */
int  ds4f_gpu_init(void);
void ds4f_gpu_free(void);

/* Layer kinds, decided by the engine the way ds4f_attn_qwen_step does
 * (src/attn_qwen.c:1259-1263: q3_q role -> GQA, q3_conv/q3_pqkv -> linear). */
#define DS4F_LAYER_NONE   0
#define DS4F_LAYER_LINEAR 1
#define DS4F_LAYER_GQA    2

/* Geometry, in the reference's terms (src/attn_qwen.c:249-252, :451-453):
 * GQA q heads = linear key heads = n_heads, GQA kv heads = n_kv_heads,
 * linear value heads = 16 * n_kv_heads, kd = vd = 128, head_dim = 256. */
typedef struct Ds4fGpuAttnGeom {
    int n_layers;    /* Ds4fKvCache.n_layers */
    int max_tokens;  /* Ds4fKvCache.max_tokens */
    int n_heads;     /* cfg->n_heads */
    int n_kv_heads;  /* cfg->n_kv_heads */
    int head_dim;    /* GQA head dim (krows / kv_heads) */
    int lin_kd;      /* delta-rule key dim (128) */
    int lin_vd;      /* delta-rule value dim (128) */
} Ds4fGpuAttnGeom;

/* Bind the engine's state arrays (the Ds4fKvCache fields kv / lin / conv,
 * allocated by ds4f_kv_init / _lin_init / _conv_init, src/attn.c:27-91):
 *   host_kv   [n_layers][max_tokens][2*n_kv_heads*head_dim] or NULL
 *   host_lin  [n_layers][16*n_kv_heads][lin_kd][lin_vd]     or NULL
 *   host_conv [n_layers][4][conv_rows]                      or NULL
 * with conv_rows = 2*n_heads*lin_kd + 16*n_kv_heads*lin_vd.  Allocates the
 * device mirrors (KV only for GQA layers) and uploads the first
 * n_kv_tokens cache rows plus the whole lin/conv arrays; NULL arrays start
 * as zeros on the device.  Rebinding replaces the previous binding. */
int ds4f_gpu_attn_bind(const Ds4fGpuAttnGeom *geom, const int *layer_kind,
                       float *host_kv, float *host_lin, float *host_conv,
                       int n_kv_tokens);
int ds4f_gpu_attn_unbind(void);

/* Move state between the device mirrors and the bound host arrays.
 * L = -1: every layer.  n_kv_tokens: cache rows [0, n) to move. */
#define DS4F_SYNC_TO_HOST   0
#define DS4F_SYNC_TO_DEVICE 1
int ds4f_gpu_attn_sync(int L, int dir, int n_kv_tokens);

/* ---- host-pointer entry points (synchronous on return) ---------------- */

/* One decode token of a GQA layer (gqa_body :279-396).
 *   q_gate   [n_heads][2*head_dim]  (q | gate per head)
 *   k        [n_kv_heads][head_dim] normed + rotated in place, as the
 *            reference mutates its k (:292-293, :317-325)
 *   v        [n_kv_heads][head_dim]
 *   attn_out [n_heads][head_dim]
 * token >= max_tokens or < 0 is the reference's silent skip (:256):
 * returns 0 with nothing written. */
int ds4f_gpu_gqa_decode(int L, int token, const float *q_gate, float *k,
                        const float *v, const uint16_t *qn_w,
                        const uint16_t *kn_w, float *attn_out);

/* One decode token of a gated delta-rule layer (lin_body :470-764).
 *   qkv  [conv_rows] raw projection in; post-conv, normed values out
 *        (the reference mutates it in place: :503, :535)
 *   z    [16*n_kv_heads*lin_vd]; a, b [16*n_kv_heads] (in_proj_a/b outputs)
 *   out  [16*n_kv_heads*lin_vd] gated normed readout (the o_proj input) */
int ds4f_gpu_lin_decode(int L, int token, float *qkv, const float *z,
                        const float *a, const float *b,
                        const uint16_t *conv_w, const float *A_log,
                        const uint16_t *dt_bias, const uint16_t *norm_w,
                        float *out);

/* Prefill of B tokens t0..t0+B-1 of a GQA layer: the results of B
 * ds4f_gpu_gqa_decode calls in order, computed as one causal flash
 * attention (fp16 MFMA).  Arrays are [B][...] of the decode shapes. */
int ds4f_gpu_gqa_prefill(int L, int t0, int B, const float *q_gate, float *k,
                         const float *v, const uint16_t *qn_w,
                         const uint16_t *kn_w, float *attn_out);

/* Prefill of B tokens t0..t0+B-1 of a delta-rule layer: the results of B
 * ds4f_gpu_lin_decode calls in order (up to fp32 rounding), computed in
 * chunked WY form (64-token chunks, fp32 MFMA).  qkv [B][conv_rows] is
 * mutated like the decode's; z / out [B][16*n_kv_heads*lin_vd], a / b
 * [B][16*n_kv_heads]. */
int ds4f_gpu_lin_prefill(int L, int t0, int B, float *qkv, const float *z,
                         const float *a, const float *b,
                         const uint16_t *conv_w, const float *A_log,
                         const uint16_t *dt_bias, const uint16_t *norm_w,
                         float *out);

/* ---- device-pointer entry points (enqueue only) ----------------------- *
 * The same operations with every tensor already in device memory; they
 * enqueue on `stream` (a hipStream_t; NULL = the plugin's stream) and
 * return without waiting, so a caller can keep inputs resident in HBM and
 * capture the launches in a HIP graph.  k_post / qkv_post may be NULL. */
int ds4f_hip_gqa_decode_async(int L, int token, const float *q_gate,
                              const float *k, const float *v,
                              const uint16_t *qn_w, const uint16_t *kn_w,
                              float *attn_out, float *k_post, void *stream);
/* Prefill of B tokens t0.. of a GQA layer (fp16 MFMA flash attention).
 * The first call allocates the fp16 K / V workspace for the whole cache
 * (max_tokens positions: every later t0 + B fits) and is not capturable;
 * later calls allocate nothing unless a delta-rule prefill has since grown
 * the shared workspace, which frees the previous one, so a HIP graph
 * captured before such growth must be captured again. */
int ds4f_hip_gqa_prefill_async(int L, int t0, int B, const float *q_gate,
                               const float *k, const float *v,
                               const uint16_t *qn_w, const uint16_t *kn_w,
                               float *attn_out, float *k_post, void *stream);
/* Prefill of B tokens t0.. of a delta-rule layer (chunked form).  qkv_post
 * [B][conv_rows] receives the post-conv, normed values (may be NULL).
 * Allocates its workspace (sized by B) on first use or when B exceeds
 * every earlier call's (not capturable then; growth is by at least half);
 * growth frees the previous workspace, so a HIP graph captured before it
 * must be captured again. */
int ds4f_hip_lin_prefill_async(int L, int t0, int B, const float *qkv,
                               const float *z, const float *a, const float *b,
                               const uint16_t *conv_w, const float *A_log,
                               const uint16_t *dt_bias, const uint16_t *norm_w,
                               float *out, float *qkv_post, void *stream);
/* The delta-rule prefill of ds4f_hip_lin_prefill_async with no allocation:
 * no counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  The kernels and the results are those of
 * ds4f_hip_lin_prefill_async; the workspace is one static 8 MiB device array
 * per GPU instead of the plugin's grow-only buffer, so a call takes at most
 * 128 tokens (two 64-token chunks; 6.1 MiB of workspace at 16 key / 32
 * value heads).  A larger B (after the clip at max_tokens), or a geometry
 * whose workspace exceeds the array, returns -1 (error text in
 * ds4f_gpu_last_error) with nothing launched.  Every call on one GPU uses
 * that GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race. */
int ds4f_hip_lin_prefill_noalloc(int L, int t0, int B, const float *qkv,
                                 const float *z, const float *a, const float *b,
                                 const uint16_t *conv_w, const float *A_log,
                                 const uint16_t *dt_bias, const uint16_t *norm_w,
                                 float *out, float *qkv_post, void *stream);
int ds4f_hip_lin_decode_async(int L, int token, const float *qkv,
                              const float *z, const float *a, const float *b,
                              const uint16_t *conv_w, const float *A_log,
                              const uint16_t *dt_bias, const uint16_t *norm_w,
                              float *out, float *qkv_post, void *stream);

/* ---- synthetic state for benchmarks and tests ------------------------- *
 * Fill device memory with the splitmix64 / Box-Muller streams of the
 * workload generator (seed, tensor id; index = logical element index).
 * dtype 0 = float32, 1 = bf16, 2 = float32 holding the bf16-rounded value;
 * dist 0 = normal(p0 = mean, p1 = sigma),
 * 1 = uniform(p0 = lo, p1 = hi). */
int ds4f_hip_synth(void *dst, int64_t n, int dtype, int dist, double p0,
                   double p1, uint64_t seed, uint64_t tid, void *stream);
/* Bound GQA layer L: cache rows [0, n_past) drawn bf16 N(0,1) in the
 * reference row order [pos][kv_head][dim] (streams tid_k, tid_v). */
int ds4f_hip_synth_gqa_cache(int L, int n_past, uint64_t seed, uint64_t tid_k,
                             uint64_t tid_v, void *stream);
/* Bound linear layer L: state N(0, sigma) in the order [vh][kd][vd]; conv
 * ring rows of positions token-3..token-1 drawn N(0,1) as [3][conv_rows]. */
int ds4f_hip_synth_lin_state(int L, double sigma, uint64_t seed, uint64_t tid,
                             void *stream);
int ds4f_hip_synth_conv_history(int L, int token, uint64_t seed, uint64_t tid,
                                void *stream);

/* ---- measurement ------------------------------------------------------ *
 * Enqueue n launches of a kernel that does nothing (grid workgroups of
 * block threads) on `stream`: captured in a HIP graph, they time the fixed
 * cost of a kernel boundary, the floor of every latency-bound launch.  No
 * counterpart in the reference. */
int ds4f_hip_launch_floor(int n, int grid, int block, void *stream);

/* ---- the MLX-4bit matvecs of include/ds4f/gpu.h (:29-54) --------------- *
 * y = W x for an MLX 4-bit affine [R x C] weight in the layout of
 * ds4f_mlx4_matvec (src/kernels.c:104-219): U32 words of 8 nibbles, low
 * nibble first, BF16 scale and optional BF16 bias per 64 elements of the
 * flattened matrix, w = q * scale + bias.  Host pointers; the result is in
 * y on return.  Shapes with C % 32 == 0 and 32 <= C <= 8192 run on the
 * GPU; any other shape, or an uninitialised plugin, returns -1 (the
 * caller runs its CPU matvec), as gpu.h specifies.  Results differ from
 * the CPU path by float32 summation order only (gpu.h:13-18).
 *
 * ds4f_gpu_mlx4_matvec replaces the Metal/stub function of the same name
 * (src/gpu_metal.mm:83-128, src/gpu_stub.c); the weight is uploaded once
 * and kept on the device while the vals pointer and shape stay the same
 * (the output head). */
int ds4f_gpu_mlx4_matvec(const uint32_t *vals, const uint16_t *scales,
                         const uint16_t *biases, int R, int C,
                         const float *x, float *y);
/* Batched expert matvec (gpu.h:31-54): y[j] = W_j x_j, every job sharing
 * R and C; weights are cached per stable id ids[j] (first sight uploads);
 * one dispatch for the batch.  biases may be NULL (no biases) or hold NULL
 * entries. */
int ds4f_gpu_mlx4_batch(const uint32_t *const *vals,
                        const uint16_t *const *scales,
                        const uint16_t *const *biases,
                        const float *const *xs, float *const *ys,
                        const void *const *ids, int R, int C, int njobs);
/* Device-resident form of ds4f_mlx4_matvec (src/kernels.c:158-219): all
 * pointers are device memory, the call only enqueues on `stream` (NULL:
 * the plugin's stream).  For callers that keep activations in HBM (the
 * attention projections of src/attn_qwen.c:160-165, :932-948). */
int ds4f_hip_mlx4_matvec_async(const uint32_t *vals, const uint16_t *scales,
                               const uint16_t *biases, int R, int C,
                               const float *x, float *y, void *stream);

/* ---- whole attention layers on the device (src/attn_qwen.c:87-225,
 * :837-968) --------------------------------------------------------------- *
 * One MLX 4-bit weight as the reference's mlx4_proj reads it from the trunk
 * (src/attn_qwen.c:59-70): the U32 nibble tensor, its BF16 scales and
 * optional BF16 biases, decoded shape rows x cols. */
typedef struct Ds4fGpuMlx4W {
    const uint32_t *vals;
    const uint16_t *scales, *biases;
    int rows, cols;
} Ds4fGpuMlx4W;

/* The weights of one attention layer (host pointers into the trunk; the
 * roles of Ds4fTrunkLayout the reference's steps read).  A GQA layer fills
 * in_norm, q, k, v, o, q_norm, k_norm (gqa_step :89-97); a linear layer
 * in_norm, qkv, z, a, b, out, conv_w, A_log, dt_bias, norm_w (linear_step
 * :840-849).  in_norm NULL means no input_layernorm (:158-159). */
typedef struct Ds4fGpuLayerW {
    const uint16_t *in_norm;
    Ds4fGpuMlx4W q, k, v, o;
    const uint16_t *q_norm, *k_norm;
    Ds4fGpuMlx4W qkv, z, a, b, out;
    const uint16_t *conv_w, *dt_bias, *norm_w;
    const float *A_log;
} Ds4fGpuLayerW;

/* Upload layer L's weights to the device, keyed by the layer id (the trunk
 * ring slot behind the pointers may be reused later, include/ds4f/ds4f.h:
 * 172-174).  The layer must be bound (ds4f_gpu_attn_bind) with its kind;
 * shapes are checked against the bound geometry and one hidden size for
 * every layer (the projections' cols).  A second call replaces the copy. */
int ds4f_gpu_attn_weights(int L, const Ds4fGpuLayerW *w);

/* One tensor of a layer's entry in the engine's packed trunk, laid out as
 * the engine's own Ds4fTrunkTensor (include/ds4f/moe.h:49-56) so the engine
 * passes its parsed list (tl->t + tl->t_off[L]) unchanged: checkpoint name,
 * dtype code (0 = F32, 4 = BF16, 5 = U32, as src/moe.c:36-42), dims, rank,
 * byte offset in the layer's payload (its bytes of trunk.bin), size. */
typedef struct Ds4fGpuTrunkTensor {
    char name[96];
    int  dtype;
    long dims[4];
    int  rank;
    long off;
    long nbytes;
} Ds4fGpuTrunkTensor;

/* Indices into a layer's tensor list of the roles the attention steps read
 * (-1: absent); an MLX projection is [weight, scales, biases]. */
typedef struct Ds4fGpuTrunkRoles {
    int in_norm;
    int q[3], k[3], v[3], o[3];
    int q_norm, k_norm;
    int conv, A_log, dt_bias;
    int qkv[3], z[3], a[3], b[3], out[3];
    int norm;
} Ds4fGpuTrunkRoles;

/* Resolve the roles of one layer's tensor list by the reference's name
 * suffixes, first match winning (ds4f_trunk_layout_load, src/moe.c:372-373,
 * :425-490).  Returns the layer's kind by the dispatch of
 * ds4f_attn_qwen_step (src/attn_qwen.c:1259-1263): DS4F_LAYER_GQA when a
 * q_proj weight is present, DS4F_LAYER_LINEAR when conv1d or in_proj_qkv is,
 * DS4F_LAYER_NONE otherwise; -1 on bad arguments.  Needs no GPU. */
int ds4f_gpu_trunk_roles(const Ds4fGpuTrunkTensor *t, int n, Ds4fGpuTrunkRoles *roles);

/* ds4f_gpu_attn_weights from the trunk: layer L's tensor list t[0..n) and
 * its payload tr (the layer's bytes of trunk.bin, as the engine streams
 * them, src/trunk.c).  MLX weights are U32 [rows, cols / 8] (decoded cols
 * dims[1] * 8, src/attn_qwen.c:103-105) with BF16 scales / biases; norms,
 * conv1d and dt_bias BF16; A_log F32.  The input norm is the tensor named
 * *.attn_norm.weight or *.input_layernorm.weight (src/moe.c:371-373).  A
 * list with no attention roles uploads nothing and returns 0.  A list that
 * lacks a role the layer's step requires (GQA: q/k/v/o_proj weights,
 * q_norm, k_norm; linear: in_proj_qkv/z/a/b and out_proj weights, conv1d,
 * norm, A_log, dt_bias) uploads nothing, returns 0 and marks the layer
 * incomplete: every later ds4f_gpu_attn_step / _chunk of it (and their
 * device-pointer forms) returns 0 with the states unchanged, as gqa_step
 * and linear_step skip such a layer (src/attn_qwen.c:96-97, :849-856).  A
 * dtype, rank or size other than these returns -1 with the reason in
 * ds4f_gpu_last_error. */
int ds4f_gpu_attn_weights_trunk(int L, const Ds4fGpuTrunkTensor *t, int n,
                                const uint8_t *tr);

/* One decode token of layer L on the residual stream, the whole of
 * ds4f_attn_qwen_step for that layer (src/attn_qwen.c:1255-1264 ->
 * gqa_step :87-225 or linear_step :837-968): xin = input_layernorm(state),
 * the MLX 4-bit projections of xin, the attention core, the output
 * projection, state += o.  state [hidden] is updated in place.  A layer of
 * kind NONE and a token outside [0, max_tokens) are silent skips (0). */
int ds4f_gpu_attn_step(int L, int token, float *state);
/* The same with state in device memory, enqueued on `stream` (NULL: the
 * plugin's stream); four launches (GQA: projections, split, merge, output)
 * or three (linear: projections, core, output), no allocation, so a
 * decode step can be captured in a HIP graph. */
int ds4f_hip_attn_step_async(int L, int token, float *state, void *stream);

/* A prefill chunk of B tokens t0 .. t0+B-1 of layer L on the residual
 * stream: the whole of ds4f_attn_gqa_chunk (src/attn_qwen.c:1145-1252) or
 * ds4f_attn_linear_chunk (:977-1135), as src/main.c:604-660 calls them per
 * layer: the tokens' input_layernorm, the batched MLX 4-bit projections
 * (ds4f_mlx4_matvec_batch, src/kernels.c:581-619, here one fp16-MFMA GEMM
 * launch for all of a layer's projections), the layer's prefill core, the
 * batched output projection and the residual adds.  states holds B
 * pointers to the tokens' hidden states [hidden], updated in place.  The
 * results are those of B ds4f_gpu_attn_step calls in token order, up to
 * float32 summation order. */
int ds4f_gpu_attn_chunk(int L, int t0, int B, float *const *states);
/* The same with the states in device memory, [B][hidden] contiguous,
 * enqueued on `stream`.  Allocates its workspaces on first use or growth
 * (not capturable then): the GEMM and delta-rule workspaces grow with B
 * (by at least half), the GQA one is reserved for the whole cache on the
 * first GQA chunk.  Growth frees the previous workspace, so a HIP graph
 * captured before it must be captured again -- a caller that captures
 * chunks first runs, outside the capture, one chunk of a GQA layer and
 * one of a delta-rule layer at its largest B; no later chunk of at most
 * that B (at any t0) allocates. */
int ds4f_hip_attn_chunk_async(int L, int t0, int B, float *states, void *stream);

/* The prefill paths compute with fp16 operands (the GQA prefill's q, k, v
 * and the chunk GEMM's X), which hold magnitudes below 65520; the
 * reference is fp32 throughout (src/attn_qwen.c:328-386, :1222-1231).
 * Their kernels set bits of a status word when a value is out of that
 * range: 1 = a GQA prefill operand, 2 = a chunk GEMM X operand.  The host
 * entries ds4f_gpu_gqa_prefill and ds4f_gpu_attn_chunk clear the word
 * before their launches, read it after, and recompute a flagged call on
 * the decode kernels (fp32 activations, bf16 cache) in token order, from
 * the state the call started from, so their results stay exact.  Callers
 * of the device-pointer prefills (ds4f_hip_gqa_prefill_async,
 * ds4f_hip_attn_chunk_async) read the word here: this synchronises
 * `stream` (NULL: the plugin's stream) and returns the bits set since the
 * last clear (0: every fp16 operand was in range; -1 on error); clear != 0
 * clears them.  The host entries keep bits that were already set when they
 * start (they clear and report only their own), so a device-pointer
 * caller's flag survives an intervening host-entry prefill.  A flagged
 * device-pointer call's outputs are not valid, and neither is what it
 * advanced in place: a GQA call's cache rows t0 .. t0+B-1, and a delta-rule
 * call's recurrent state and conv ring, which it updated from the
 * out-of-range operand.  A caller that wants to recompute such a call
 * snapshots the layer's state (ds4f_gpu_attn_sync to the host, or its own
 * device copy) before the call; the host entries do this themselves. */
int ds4f_hip_f16_status(void *stream, int clear);

/* Last error text of the plugin (static storage). */
const char *ds4f_gpu_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* DS4F_GPU_ATTN_H */
