/*
 * gqa_prefill.hip -- causal GQA prefill of B tokens on gfx950: fp16 MFMA
 * flash attention.
 *
 * Replaces the serial gqa_body loop of ds4f_attn_gqa_chunk
 * (src/attn_qwen.c:1222-1231): the results equal B decode steps in order.
 *
 * 1. prep:   one wave per new token: k_norm + half-split RoPE of the kv heads
 *            (src/attn_qwen.c:287-326), their bf16 cache rows and fp16
 *            copies in the MFMA-ready key workspace; vprep: v into the fp16
 *            workspace and the bf16 cache, transposed through LDS per
 *            32-key block.  q is normalised and rotated by the attention
 *            kernel as it loads its q block (below).
 * 2. prefix: cache rows of positions before t0 (earlier chunks) into the
 *            fp16 key / value workspaces; zero padding rows (only launched
 *            when there are such rows).
 * 3. attn:   grid = (pairs of 16-position q blocks, kv heads), 8 waves in
 *            two groups of 4.  A group serves the 8 q heads of its kv head
 *            for one q block (wave w: heads 2w, 2w+1 x 16 positions = 32
 *            columns); group A runs the long block's first key tiles,
 *            group B the short block and then the long block's remaining
 *            tiles, and hands its partial to group A through LDS at the
 *            end, so every workgroup (and each SIMD's two waves) carries
 *            the same causal work.  Per 32-key block:
 *              S^T[32 key][32 q] = K Q^T   (16 x v_mfma_f32_32x32x16_f16),
 *              online softmax per column (rescaled only when a column max
 *              grows by more than 8 in scaled units, which keeps P <= e^8
 *              in fp16),
 *              O^T[256][32 q] += V^T P^T  (16 x 32x32x16 f16; the S^T
 *              accumulator registers are P's B operand as they stand, the
 *              value tile is stored in the matching key order).
 *            Output O / l times sigmoid(gate), fp32.  K / V tiles go
 *            global -> LDS by direct-to-LDS buffer loads into two stages
 *            per group; the K workspace is granule-major and the V
 *            workspace row-swizzled, so each stage is a verbatim copy and
 *            the operand reads are bank-conflict free.
 * Operands are fp16 (11-bit mantissa): a single MFMA pass keeps the
 * outputs within the parity bar (max abs error ~1e-3 against the fp32
 * reference at T = 4096), where bf16 operands would not.
 */
#include "q35_device.h"
#include "q35_launch.h"

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;

namespace {

constexpr int D = Q35_GQA_D, G = Q35_GQA_GROUP, RD = Q35_ROPE_DIMS;
constexpr float SCALE = 0.0625f;                        /* 1/sqrt(256) */
constexpr float RESCALE_MARGIN = 8.0f;                  /* in scaled units */
constexpr float EXP_K = SCALE * 1.4426950408889634f;    /* exp(SCALE x) = 2^(EXP_K x) */

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

/* compile-time switch of the staging loads an MFMA phase issues */
template <bool ON>
struct DmaOn {
    static constexpr bool value = ON;
};

__device__ __forceinline__ uint16_t f16_bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}

/* slot of key r (0..31) of a block inside the value tile: within each
 * 16-key k-step the MFMA B operand of lane half h holds keys
 * {4h..4h+3, 8+4h..8+4h+3}, so slot order is 0-3, 8-11, 4-7, 12-15 */
__device__ __forceinline__ int v_slot(int r) {
    const int ks = r >> 4, r16 = r & 15;
    const int s16 = (r16 < 8) ? ((r16 >> 2) * 8 + (r16 & 3)) : (((r16 - 8) >> 2) * 8 + 4 + (r16 & 3));
    return ks * 16 + s16;
}

/* the inverse: key (0..31) held at slot s of a block */
__device__ __forceinline__ int v_key(int s) {
    const int ks = s >> 4, s16 = s & 15;
    const int r16 = ((s16 >> 3) << 2) + (s16 & 3) + ((s16 & 4) ? 8 : 0);
    return ks * 16 + r16;
}

/* fp16 key workspace: one 16 KB tile per 32 keys, granule-major (the
 * dims 8c..8c+7 of key r at granule 32c + r).  A tile goes to LDS as it
 * lies, and an MFMA operand read (32 keys x one granule) is 512
 * consecutive bytes. */
__device__ __forceinline__ size_t kw_index(int g, int kbt, int pos, int d) {
    return ((((size_t)g * kbt + (pos >> 5)) * 32 + (d >> 3)) * 32 + (pos & 31)) * 8 + (d & 7);
}

/* fp16 value workspace: one 16 KB tile per 32 keys, dim rows of 32 key
 * slots (4 granules); granule gr of row d is stored at gr ^ ((d >> 2) & 3),
 * so the operand reads of 16 consecutive rows hit 16 distinct bank groups. */
__device__ __forceinline__ size_t vw_index(int g, int kbt, int kb, int d, int slot) {
    return (((size_t)g * kbt + kb) * D + d) * 32 + (((slot >> 3) ^ ((d >> 2) & 3)) << 3) + (slot & 7);
}

/* k of the new tokens, one wave a token (4 a 256-thread block bx): q35's
 * k norm and RoPE -> k_post, the fp16 key workspace and the bf16 cache */
__device__ __forceinline__ void prep_rows(const Q35GqaPrefill &p, int bx) {
    const int b = 4 * bx + (threadIdx.x >> 6), pos = p.t0 + b;
    const int lane = threadIdx.x & 63, d0 = lane * 4;
    if (b >= p.B) return;                   /* wave-uniform; no barrier follows */
    const float *rope = p.rope + (size_t)pos * RD;
    float4 rc = make_float4(1.f, 1.f, 1.f, 1.f), rs = make_float4(0.f, 0.f, 0.f, 0.f);
    if (lane < RD / 4) {
        rc = *reinterpret_cast<const float4 *>(rope + (d0 & (RD / 2 - 1)));
        rs = *reinterpret_cast<const float4 *>(rope + RD / 2 + (d0 & (RD / 2 - 1)));
    }
    const uint2 wk = *reinterpret_cast<const uint2 *>(p.kn_w + d0);
    float4 xk[2];
#pragma unroll
    for (int g = 0; g < 2; g++)
        xk[g] = *reinterpret_cast<const float4 *>(p.k_in + ((size_t)b * p.kv_heads + g) * D + d0);
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const float4 y = q35_norm_rope_head(xk[g], wk, rc, rs, lane);
        q35_f16_guard(p.status, Q35_STATUS_GQA_F16, q35_f16_over(y.x) || q35_f16_over(y.y) ||
                                                        q35_f16_over(y.z) || q35_f16_over(y.w));
        if (p.k_post)
            *reinterpret_cast<float4 *>(p.k_post + ((size_t)b * p.kv_heads + g) * D + d0) = y;
        uint16_t *dst = p.kw + kw_index(g, p.kbt, pos, d0);
        *reinterpret_cast<uint2 *>(dst) =
            make_uint2((uint32_t)f16_bits(y.x) | ((uint32_t)f16_bits(y.y) << 16),
                       (uint32_t)f16_bits(y.z) | ((uint32_t)f16_bits(y.w) << 16));
        /* the 4 dims are consecutive in the cache tile (one 8-byte store) */
        *reinterpret_cast<uint2 *>(p.kt + q35_k_index(g, pos, d0, p.t_tiles)) =
            make_uint2((uint32_t)q35_f2bf(y.x) | ((uint32_t)q35_f2bf(y.y) << 16),
                       (uint32_t)q35_f2bf(y.z) | ((uint32_t)q35_f2bf(y.w) << 16));
    }
}

/* v of the new tokens -> the fp16 value workspace and the bf16 cache,
 * both dim-major ([dim][keys]).  One workgroup per (32-key block, kv head)
 * transposes the block's rows through LDS; a lane then stores 8 keys of
 * one dim row as one 16-byte granule (workspace slots 8i..8i+7, cache
 * positions 8i..8i+7 of a 16-position tile).  Keys outside [t0, t0+B) are
 * left alone: earlier positions belong to the cache, later ones are
 * workspace padding; a granule holding such keys (the block at t0 or at
 * t0 + B when those are not multiples of 32) is stored key by key. */
__device__ __forceinline__ void vprep_block(const Q35GqaPrefill &p, int bx, int g) {
    const int kb = (p.t0 >> 5) + bx;
    const int t = threadIdx.x;
    __shared__ float sv[32][D + 1];
    /* rows: key r of the block is position 32kb + r.  All eight loads of a
     * thread go out before any is used, as range-checked buffer loads
     * (positions before t0 addressed at the view's end, rows past the batch
     * beyond it: both read zero); as guarded loads each waited for the one
     * before it, eight memory round trips in a row. */
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<float *>(p.v_in)), 0, p.B * p.kv_heads * D * 4, Q35_BUF_DW3);
    float4 vv[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int idx = u * 256 + t, r = idx >> 6, c4 = (idx & 63) * 4;
        const int b = 32 * kb + r - p.t0;
        const uint32_t off = b >= 0 ? (uint32_t)(((b * p.kv_heads + g) * D + c4) * 4)
                                    : (uint32_t)(p.B * p.kv_heads * D * 4);
        vv[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0));
    }
    bool over = false;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int idx = u * 256 + t, r = idx >> 6, c4 = (idx & 63) * 4;
        const float4 v = vv[u];
        over = over || q35_f16_over(v.x) || q35_f16_over(v.y) || q35_f16_over(v.z) || q35_f16_over(v.w);
        sv[r][c4] = v.x;
        sv[r][c4 + 1] = v.y;
        sv[r][c4 + 2] = v.z;
        sv[r][c4 + 3] = v.w;
    }
    q35_f16_guard(p.status, Q35_STATUS_GQA_F16, over);
    q35_lds_barrier();
    const bool whole = 32 * kb >= p.t0 && 32 * kb + 32 <= p.t0 + p.B;   /* block-uniform */
    /* workspace: lane (d, granule q of 4 a dim row), slots 8q..8q+7 */
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int idx = u * 256 + t, d = idx >> 2, q = idx & 3;
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; e++) h[e] = f16_bits(sv[v_key(8 * q + e)][d]);
        uint16_t *dst = p.vw + vw_index(g, p.kbt, kb, d, 8 * q);
        if (whole) {
            *reinterpret_cast<uint4 *>(dst) =
                make_uint4(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                           h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16));
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int pos = 32 * kb + v_key(8 * q + e);
                if (pos >= p.t0 && pos < p.t0 + p.B) dst[e] = h[e];
            }
        }
    }
    /* cache: lane (tile tt, d, half hf), positions 16tt + 8hf .. +7 */
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int idx = u * 256 + t, tt = idx >> 9, d = (idx >> 1) & (D - 1), hf = idx & 1;
        const int r0 = 16 * tt + 8 * hf;
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; e++) h[e] = q35_f2bf(sv[r0 + e][d]);
        uint16_t *dst = p.vt + q35_v_index(g, 32 * kb + r0, d, p.t_tiles);
        if (whole) {
            *reinterpret_cast<uint4 *>(dst) =
                make_uint4(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                           h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16));
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int pos = 32 * kb + r0 + e;
                if (pos >= p.t0 && pos < p.t0 + p.B) dst[e] = h[e];
            }
        }
    }
}

/* key / value workspace rows that the prep kernel does not write: positions
 * [0, t0) from the bf16 cache and padding positions [t0+B, 32*kbt) as
 * zeros.  Threads cover (kv head, row r of n_rows, dim); row r maps to
 * position r below t0, else to the padding. */
__device__ __forceinline__ void prefix_rows(const Q35GqaPrefill &p, int n_rows, int bx) {
    const int64_t i = (int64_t)bx * 256 + threadIdx.x;
    if (i >= (int64_t)p.kv_heads * n_rows * D) return;
    const int g = (int)(i / ((int64_t)n_rows * D));
    const int r = (int)((i / D) % n_rows), d = (int)(i % D);
    const int pos = r < p.t0 ? r : p.t0 + p.B + (r - p.t0);
    float kf = 0.0f, vf = 0.0f;
    if (pos < p.t0) {
        kf = q35_bf2f(p.kt[q35_k_index(g, pos, d, p.t_tiles)]);
        vf = q35_bf2f(p.vt[q35_v_index(g, pos, d, p.t_tiles)]);
        q35_f16_guard(p.status, Q35_STATUS_GQA_F16, q35_f16_over(kf) || q35_f16_over(vf));
    }
    p.kw[kw_index(g, p.kbt, pos, d)] = f16_bits(kf);
    p.vw[vw_index(g, p.kbt, pos >> 5, d, v_slot(pos & 31))] = f16_bits(vf);
}

/* the three set-up passes in one launch (they write disjoint workspace
 * and cache elements; as three launches the two dispatch gaps and the
 * smaller kernels' tails cost about as much as the work): blocks [0, nk)
 * prep_rows, the next nvb * kv_heads blocks vprep_block, the rest
 * prefix_rows.  Every branch is block-uniform, so vprep_block's barrier
 * sees all of its block's threads. */
__global__ __launch_bounds__(256) void prep_kernel(Q35GqaPrefill p, int nvb, int n_rows) {
    const int nk = (p.B + 3) / 4, nv = nvb * p.kv_heads, bx = (int)blockIdx.x;
    if (bx < nk)
        prep_rows(p, bx);
    else if (bx < nk + nv)
        vprep_block(p, (bx - nk) % nvb, (bx - nk) / nvb);
    else
        prefix_rows(p, n_rows, bx - nk - nv);
}

/* LDS: per group, two stages of one 32-key block, each the K tile (16 KB,
 * granule-major as in the workspace) followed by the V tile (16 KB, rows
 * swizzled as in the workspace).  A stage is a verbatim copy of the two
 * workspace tiles: 32 direct-to-LDS loads of 1 KB (lane l -> bytes 16l..
 * of the block), 8 per wave. */
constexpr int TILE_HALFS = 32 * D;                               /* one K or V tile */
constexpr int STAGE = 2 * TILE_HALFS;                            /* halfs a stage */
constexpr uint32_t TILE_BYTES = TILE_HALFS * 2;
static_assert(4 * STAGE * 2 == 8 * 16 * 64 * 4 * 4, "the merge area is the four stages");

/* Instruction order for 16 MFMAs fed by 16 LDS fragment reads: READS reads
 * ahead, then (READS MFMAs, READS reads) repeated, then the last MFMAs, so
 * a batch of reads is always in flight under the previous batch's MFMAs.
 * Left to itself the scheduler minimises registers and waits on each read. */
template <int READS>
__device__ __forceinline__ void sched_reads_ahead() {
    __builtin_amdgcn_sched_group_barrier(0x100, READS, 0);   /* DS reads */
#pragma unroll
    for (int i = 0; i < 16 / READS - 1; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, READS, 0);  /* MFMA */
        __builtin_amdgcn_sched_group_barrier(0x100, READS, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, READS, 0);
}

/* max of v over the two 32-lane halves (lanes l and l ^ 32), on the
 * cross-half swap of gfx950 instead of an LDS permute */
__device__ __forceinline__ float half_pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(fmaxf(v, __uint_as_float(r[0])), __uint_as_float(r[1]));
}

/* this wave's direct-to-LDS loads have landed */
__device__ __forceinline__ void wait_dma() { q35_wait_vm<0>(); }

/* q block qb's output rows of this wave: O / l times sigmoid(gate), fp32;
 * the sigmoid on the hardware exp / reciprocal (q35_sigmoid_fast) */
__device__ __forceinline__ void store_rows(const Q35GqaPrefill &p, int g, int qb, int hl, int col,
                                           int h, float l_run, const f32x16_t (&acc)[8]) {
    const int end = p.t0 + p.B, qpos = p.t0 + 16 * qb + (col & 15);
    const float L = l_run + __shfl_xor(l_run, 32);
    if (qpos >= end) return;
    const int b = qpos - p.t0, head = g * G + hl;
    const float *gate = p.q_gate + ((size_t)b * p.heads + head) * 2 * D + D;
    float *out = p.attn_out + ((size_t)b * p.heads + head) * D;
    const float inv = 1.0f / L;
    /* the gate values of two dim tiles are loaded before any of their
     * outputs is stored: gate and out may alias for the compiler, which
     * keeps a load behind every earlier store, so one load per store made
     * 32 dependent round trips to memory (6-8 us a call at 4096 tokens;
     * batches of one or four tiles measure slower, eight spill) */
#pragma unroll
    for (int d0 = 0; d0 < 8; d0 += 2) {
        float4 gv[2][4];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                gv[u][j] = *reinterpret_cast<const float4 *>(gate + 32 * (d0 + u) + 8 * j + 4 * h);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int dt = d0 + u;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float4 o;
                o.x = acc[dt][4 * j + 0] * inv * q35_sigmoid_fast(gv[u][j].x);
                o.y = acc[dt][4 * j + 1] * inv * q35_sigmoid_fast(gv[u][j].y);
                o.z = acc[dt][4 * j + 2] * inv * q35_sigmoid_fast(gv[u][j].z);
                o.w = acc[dt][4 * j + 3] * inv * q35_sigmoid_fast(gv[u][j].w);
                *reinterpret_cast<float4 *>(out + 32 * dt + 8 * j + 4 * h) = o;
            }
        }
    }
}

/* Q^T of q block qb as the B operand for the wave's 32 columns, all 16
 * k-steps, straight from the fp32 q rows: lane (col, h) holds dims
 * 16 ks + 8 h .. +7 of column col (head 2 wg + col / 16, position col % 16
 * of the block), so a head's 256 dims are split between lanes l and l ^ 32
 * and the half-split RoPE pairs (d, d + 32), d < 32, sit in k-steps ks and
 * ks + 2 of one lane.  q_norm as src/attn_qwen.c:287-300 (the square sum in
 * double, eps on the mean) and the RoPE as :302-326, in the operation order
 * of q35_norm_rope_head, except that x / r is x times 1 / r: the operand is
 * rounded to fp16 next (2^-11 relative), which hides the last-place
 * difference, and 128 IEEE divisions a lane would sit on the attention
 * kernel's critical path.  Two passes over the row (the sum, then the
 * normalised values), the second from L2.  Rows past the batch are
 * range-checked loads that read zero. */
__device__ __forceinline__ void load_q(const Q35GqaPrefill &p, int g, int qb, int hl, int col, int h,
                                       f16x8_t (&qop)[16]) {
#pragma clang fp contract(off)
    const int b = 16 * qb + (col & 15);
    const bool live = b < p.B;
    const int head = g * G + hl;
    /* a view of the block's (at most 16) rows; a dead row's offset lies
     * past it for every k-step */
    const int rows = min(16, p.B - 16 * qb);
    const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<float *>(p.q_gate + (size_t)16 * qb * p.heads * 2 * D)), 0,
        rows * p.heads * 2 * D * 4, Q35_BUF_DW3);
    const uint32_t off = live ? (uint32_t)(((col & 15) * p.heads + head) * 2 * D + 8 * h) * 4 : 0x80000000u;
    auto ld8 = [&](int ks, float (&x)[8]) {
        const u32x4_t a0 = __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(off + 64 * ks), 0, 0);
        const u32x4_t a1 = __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(off + 64 * ks + 16), 0, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[e] = __uint_as_float(a0[e]);
            x[4 + e] = __uint_as_float(a1[e]);
        }
    };
    double ss = 0.0;
#pragma unroll
    for (int ks = 0; ks < 16; ks++) {
        float x[8];
        ld8(ks, x);
#pragma unroll
        for (int e = 0; e < 8; e++) ss += (double)x[e] * x[e];
    }
    ss += __shfl_xor(ss, 32);
    const float r = sqrtf((float)(ss / (double)D) + 1e-6f), ri = 1.0f / r;
    const float *rope = p.rope + (size_t)(p.t0 + (live ? b : 0)) * RD;
    float y[2][8];                  /* dims of k-steps 0, 1 until their RoPE partners come */
    bool over = false;
#pragma unroll
    for (int ks = 0; ks < 16; ks++) {
        float x[8];
        ld8(ks, x);
        const uint2 w0 = *reinterpret_cast<const uint2 *>(p.qn_w + 16 * ks + 8 * h);
        const uint2 w1 = *reinterpret_cast<const uint2 *>(p.qn_w + 16 * ks + 8 * h + 4);
        const uint32_t wd[4] = {w0.x, w0.y, w1.x, w1.y};
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = x[e] * ri * q35_bf2f((uint16_t)(wd[e >> 1] >> (16 * (e & 1))));
        if (ks < 2) {
#pragma unroll
            for (int e = 0; e < 8; e++) y[ks][e] = v[e];
        } else if (ks < 4) {
            /* RoPE of the pairs (ks - 2, ks), rotary index 16 (ks - 2) + 8 h + e */
            const float *cs = rope + 16 * (ks - 2) + 8 * h;
            const float4 c0 = *reinterpret_cast<const float4 *>(cs);
            const float4 c1 = *reinterpret_cast<const float4 *>(cs + 4);
            const float4 s0 = *reinterpret_cast<const float4 *>(cs + RD / 2);
            const float4 s1 = *reinterpret_cast<const float4 *>(cs + RD / 2 + 4);
            const float cc[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float v0 = y[ks - 2][e], v1 = v[e];
                const float a0 = v0 * cc[e] - v1 * sn[e];      /* x0*c - x1*s */
                const float a1 = v0 * sn[e] + v1 * cc[e];      /* x0*s + x1*c */
                qop[ks - 2][e] = (_Float16)a0;
                qop[ks][e] = (_Float16)a1;
                over = over || q35_f16_over(a0) || q35_f16_over(a1);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                qop[ks][e] = (_Float16)v[e];
                over = over || q35_f16_over(v[e]);
            }
        }
    }
    q35_f16_guard(p.status, Q35_STATUS_GQA_F16, over);
}

/* Causal work per q block grows with its position.  Workgroup x serves a
 * long q block (nqb-1-x) and a short one (x) of one kv head with 8 waves in
 * two groups of 4 (one wave of each group per SIMD).  Wave w of a group owns
 * 32 query columns: heads 2w, 2w+1 of the kv head x the block's 16
 * positions.  With nL and nS the blocks' 32-key tile counts, group A runs
 * the long block's tiles [0, nA), nA = ceil((nL + nS) / 2); group B runs the
 * short block's nS tiles, stores its rows, then the long block's tiles
 * [nA, nL).  Both groups step through nA intervals between workgroup
 * barriers, so every workgroup carries the same causal work.  At the end
 * group B hands its partial (max, sum, O) of the long block to group A
 * through LDS, and group A merges and stores the long block's rows.
 * Per tile and wave:
 *   S^T[32 key][32 q] = K Q^T   (16 x v_mfma_f32_32x32x16_f16),
 *   online softmax per column (rescaled only when a column max grows by
 *   more than 8 in scaled units, which keeps P <= e^8 in fp16),
 *   O^T[256][32 q] += V^T P^T  (16 x 32x32x16 f16; the S^T accumulator
 *   registers are P's B operand as they stand, the value tile is stored in
 *   the matching key order).
 * The two waves of a SIMD run out of phase: in interval it group A does
 * QK, softmax and PV of its tile it, while group B does softmax and PV of
 * its tile it-1 and then QK of its tile it, so one wave's softmax (VALU)
 * runs under the other's MFMAs.
 * K / V tiles move global -> LDS by direct-to-LDS buffer loads into two
 * stages per group, issued one interval ahead of use: for group A the K
 * and V tiles of tile it+1; for group B the K tile of tile it+1 and the V
 * tile of tile it (which it reads in the next interval), so no stage part
 * is written in an interval in which its group reads it.  Group A issues
 * its loads among its QK MFMAs, group B among its PV MFMAs. */
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512))) void attn_kernel(Q35GqaPrefill p) {
    /* 1-D grid over (pair, kv head).  Workgroups go to the 8 XCDs in turn
     * (id mod 8); with the pair count a multiple of 4, XCDs 0-3 take kv
     * head 0 and XCDs 4-7 kv head 1, so each XCD's L2 holds one head's K /
     * V workspaces (4 MB at 4096 tokens) instead of both */
    const int np = (p.nqb + 1) / 2, L = blockIdx.x;
    int x, g;
    if (p.kv_heads == 2 && (np & 3) == 0) {
        g = (L & 7) >> 2;
        x = (L >> 3) * 4 + (L & 3);
    } else {
        g = L / np;
        x = L % np;
    }
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int grp = w >> 2, wg = w & 3;
    const int h = lane >> 5, col = lane & 31;
    const int hl = 2 * wg + (col >> 4);
    const int end = p.t0 + p.B;

    __shared__ __align__(16) _Float16 smem[4 * STAGE];   /* [group][stage] */
    __shared__ float sml[4][2][64];                      /* group B's m, l */

    const int qL = p.nqb - 1 - x, qS = x;
    const bool has_short = qS < qL;
    const int nL = (min(p.t0 + 16 * qL + 16, end) + 31) >> 5;
    const int nS = has_short ? (min(p.t0 + 16 * qS + 16, end) + 31) >> 5 : 0;
    const int nA = (nL + nS + 1) >> 1;          /* intervals, and group A's tiles */
    const int nB = nS + nL - nA;                /* group B's tiles, nB <= nA */
    /* group B's j-th tile and its q block */
    auto tile_b = [&](int j) { return j < nS ? j : nA + j - nS; };
    auto block_b = [&](int j) { return j < nS ? qS : qL; };

    /* direct-to-LDS staging: this wave copies 1 KB blocks wg + 4i of a
     * stage part (the K tile, then the V tile) */
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(p.kw + (size_t)g * p.kbt * TILE_HALFS)), 0,
        p.kbt * TILE_BYTES, Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(p.vw + (size_t)g * p.kbt * TILE_HALFS)), 0,
        p.kbt * TILE_BYTES, Q35_BUF_DW3);
    const uint32_t dma_lane = (uint32_t)lane * 16;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) _Float16 *)smem;
    auto stage_part = [&](int stage, int part, int tile) {
        const uint32_t base = lds0 + (uint32_t)((grp * 2 + stage) * STAGE + part * TILE_HALFS) * 2;
        const uint32_t so = (uint32_t)tile * TILE_BYTES;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int j = wg + 4 * i;
            q35_dma16(part ? vrs : krs, base + j * 1024, dma_lane, so + j * 1024);
        }
    };
    /* Two stage parts (tiles t0 and t1, both below nL) whose eight loads
     * are issued between the operand-read batches of an MFMA phase: a
     * load's issue waits while the CU's address unit is busy with other
     * waves' loads, and placed there that wait runs under the MFMAs
     * already issued instead of in front of them.  Load i of the pair is
     * 1 KB block wg + 4 (i & 3) of part (i < 4 ? 0 : 1). */
    struct Dma2 {
        uint32_t base[2], so[2];
        int part[2];
    };
    auto dma2 = [&](int stage0, int part0, int tile0, int stage1, int part1, int tile1) {
        Dma2 d;
        d.base[0] = lds0 + (uint32_t)((grp * 2 + stage0) * STAGE + part0 * TILE_HALFS) * 2;
        d.base[1] = lds0 + (uint32_t)((grp * 2 + stage1) * STAGE + part1 * TILE_HALFS) * 2;
        d.so[0] = (uint32_t)tile0 * TILE_BYTES;
        d.so[1] = (uint32_t)tile1 * TILE_BYTES;
        d.part[0] = part0;
        d.part[1] = part1;
        return d;
    };
    auto dma_issue = [&](const Dma2 &d, int i) {
        const int k = i >> 2, j = wg + 4 * (i & 3);
        q35_dma16(d.part[k] ? vrs : krs, d.base[k] + j * 1024, dma_lane, d.so[k] + j * 1024);
    };

    /* operand read addresses: K granule 2ks + h of key col at
     * (2ks + h) * 32 + col; V row 32dt + col, granule h + 2(u & 1) (swizzled) */
    const int kbase = (h * 32 + col) * 8;                             /* + 512 ks halfs */
    const int vsw = (col >> 2) & 3;
    const int vb0 = TILE_HALFS + col * 32 + ((h ^ vsw) << 3);         /* + 1024 dt halfs */
    const int vb1 = TILE_HALFS + col * 32 + (((h + 2) ^ vsw) << 3);

    f16x8_t qop[16];
    f32x16_t acc[8];
    float m_used, l_run;
    auto reset = [&]() {
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[dt][i] = 0.0f;
        m_used = -INFINITY;
        l_run = 0.0f;
    };

    /* S^T = K Q^T: lane holds column col, keys 32kb + 8j + 4h + i' */
    auto qk = [&](auto dma_on, const Dma2 &d, int stage, f32x16_t &s) {
        const _Float16 *sb = smem + (grp * 2 + stage) * STAGE;
#pragma unroll
        for (int i = 0; i < 16; i++) s[i] = 0.0f;
        f16x8_t ka[16];
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            ka[ks] = *reinterpret_cast<const f16x8_t *>(sb + kbase + 512 * ks);
            if constexpr (decltype(dma_on)::value) {
                if (ks == 7 || ks == 11 || ks == 15) {
                    dma_issue(d, 2 * (ks >> 2) - 2);
                    dma_issue(d, 2 * (ks >> 2) - 1);
                }
            }
        }
#pragma unroll
        for (int ks = 0; ks < 16; ks++) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks], qop[ks], s, 0, 0, 0);
        if constexpr (decltype(dma_on)::value) {
            dma_issue(d, 6);
            dma_issue(d, 7);
        }
        sched_reads_ahead<4>();
    };

    /* online softmax of tile kb of q block qb, then O^T += V^T P^T */
    auto softmax_pv = [&](auto dma_on, const Dma2 &d, int stage, f32x16_t &s, int kb, int qb) {
        /* element i is key 32kb + 8(i/4) + 4h + i%4: causal (key <= qpos) and
         * inside the batch (key < end) as one per-lane bound on the
         * compile-time offset 8(i/4) + i%4, applied only on a tile that
         * reaches past the block's first position or the batch end.  Scores
         * stay unscaled here; the 1/16 scale rides in the exponent's
         * multiplier. */
        const int q0 = p.t0 + 16 * qb;
        if (32 * kb + 32 > min(q0 + 1, end)) {
            const int lim = min(q0 + (col & 15) + 1, end) - 32 * kb - 4 * h;
#pragma unroll
            for (int i = 0; i < 16; i++) s[i] = (8 * (i >> 2) + (i & 3)) < lim ? s[i] : -INFINITY;
        }
        float mx = s[0];
#pragma unroll
        for (int i = 1; i < 16; i++) mx = fmaxf(mx, s[i]);
        mx = half_pair_max(mx);
        const bool need = mx > m_used + RESCALE_MARGIN / SCALE;
        /* A column whose keys so far were all masked keeps m_used = -inf
         * and weights 0 (group B's first tile of the long block can lie
         * wholly after the block's first positions when t0 is not a multiple
         * of 16): its factor is 1, not exp2(-inf - -inf), and its exponent
         * offset stays finite.  need implies a finite mx, so a first use
         * gives exp2(-inf) = 0. */
        if (__any(need)) {
            const float alpha = need ? exp2f_fast((m_used - mx) * EXP_K) : 1.0f;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                acc[dt] *= alpha;
                __builtin_amdgcn_sched_barrier(0);
            }
            m_used = need ? mx : m_used;
        }
        f16x8_t pb[2];
        const float mk = m_used == -INFINITY ? 0.0f : m_used * EXP_K;
#pragma unroll
        for (int i = 0; i < 16; i++) pb[i >> 3][i & 7] = (_Float16)exp2f_fast(fmaf(s[i], EXP_K, -mk));
        /* the row sum of the fp16 weights the PV product uses, two a step */
        float ps = 0.0f;
        const f16x2_t one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f16x2_t pr = {pb[i >> 2][2 * (i & 3)], pb[i >> 2][2 * (i & 3) + 1]};
            ps = __builtin_amdgcn_fdot2(pr, one2, ps, false);
        }
        l_run += ps;
        const _Float16 *sb = smem + (grp * 2 + stage) * STAGE;
        f16x8_t va[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            va[u] = *reinterpret_cast<const f16x8_t *>(sb + ((u & 1) ? vb1 : vb0) + 1024 * (u >> 1));
            if constexpr (decltype(dma_on)::value) {
                if (u == 7 || u == 11 || u == 15) {
                    dma_issue(d, 2 * (u >> 2) - 2);
                    dma_issue(d, 2 * (u >> 2) - 1);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < 16; u++)
            acc[u >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[u], pb[u & 1], acc[u >> 1], 0, 0, 0);
        if constexpr (decltype(dma_on)::value) {
            dma_issue(d, 6);
            dma_issue(d, 7);
        }
        sched_reads_ahead<2>();   /* PV: two reads ahead (four: +5 us a call at 4096 tokens) */
    };

    reset();
    f32x16_t s;
    const Dma2 dnone = dma2(0, 0, 0, 0, 0, 0);
    if (grp == 0) {
        load_q(p, g, qL, hl, col, h, qop);
        stage_part(0, 0, 0);
        stage_part(0, 1, 0);
        wait_dma();
        q35_lds_barrier();
        for (int it = 0; it < nA; it++) {
            /* the next tile's K and V, issued among this tile's QK MFMAs;
             * in the last interval the clamp reloads tile it into the
             * stage nobody reads again */
            const int tn = min(it + 1, nA - 1);
            qk(DmaOn<true>{}, dma2((it + 1) & 1, 0, tn, (it + 1) & 1, 1, tn), it & 1, s);
            softmax_pv(DmaOn<false>{}, dnone, it & 1, s, it, qL);
            wait_dma();
            q35_lds_barrier();
        }
    } else {
        if (nB > 0) {
            load_q(p, g, block_b(0), hl, col, h, qop);
            stage_part(0, 0, tile_b(0));
        }
        wait_dma();
        q35_lds_barrier();
        for (int it = 0; it < nA; it++) {
            /* (separate conditions: as an if / else-if chain the
             * compiler spills a kilobyte a lane) */
            if (it == 0 && nB > 0) stage_part(0, 1, tile_b(0));
            if (it == 0 && 1 < nB) stage_part(1, 0, tile_b(1));
            if (it >= 1 && it <= nB) {
                /* V of tile it and K of tile it + 1, issued among the PV
                 * MFMAs of tile it - 1; past the last tile the clamp
                 * reloads it into stage parts nobody reads again */
                const int tv = tile_b(min(it, nB - 1)), tk = tile_b(min(it + 1, nB - 1));
                softmax_pv(DmaOn<true>{}, dma2(it & 1, 1, tv, (it + 1) & 1, 0, tk), (it - 1) & 1, s,
                           tile_b(it - 1), block_b(it - 1));
                if (it == nS && it < nB) {
                    /* the short block is done: its rows out, the long
                     * block's tail next */
                    store_rows(p, g, qS, hl, col, h, l_run, acc);
                    reset();
                    load_q(p, g, qL, hl, col, h, qop);
                    /* all of this wave's loads done: the compiler then
                     * places no load-count waits for q on the common
                     * path, where they would also wait for staging loads */
                    wait_dma();
                }
            }
            if (it < nB) qk(DmaOn<false>{}, dnone, it & 1, s);
            wait_dma();
            q35_lds_barrier();
        }
        /* after the last barrier the stages become the merge area: no
         * staging loads here */
        if (nB == nA && nB > 0)
            softmax_pv(DmaOn<false>{}, dnone, (nB - 1) & 1, s, tile_b(nB - 1), block_b(nB - 1));
    }

    /* group B's partial of the long block -> LDS -> group A; the stages are
     * idle after the last barrier.  When group B has no long tiles
     * (nB = nS), its rows are the short block's, and it hands over an
     * empty partial. */
    q35_lds_barrier();
    float *mrg = reinterpret_cast<float *>(smem) + wg * 128 * 64 + lane;
    if (grp == 1) {
        if (nS > 0 && nB == nS) {
            store_rows(p, g, qS, hl, col, h, l_run, acc);
            m_used = -INFINITY;
        }
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int i = 0; i < 16; i++) mrg[(16 * dt + i) * 64] = acc[dt][i];
        sml[wg][0][lane] = m_used;
        sml[wg][1][lane] = l_run;
    }
    q35_lds_barrier();
    if (grp == 0) {
        const float mB = sml[wg][0][lane], lB = sml[wg][1][lane];
        const float M = fmaxf(m_used, mB);
        const float fa = exp2f_fast((m_used - M) * EXP_K);
        const float fb = mB == -INFINITY ? 0.0f : exp2f_fast((mB - M) * EXP_K);
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[dt][i] = acc[dt][i] * fa + mrg[(16 * dt + i) * 64] * fb;
        store_rows(p, g, qL, hl, col, h, l_run * fa + lB * fb, acc);
    }
}

}  // namespace

extern "C" void q35_gqa_prefill_ws_bytes(int t0, int B, int kv_heads, size_t *kw, size_t *vw) {
    const size_t kbt = (size_t)(t0 + B + 31) / 32;
    *kw = (size_t)kv_heads * kbt * 32 * D * 2;
    *vw = *kw;
}

extern "C" hipError_t q35_gqa_prefill(const Q35GqaPrefill *pin, hipStream_t stream) {
    Q35GqaPrefill p = *pin;
    if (p.heads != p.kv_heads * G || p.kv_heads != 2 || p.B < 1 || p.t0 < 0) return hipErrorInvalidValue;
    p.nqb = (p.B + 15) / 16;
    p.kbt = (p.t0 + p.B + 31) / 32;
    /* value blocks of the new keys, and rows prep_rows / vprep_block leave:
     * the prefix and the key padding */
    const int nvb = ((p.t0 + p.B - 1) >> 5) - (p.t0 >> 5) + 1;
    const int n_rows = p.t0 + (p.kbt * 32 - (p.t0 + p.B));
    const int64_t nblk = (p.B + 3) / 4 + (int64_t)nvb * p.kv_heads +
                         ((int64_t)p.kv_heads * n_rows * D + 255) / 256;
    if (nblk > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(prep_kernel, dim3((unsigned)nblk), dim3(256), 0, stream, p, nvb, n_rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_kernel, dim3((p.nqb + 1) / 2 * p.kv_heads), dim3(512), 0, stream, p);
    return hipGetLastError();
}
