/*
 * gqa_prefill.hip -- causal GQA prefill of B tokens on gfx950: fp16 MFMA
 * flash attention.
 *
 * Replaces the serial gqa_body loop of ds4f_attn_gqa_chunk
 * (src/attn_qwen.c:1222-1231): the results equal B decode steps in order.
 *
 * 1. prep:   one workgroup per new token: q_norm / k_norm + half-split RoPE
 *            (src/attn_qwen.c:287-326), the bf16 cache rows of k, and fp16
 *            copies of q and k in MFMA-ready workspaces; vprep: v into the
 *            fp16 workspace and the bf16 cache, transposed through LDS per
 *            32-key block.
 * 2. prefix: cache rows of positions before t0 (earlier chunks) into the
 *            fp16 key / value workspaces; zero padding rows (only launched
 *            when there are such rows).
 * 3. attn:   grid = (pairs of 16-position q blocks, kv heads), 4 waves.  A
 *            workgroup serves the 8 q heads of its kv head (wave w: heads
 *            2w, 2w+1 x 16 positions = 32 columns), so every K / V tile
 *            staged in LDS feeds 128 query rows.  Per 32-key block:
 *              S^T[32 key][32 q] = K Q^T   (16 x v_mfma_f32_32x32x16_f16),
 *              online softmax per column (rescaled only when a column max
 *              grows by more than 8 in scaled units, which keeps P <= e^8
 *              in fp16),
 *              O^T[256][32 q] += V^T P^T  (16 x 32x32x16 f16; the S^T
 *              accumulator registers are P's B operand as they stand, the
 *              value tile is stored in the matching key order).
 *            Output O / l times sigmoid(gate), fp32.  K / V tiles move
 *            global -> registers (buffer loads, one tile ahead) -> padded
 *            LDS (two stages); each workgroup runs a long and a short q
 *            block so every workgroup carries the same causal work.
 * Operands are fp16 (11-bit mantissa): a single MFMA pass keeps the
 * outputs within the parity bar (max abs error ~1e-3 against the fp32
 * reference at T = 4096), where bf16 operands would not.
 */
#include "q35_device.h"
#include "q35_launch.h"

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4_t;

namespace {

constexpr int D = Q35_GQA_D, G = Q35_GQA_GROUP, RD = Q35_ROPE_DIMS;
constexpr float SCALE = 0.0625f;                        /* 1/sqrt(256) */
constexpr float RESCALE_MARGIN = 8.0f;                  /* in scaled units */
constexpr float EXP_K = SCALE * 1.4426950408889634f;    /* exp(SCALE x) = 2^(EXP_K x) */

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

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

__global__ __launch_bounds__(256) void prep_kernel(Q35GqaPrefill p) {
    const int b = blockIdx.x, pos = p.t0 + b;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, d0 = lane * 4;
    const float *rope = p.rope + (size_t)pos * RD;

    float4 xq[4];
#pragma unroll
    for (int hh = 0; hh < 4; hh++)
        xq[hh] = *reinterpret_cast<const float4 *>(p.q_gate + ((size_t)b * p.heads + 4 * w + hh) * 2 * D + d0);
    const uint2 wq = *reinterpret_cast<const uint2 *>(p.qn_w + d0);
    float4 rc = make_float4(1.f, 1.f, 1.f, 1.f), rs = make_float4(0.f, 0.f, 0.f, 0.f);
    if (lane < RD / 4) {
        rc = *reinterpret_cast<const float4 *>(rope + (d0 & (RD / 2 - 1)));
        rs = *reinterpret_cast<const float4 *>(rope + RD / 2 + (d0 & (RD / 2 - 1)));
    }
    float4 xk[2];
    uint2 wk = make_uint2(0, 0);
    if (w == 0) {
        wk = *reinterpret_cast<const uint2 *>(p.kn_w + d0);
#pragma unroll
        for (int g = 0; g < 2; g++)
            xk[g] = *reinterpret_cast<const float4 *>(p.k_in + ((size_t)b * p.kv_heads + g) * D + d0);
    }

    const int qb = b >> 4, qp = b & 15;
#pragma unroll
    for (int hh = 0; hh < 4; hh++) {
        const int head = 4 * w + hh, g = head / G, hl = head % G;
        const float4 y = q35_norm_rope_head(xq[hh], wq, rc, rs, lane);
        uint16_t *dst = p.qw + ((((size_t)g * p.nqb + qb) * G + hl) * 16 + qp) * D + d0;
        const uint2 pk = make_uint2((uint32_t)f16_bits(y.x) | ((uint32_t)f16_bits(y.y) << 16),
                                    (uint32_t)f16_bits(y.z) | ((uint32_t)f16_bits(y.w) << 16));
        *reinterpret_cast<uint2 *>(dst) = pk;
    }
    const int kb = pos >> 5, kr = pos & 31;
    if (w == 0) {
#pragma unroll
        for (int g = 0; g < 2; g++) {
            const float4 y = q35_norm_rope_head(xk[g], wk, rc, rs, lane);
            if (p.k_post)
                *reinterpret_cast<float4 *>(p.k_post + ((size_t)b * p.kv_heads + g) * D + d0) = y;
            uint16_t *dst = p.kw + (((size_t)g * p.kbt + kb) * 32 + kr) * D + d0;
            *reinterpret_cast<uint2 *>(dst) =
                make_uint2((uint32_t)f16_bits(y.x) | ((uint32_t)f16_bits(y.y) << 16),
                           (uint32_t)f16_bits(y.z) | ((uint32_t)f16_bits(y.w) << 16));
            const float yy[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
            for (int e = 0; e < 4; e++) p.kt[q35_k_index(g, pos, d0 + e, p.t_tiles)] = q35_f2bf(yy[e]);
        }
    }
}

/* v of the new tokens -> the fp16 value workspace and the bf16 cache,
 * both dim-major ([dim][keys]).  One workgroup per (32-key block, kv head)
 * transposes the block's rows through LDS, so consecutive lanes write
 * consecutive keys of one dim row (64 B of workspace, 32 B of cache) rather
 * than one 2-byte value per row.  Keys outside [t0, t0+B) are left alone:
 * earlier positions belong to the cache, later ones are workspace padding. */
__global__ __launch_bounds__(256) void vprep_kernel(Q35GqaPrefill p) {
    const int kb = (p.t0 >> 5) + (int)blockIdx.x, g = blockIdx.y;
    const int t = threadIdx.x;
    __shared__ float sv[32][D + 1];
    /* rows: key r of the block is position 32kb + r */
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int idx = u * 256 + t, r = idx >> 6, c4 = (idx & 63) * 4;
        const int pos = 32 * kb + r;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (pos >= p.t0 && pos < p.t0 + p.B)
            v = *reinterpret_cast<const float4 *>(p.v_in + ((size_t)(pos - p.t0) * p.kv_heads + g) * D + c4);
        sv[r][c4] = v.x;
        sv[r][c4 + 1] = v.y;
        sv[r][c4 + 2] = v.z;
        sv[r][c4 + 3] = v.w;
    }
    q35_lds_barrier();
    /* workspace: lane (d, slot) of 32 slots a dim row, key = the slot's key */
#pragma unroll
    for (int u = 0; u < 32; u++) {
        const int idx = u * 256 + t, d = idx >> 5, slot = idx & 31;
        const int r = v_key(slot), pos = 32 * kb + r;
        if (pos >= p.t0 && pos < p.t0 + p.B)
            p.vw[(((size_t)g * p.kbt + kb) * D + d) * 32 + slot] = f16_bits(sv[r][d]);
    }
    /* cache: two 16-token tiles, lane (tile, d, token) */
#pragma unroll
    for (int u = 0; u < 32; u++) {
        const int idx = u * 256 + t, tt = idx >> 12, d = (idx >> 4) & (D - 1), r16 = idx & 15;
        const int r = tt * 16 + r16, pos = 32 * kb + r;
        if (pos >= p.t0 && pos < p.t0 + p.B)
            p.vt[q35_v_index(g, pos, d, p.t_tiles)] = q35_f2bf(sv[r][d]);
    }
}

/* key / value workspace rows that the prep kernel does not write: positions
 * [0, t0) from the bf16 cache and padding positions [t0+B, 32*kbt) as
 * zeros.  Threads cover (kv head, row r of n_rows, dim); row r maps to
 * position r below t0, else to the padding. */
__global__ void prefix_kernel(Q35GqaPrefill p, int n_rows) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)p.kv_heads * n_rows * D) return;
    const int g = (int)(i / ((int64_t)n_rows * D));
    const int r = (int)((i / D) % n_rows), d = (int)(i % D);
    const int pos = r < p.t0 ? r : p.t0 + p.B + (r - p.t0);
    float kf = 0.0f, vf = 0.0f;
    if (pos < p.t0) {
        kf = q35_bf2f(p.kt[q35_k_index(g, pos, d, p.t_tiles)]);
        vf = q35_bf2f(p.vt[q35_v_index(g, pos, d, p.t_tiles)]);
    }
    const int kb = pos >> 5, kr = pos & 31;
    p.kw[(((size_t)g * p.kbt + kb) * 32 + kr) * D + d] = f16_bits(kf);
    p.vw[(((size_t)g * p.kbt + kb) * D + d) * 32 + v_slot(kr)] = f16_bits(vf);
}

/* q workspace rows [B, 16*nqb) of the last block: zeros */
__global__ void qpad_kernel(Q35GqaPrefill p, int n_pad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)p.kv_heads * G * n_pad * D) return;
    const int d = (int)(i % D);
    const int64_t row = i / D;
    const int qpos = p.B + (int)(row % n_pad);
    const int hl = (int)((row / n_pad) % G), g = (int)(row / ((int64_t)n_pad * G));
    p.qw[((((size_t)g * p.nqb + (qpos >> 4)) * G + hl) * 16 + (qpos & 15)) * D + d] = 0;
}



/* LDS tiles of one 32-key block.  Rows are padded by one 16-byte granule
 * so the MFMA operand reads are conflict-free and take one address
 * register plus immediate offsets:
 *   K tile: 32 key rows x 33 granules (528 B; granule 32 unused),
 *   V tile: 256 dim rows x 5 granules (80 B; granule 4 unused). */
constexpr int KROW = 33, VROW = 5;
constexpr int KTILE = 32 * KROW * 8, VTILE = D * VROW * 8;      /* halfs */

/* Instruction order for a block of 16 MFMAs fed by 16 LDS fragment reads:
 * 8 reads, then (4 MFMAs, 4 reads) x 3, then 4 MFMAs, so a batch of reads
 * is always in flight under the previous batch's MFMAs.  Left to itself
 * the scheduler minimises registers and waits on each read. */
__device__ __forceinline__ void sched_reads_ahead() {
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);    /* DS reads */
#pragma unroll
    for (int i = 0; i < 3; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  /* MFMA */
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
}

/* max of v over the two 32-lane halves (lanes l and l ^ 32), on the
 * cross-half swap of gfx950 instead of an LDS permute */
__device__ __forceinline__ float half_pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(fmaxf(v, __uint_as_float(r[0])), __uint_as_float(r[1]));
}

/* Causal work per q block grows with its position, so workgroup x runs
 * the pair of q blocks (nqb-1-x, x): the longest with the shortest, equal
 * total work for every workgroup whatever CU it lands on. */
__global__ __launch_bounds__(256, 1) void attn_kernel(Q35GqaPrefill p) {
    const int g = blockIdx.y;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int h = lane >> 5, col = lane & 31;
    const int hl = 2 * w + (col >> 4);
    const int end = p.t0 + p.B;

    __shared__ __align__(16) _Float16 sK[2][KTILE];
    __shared__ __align__(16) _Float16 sV[2][VTILE];

    /* staging: thread t moves granules t + 256 j (j < 4) of the K tile
     * (row (t + 256 j) / 32) and of the V tile (row (t + 256 j) / 4) through
     * registers.  Buffer loads on a range-checked resource per kv head: the
     * tile offset is the scalar offset, the lane's offset a loop-invariant
     * VGPR. */
    const uint32_t tile_bytes = 32 * D * 2;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(p.kw + (size_t)g * p.kbt * 32 * D), 0, p.kbt * tile_bytes, Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(p.vw + (size_t)g * p.kbt * D * 32), 0, p.kbt * tile_bytes, Q35_BUF_DW3);
    uint32_t kgo[4], vgo[4];
    int klo[4], vlo[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int gi = t + 256 * j;
        kgo[j] = (uint32_t)gi * 16u;                 /* K tile: 32 granules a row */
        vgo[j] = (uint32_t)gi * 16u;                 /* V tile: 4 granules a row */
        klo[j] = ((gi >> 5) * KROW + (gi & 31)) * 8;
        vlo[j] = ((gi >> 2) * VROW + (gi & 3)) * 8;
    }
    const int kbase = (col * KROW + h) * 8;          /* + 16 ks halfs */
    const int vbase = (col * VROW + h) * 8;          /* + dt * 32 rows + 16 ks halfs */

  for (int item = 0; item < 2; item++) {
    const int qb = item == 0 ? p.nqb - 1 - (int)blockIdx.x : (int)blockIdx.x;
    if (item == 1 && qb >= p.nqb - 1 - (int)blockIdx.x) break;   /* odd middle block */
    const int q0 = p.t0 + 16 * qb;
    const int qpos = q0 + (col & 15);
    const int n_keys = min(q0 + 16, end);
    const int nkb = (n_keys + 31) >> 5;

    /* Q^T as the B operand for the wave's 32 columns, all 16 k-steps */
    const uint16_t *qrow = p.qw + ((((size_t)g * p.nqb + qb) * G + hl) * 16 + (col & 15)) * D;
    f16x8_t qop[16];
#pragma unroll
    for (int ks = 0; ks < 16; ks++)
        qop[ks] = *reinterpret_cast<const f16x8_t *>(qrow + 16 * ks + 8 * h);

    f32x16_t acc[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[dt][i] = 0.0f;
    float m_used = -INFINITY, l_run = 0.0f;

    /* tile 0 into stage 0, tile 1 into the staging registers; every load is
     * unconditional (a tile index past the end is clamped and its copy is
     * never read), so the compiler waits on exactly the loads it needs */
    u32x4_t stg[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        stg[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, kgo[j], 0, 0);
        stg[4 + j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, vgo[j], 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        *reinterpret_cast<u32x4_t *>(&sK[0][klo[j]]) = stg[j];
        *reinterpret_cast<u32x4_t *>(&sV[0][vlo[j]]) = stg[4 + j];
    }
    {
        const uint32_t so = (uint32_t)min(1, nkb - 1) * tile_bytes;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            stg[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, kgo[j], so, 0);
            stg[4 + j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, vgo[j], so, 0);
        }
    }
    q35_lds_barrier();

    for (int kb = 0; kb < nkb; kb++) {
        const int buf = kb & 1;
        /* S^T = K Q^T: lane holds column col, keys 32kb + 8j + 4h + i' */
        f32x16_t s;
#pragma unroll
        for (int i = 0; i < 16; i++) s[i] = 0.0f;
        {
            const _Float16 *kp = &sK[buf][kbase];
            f16x8_t ka[2][4];
#pragma unroll
            for (int u = 0; u < 4; u++) ka[0][u] = *reinterpret_cast<const f16x8_t *>(kp + 16 * u);
#pragma unroll
            for (int bq = 0; bq < 4; bq++) {
                if (bq < 3) {
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        ka[(bq + 1) & 1][u] =
                            *reinterpret_cast<const f16x8_t *>(kp + 16 * (4 * (bq + 1) + u));
                }
#pragma unroll
                for (int u = 0; u < 4; u++)
                    s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[bq & 1][u], qop[4 * bq + u], s, 0, 0, 0);
            }
            sched_reads_ahead();
        }
        /* element i is key 32kb + 8(i/4) + 4h + i%4: causal (key <= qpos) and
         * inside the batch (key < end) as one per-lane bound on the
         * compile-time offset 8(i/4) + i%4.  Scores stay unscaled here; the
         * 1/16 scale rides in the exponent's multiplier. */
        const int lim = min(qpos + 1, end) - 32 * kb - 4 * h;
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float v = (8 * (i >> 2) + (i & 3)) < lim ? s[i] : -INFINITY;
            s[i] = v;
            mx = fmaxf(mx, v);
        }
        mx = half_pair_max(mx);
        const bool need = mx > m_used + RESCALE_MARGIN / SCALE;
        if (__any(need)) {
            const float m_new = need ? mx : m_used;
            const float alpha = exp2f_fast((m_used - m_new) * EXP_K);   /* -inf -> 0 on first use */
            l_run *= alpha;
            /* one 16-register tile at a time: the accumulators live in
             * AGPRs and this rare path must not hold all 128 in VGPRs */
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                acc[dt] *= alpha;
                __builtin_amdgcn_sched_barrier(0);
            }
            m_used = m_new;
        }
        f16x8_t pb[2];
        float ps = 0.0f;
        const float mk = m_used * EXP_K;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float pv = exp2f_fast(fmaf(s[i], EXP_K, -mk));
            ps += pv;
            pb[i >> 3][i & 7] = (_Float16)pv;
        }
        l_run += ps;
        /* O^T += V^T P^T, V fragments in batches of 4 (two dim tiles) */
        {
            const _Float16 *vp = &sV[buf][vbase];
            f16x8_t va[2][4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                va[0][u] = *reinterpret_cast<const f16x8_t *>(vp + (u >> 1) * 32 * VROW * 8 + 16 * (u & 1));
#pragma unroll
            for (int bq = 0; bq < 4; bq++) {
                if (bq < 3) {
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int dt = 2 * (bq + 1) + (u >> 1);
                        va[(bq + 1) & 1][u] =
                            *reinterpret_cast<const f16x8_t *>(vp + dt * 32 * VROW * 8 + 16 * (u & 1));
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int dt = 2 * bq + (u >> 1);
                    acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[bq & 1][u], pb[u & 1], acc[dt],
                                                                     0, 0, 0);
                }
            }
            sched_reads_ahead();
        }
        /* staged tile kb+1 into the other stage (every wave finished tile
         * kb-1, its previous occupant, before the last barrier), then the
         * loads of tile kb+2 */
#pragma unroll
        for (int j = 0; j < 4; j++) {
            *reinterpret_cast<u32x4_t *>(&sK[buf ^ 1][klo[j]]) = stg[j];
            *reinterpret_cast<u32x4_t *>(&sV[buf ^ 1][vlo[j]]) = stg[4 + j];
        }
        {
            const uint32_t so = (uint32_t)min(kb + 2, nkb - 1) * tile_bytes;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                stg[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, kgo[j], so, 0);
                stg[4 + j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, vgo[j], so, 0);
            }
        }
        q35_lds_barrier();
    }

    const float L = l_run + __shfl_xor(l_run, 32);
    if (qpos < end) {
        const int b = qpos - p.t0, head = g * G + hl;
        const float *gate = p.q_gate + ((size_t)b * p.heads + head) * 2 * D + D;
        float *out = p.attn_out + ((size_t)b * p.heads + head) * D;
        const float inv = 1.0f / L;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = 32 * dt + 8 * j + 4 * h;
                const float4 gv = *reinterpret_cast<const float4 *>(gate + d);
                float4 o;
                o.x = acc[dt][4 * j + 0] * inv * q35_sigmoid(gv.x);
                o.y = acc[dt][4 * j + 1] * inv * q35_sigmoid(gv.y);
                o.z = acc[dt][4 * j + 2] * inv * q35_sigmoid(gv.z);
                o.w = acc[dt][4 * j + 3] * inv * q35_sigmoid(gv.w);
                *reinterpret_cast<float4 *>(out + d) = o;
            }
        }
    }
  }
}

}  // namespace

extern "C" void q35_gqa_prefill_ws_bytes(int t0, int B, int kv_heads, size_t *qw, size_t *kw,
                                         size_t *vw) {
    const size_t nqb = (size_t)(B + 15) / 16, kbt = (size_t)(t0 + B + 31) / 32;
    *qw = (size_t)kv_heads * nqb * G * 16 * D * 2;
    *kw = (size_t)kv_heads * kbt * 32 * D * 2;
    *vw = *kw;
}

extern "C" hipError_t q35_gqa_prefill(const Q35GqaPrefill *pin, hipStream_t stream) {
    Q35GqaPrefill p = *pin;
    if (p.heads != p.kv_heads * G || p.kv_heads != 2 || p.B < 1 || p.t0 < 0) return hipErrorInvalidValue;
    p.nqb = (p.B + 15) / 16;
    p.kbt = (p.t0 + p.B + 31) / 32;
    hipLaunchKernelGGL(prep_kernel, dim3(p.B), dim3(256), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        const int nvb = ((p.t0 + p.B - 1) >> 5) - (p.t0 >> 5) + 1;
        hipLaunchKernelGGL(vprep_kernel, dim3(nvb, p.kv_heads), dim3(256), 0, stream, p);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const int n_rows = p.t0 + (p.kbt * 32 - (p.t0 + p.B));    /* prefix + key padding */
    if (n_rows > 0) {
        const int64_t n = (int64_t)p.kv_heads * n_rows * D;
        hipLaunchKernelGGL(prefix_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p,
                           n_rows);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const int n_pad = p.nqb * 16 - p.B;
    if (n_pad > 0) {
        const int64_t n = (int64_t)p.kv_heads * G * n_pad * D;
        hipLaunchKernelGGL(qpad_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p,
                           n_pad);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(attn_kernel, dim3((p.nqb + 1) / 2, p.kv_heads), dim3(256), 0, stream, p);
    return hipGetLastError();
}
