/*
 * lin_prefill.hip -- prefill of B tokens of a gated delta-rule layer on
 * gfx950, in chunked (WY / UT) form.
 *
 * Replaces the serial lin_body loop of ds4f_attn_linear_chunk
 * (src/attn_qwen.c:1088-1109): the results equal B decode steps in order
 * up to fp32 rounding.
 *
 * Per token t (state S [kd i][vd j], key head of value head h is h/2):
 *   S <- exp(g_t) S;  delta_t = beta_t (v_t - S^T k_t);  S <- S + k_t delta_t^T;
 *   o_t = S^T q_t                                   (src/attn_qwen.c:666-690)
 * Over a chunk of C = 64 tokens with G_t = sum_{s<=t} g_s (from the chunk
 * start) and S0 the state entering the chunk, this unrolls exactly to
 *   A      = strict_lower( beta_t exp(G_t - G_s) k_t.k_s )
 *   W      = (I + A)^-1 diag(beta exp(G)) K       [C][kd]
 *   U      = (I + A)^-1 diag(beta) V              [C][vd]
 *   Delta  = U - W S0                             (the chunk's delta_t rows)
 *   O      = diag(exp(G)) Q S0 + Pm Delta,  Pm = lower( exp(G_t - G_s) q_t.k_s )
 *   S_end  = exp(G_C) S0 + Kd^T Delta,      Kd[s] = exp(G_C - G_s) k_s
 * Every factor exp(G_t - G_s) has s <= t, so none exceeds 1.
 *
 * Kernels, in stream order:
 *   conv_kernel  per token: conv1d + SiLU (ring taps for positions before
 *                t0), q/k RMS-normalisation, gates -> post [B][rows] (the
 *                reference's mutated qkv) and gates [B][VH][2]
 *   ring_kernel  the last min(B, 4) raw rows into the conv ring
 *   chunk_kernel per (chunk, value head), all in parallel: K K^T and Q K^T
 *                on fp32 MFMA, A and Pm, the forward substitution that
 *                gives W and U, Kd^T and the decay vectors
 *   scan_kernel  per (value head, 16-column block of vd), sequential over
 *                chunks: the state block stays in LDS; Delta, O and S_end
 *                on fp32 MFMA (v_mfma_f32_16x16x4_f32); O unnormalised
 *                into out
 *   gnorm_kernel per (token, value head): RMSNormGated of out with z
 *                (src/attn_qwen.c:726-749)
 * All arithmetic is fp32 (MFMA fp32 products are exact, accumulation fp32),
 * the chunk-local cumulative log-decay is summed in double.
 */
#include "q35_device.h"
#include "q35_launch.h"

namespace {

constexpr int KD = 128, VD = 128, C = 64;
constexpr int XS = KD + 4;     /* LDS row stride (floats) of K / Q tiles: conflict-free b128 */
constexpr int AS = C + 4;      /* LDS row stride of A and of the Delta tile */

__device__ __forceinline__ f32x4_t mfma4(float a, float b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float el(const float4 &v, int e) {
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

/* ---- 1. conv + SiLU, q/k norms, gates ------------------------------------ *
 * grid (rows / 512, ceil(B / 8)), 4 waves; wave w owns 128-channel group
 * 4*blockIdx.x + w (q heads, then k heads, then v heads), 2 channels a
 * lane, for 8 consecutive tokens: the 11 raw rows they tap are loaded once
 * (a sliding window instead of 4 loads per output). */
constexpr int CT = 8;
__global__ __launch_bounds__(256) void conv_kernel(Q35LinPrefill p) {
    const int bb = blockIdx.y * CT;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int KH = p.k_heads, VH = p.v_heads;
    const int rows = 2 * KH * KD + VH * VD;
    const int grp = 4 * blockIdx.x + w;
    const int c0 = grp * 128 + 2 * lane;

    /* raw rows of positions t0+bb-3 .. t0+bb+CT-1 */
    float2 xr[CT + 3];
#pragma unroll
    for (int k = 0; k < CT + 3; k++) {
        const int b = bb - 3 + k, pp = p.t0 + b;
        float2 v = make_float2(0.f, 0.f);
        if (b >= 0 && b < p.B)
            v = *reinterpret_cast<const float2 *>(p.qkv + (size_t)b * rows + c0);
        else if (b < 0 && pp >= 0)
            v = *reinterpret_cast<const float2 *>(p.ring + (size_t)(pp & 3) * rows + c0);
        xr[k] = v;
    }
    const uint4 wv = *reinterpret_cast<const uint4 *>(p.conv_w + (size_t)c0 * 4);
#pragma unroll
    for (int j = 0; j < CT; j++) {
        const int b = bb + j, pos = p.t0 + b;
        if (b >= p.B) break;
        const float x0[4] = {xr[j].x, xr[j + 1].x, xr[j + 2].x, xr[j + 3].x};
        const float x1[4] = {xr[j].y, xr[j + 1].y, xr[j + 2].y, xr[j + 3].y};
        float y0 = q35_conv_silu(x0, make_uint2(wv.x, wv.y), pos);
        float y1 = q35_conv_silu(x1, make_uint2(wv.z, wv.w), pos);
        if (grp < 2 * KH) {        /* q or k head: RMS norm (src/attn_qwen.c:522-538) */
#pragma clang fp contract(off)
            double ss = (double)y0 * y0 + (double)y1 * y1;
            ss = q35_wave_sum(ss);
            const float r = sqrtf((float)(ss / (double)KD) + 1e-6f);
            const float scale = grp < KH ? 1.0f / (float)KD : 1.0f / sqrtf((float)KD);
            y0 = y0 / r * scale;
            y1 = y1 / r * scale;
        }
        *reinterpret_cast<float2 *>(p.post + (size_t)b * rows + c0) = make_float2(y0, y1);
    }

    if (blockIdx.x == 0) {
        for (int i = threadIdx.x; i < CT * VH; i += 256) {
            const int b = bb + i / VH, h = i % VH;
            if (b >= p.B) break;
            float g, beta;
            q35_lin_gates(p.a[(size_t)b * VH + h], p.b[(size_t)b * VH + h], p.A_log[h],
                          p.dt_bias[h], &g, &beta);
            *reinterpret_cast<float2 *>(p.gates + ((size_t)b * VH + h) * 2) = make_float2(g, beta);
        }
    }
}

/* ---- 2. ring: slot pos%4 <- raw row of pos, for the last min(B, 4) tokens */
__global__ void ring_kernel(Q35LinPrefill p, int n) {
    const int rows = 2 * p.k_heads * KD + p.v_heads * VD;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * rows) return;
    const int r = (int)(i / rows), ch = (int)(i % rows);
    const int b = p.B - n + r, pos = p.t0 + b;
    p.ring[(size_t)(pos & 3) * rows + ch] = p.qkv[(size_t)b * rows + ch];
}

/* ---- 3. per (chunk, value head): A, Pm, W, U, Kd^T, decay vectors -------- */
__global__ __launch_bounds__(256) void chunk_kernel(Q35LinPrefill p) {
    const int c = blockIdx.x, h = blockIdx.y, kh = h >> 1;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int l16 = lane & 15, lq = lane >> 4;
    const int KH = p.k_heads, VH = p.v_heads;
    const int rows = 2 * KH * KD + VH * VD;
    const int b0 = c * C, nv = min(C, p.B - b0);

    /* sK: K rows (later the V rows); sQA: Q rows, later A^T.  One buffer, so
     * the output transpose at the end can use both halves. */
    __shared__ __align__(16) float sbuf[2 * C * XS];
    float *sK = sbuf, *sQA = sbuf + C * XS;
    __shared__ double sG[C];
    __shared__ float sBeta[C], sGq[C], sGk[C];

    /* gates and the chunk-local cumulative log-decay (pads: g = beta = 0) */
    if (w == 0) {
        float g = 0.f, beta = 0.f;
        if (lane < nv) {
            const float2 gb = *reinterpret_cast<const float2 *>(p.gates + ((size_t)(b0 + lane) * VH + h) * 2);
            g = gb.x;
            beta = gb.y;
        }
        double G = g;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(G, off);
            if (lane >= off) G += o;
        }
        sG[lane] = G;
        sBeta[lane] = beta;
        const double Gc = __shfl(G, 63);
        const float gq = (float)exp(G), gk = (float)exp(Gc - G);
        sGq[lane] = gq;
        sGk[lane] = gk;
        float *gv = p.gvec + ((size_t)c * VH + h) * Q35_LIN_GVEC;
        gv[lane] = gq;
        gv[C + lane] = gk;
        if (lane == 0) gv[2 * C] = (float)exp(Gc);
    }
    /* K and Q rows of the chunk (key head kh) into LDS; pad rows zero */
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int idx = u * 256 + t, r = idx >> 5, c4 = (idx & 31) * 4;
        float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), qv = kv;
        if (r < nv) {
            const float *row = p.post + (size_t)(b0 + r) * rows;
            kv = *reinterpret_cast<const float4 *>(row + KH * KD + kh * KD + c4);
            qv = *reinterpret_cast<const float4 *>(row + kh * KD + c4);
        }
        *reinterpret_cast<float4 *>(&sK[r * XS + c4]) = kv;
        *reinterpret_cast<float4 *>(&sQA[r * XS + c4]) = qv;
    }
    q35_lds_barrier();

    /* K K^T and Q K^T, the 10 lower 16x16 tiles of each: tile n (0..19),
     * wave w takes n = w, w+4, ..., w+16.  Lane l holds rows 4*(l/16)+i. */
    f32x4_t res[5];
#pragma unroll
    for (int k = 0; k < 5; k++) {
        const int n = w + 4 * k, m = n % 10;
        const int tr = m < 1 ? 0 : m < 3 ? 1 : m < 6 ? 2 : 3;
        const int tc = m - (tr * (tr + 1)) / 2;
        const float *X = n < 10 ? sK : sQA;
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int blk = 0; blk < KD / 16; blk++) {
            const float4 xa = *reinterpret_cast<const float4 *>(&X[(16 * tr + l16) * XS + 16 * blk + 4 * lq]);
            const float4 yb = *reinterpret_cast<const float4 *>(&sK[(16 * tc + l16) * XS + 16 * blk + 4 * lq]);
#pragma unroll
            for (int e = 0; e < 4; e++) acc = mfma4(el(xa, e), el(yb, e), acc);
        }
        res[k] = acc;
    }
    q35_lds_barrier();                       /* Q no longer read: its LDS becomes A^T */
    float *sAT = sQA;
    float *Pm = p.Pm + ((size_t)c * VH + h) * C * C;
#pragma unroll
    for (int k = 0; k < 5; k++) {
        const int n = w + 4 * k, m = n % 10;
        const int tr = m < 1 ? 0 : m < 3 ? 1 : m < 6 ? 2 : 3;
        const int tc = m - (tr * (tr + 1)) / 2;
        const int s = 16 * tc + l16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 16 * tr + 4 * lq + i;
            const float dec = expf((float)(sG[r] - sG[s]));
            if (n < 10)
                sAT[s * AS + r] = s < r ? sBeta[r] * dec * res[k][i] : 0.0f;
            else
                Pm[r * C + s] = s <= r ? dec * res[k][i] : 0.0f;
        }
    }
    q35_lds_barrier();

    /* Kd^T [kd][C] = exp(G_C - G_s) k_s[i]: thread (row i, keys 4q..4q+3)
     * writes 16 contiguous bytes of a 256-byte row */
    {
        float *kdt = p.KdT + ((size_t)c * VH + h) * KD * C;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int idx = u * 256 + t, i = idx >> 4, s4 = (idx & 15) * 4;
            float4 o;
            o.x = sGk[s4 + 0] * sK[(s4 + 0) * XS + i];
            o.y = sGk[s4 + 1] * sK[(s4 + 1) * XS + i];
            o.z = sGk[s4 + 2] * sK[(s4 + 2) * XS + i];
            o.w = sGk[s4 + 3] * sK[(s4 + 3) * XS + i];
            *reinterpret_cast<float4 *>(kdt + (size_t)i * C + s4) = o;
        }
    }

    /* forward substitution, one right-hand-side column a thread:
     * columns 0..127 -> W (rhs beta_r exp(G_r) k_r), 128..255 -> U (beta_r v_r).
     * Right-looking: once x_s is final it is applied to every later row, so
     * each step is up to 63 independent FMAs (column s of A is row s of
     * A^T, read four entries at a time).  The W columns read K from LDS;
     * the V rows then replace K there (16-byte loads) for the U columns. */
    float x[C];
    if (t < KD) {
#pragma unroll
        for (int r = 0; r < C; r++) x[r] = sBeta[r] * sGq[r] * sK[r * XS + t];
    }
    q35_lds_barrier();                     /* K no longer read */
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int idx = u * 256 + t, r = idx >> 5, c4 = (idx & 31) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < nv)
            v = *reinterpret_cast<const float4 *>(p.post + (size_t)(b0 + r) * rows + 2 * KH * KD + h * VD + c4);
        *reinterpret_cast<float4 *>(&sK[r * XS + c4]) = v;
    }
    q35_lds_barrier();
    if (t >= KD) {
#pragma unroll
        for (int r = 0; r < C; r++) x[r] = sBeta[r] * sK[r * XS + (t - KD)];
    }
#pragma unroll
    for (int s = 0; s < C - 1; s++) {
        const float xs = x[s];
#pragma unroll
        for (int r4 = ((s + 1) >> 2) << 2; r4 < C; r4 += 4) {
            const float4 a4 = *reinterpret_cast<const float4 *>(&sAT[s * AS + r4]);
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (r4 + e > s) x[r4 + e] = fmaf(-el(a4, e), xs, x[r4 + e]);
        }
    }
    /* W and U rows out through LDS: [64 rows][256 columns (W | U)], then
     * 16-byte row stores */
    q35_lds_barrier();                     /* A^T and V no longer read */
    constexpr int OSR = 2 * KD + 4;        /* output row stride (floats) */
#pragma unroll
    for (int r = 0; r < C; r++) sbuf[r * OSR + t] = x[r];
    q35_lds_barrier();
    {
        float *wd = p.W + ((size_t)c * VH + h) * C * KD, *ud = p.U + ((size_t)c * VH + h) * C * VD;
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int idx = u * 256 + t, r = idx >> 6, c4 = (idx & 63) * 4;
            const float4 o = *reinterpret_cast<const float4 *>(&sbuf[r * OSR + c4]);
            if (c4 < KD)
                *reinterpret_cast<float4 *>(wd + (size_t)r * KD + c4) = o;
            else
                *reinterpret_cast<float4 *>(ud + (size_t)r * VD + (c4 - KD)) = o;
        }
    }
}

/* ---- 4. sequential scan over chunks per (value head, 16-column block) ---- *
 * 8 waves in two roles.  Waves 0-3 compute from LDS only: wave w owns chunk
 * rows 16w..16w+15 of Delta / O and key rows 32w..32w+31 of the state
 * block.  Waves 4-7 move the chunk operands global -> registers -> LDS in
 * two regions:
 *   R1 = W, Q, the U slice and exp(G)   read in phase 1 (W S0, Q S0, Delta)
 *   R2 = Pm, Kd^T and exp(G_C)          read in phase 2 (Pm Delta, S_end)
 * R2 of chunk c is written while phase 1 of c runs, R1 of chunk c+1 while
 * phase 2 of c runs, so each region is refilled under the other phase's
 * MFMAs; a loader's global loads are issued one step before their data is
 * written.  The compute waves issue no global loads inside the loop, so
 * their output stores never make them wait, and the loaders' loads are
 * unconditional, so their waits count exactly.
 * Workgroup n runs head (n & 7) + 8 (n >> 6), block (n >> 3) & 7: the 8
 * blocks of a head share an XCD (workgroups are dealt round-robin over the
 * 8 XCDs), so the chunk operands they all read stay in one L2. */
constexpr int OS = 20;                 /* LDS row stride of the U and O tiles */
constexpr int SCAN_THREADS = 512;

struct ScanLds {
    float W[C * XS], Q[C * XS];        /* R1: rows [t][i] */
    float U[C * OS];                   /* R1: [t][j] */
    float Gq[C];                       /* R1: exp(G_t) */
    float P[C * AS];                   /* R2: Pm [t][s], upper tiles zero */
    float Kd[KD * AS];                 /* R2: Kd^T [i][s] */
    float Gc[4];                       /* R2: exp(G_C) */
    float S[16 * XS];                  /* state block [j][i] */
    float D[16 * AS];                  /* Delta [j][t] */
    float O[C * OS];                   /* O tile [t][j] */
};

struct ScanGeo {
    int h, jb, kh, VH, rows;
};

/* Loader staging, lane lt of the 256 loader lanes.  All operand loads are
 * raw buffer loads over the chunk's own block (range-checked, 32-bit lane
 * offsets): W, Pm and Kd^T row group u of lane lt sits at byte
 * 4096 u + 16 lt of its block. */
struct StageR1 {
    u32x4_t w[8], q[8], u, g;
};
struct StageR2 {
    u32x4_t pm[4], kd[8], gc;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t blk_rsrc(const float *base, size_t n_floats) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, (int)(n_floats * 4), Q35_BUF_DW3);
}

__device__ __forceinline__ void r1_load(StageR1 &st, const Q35LinPrefill &p, const ScanGeo &g,
                                        int c, int lt) {
    const int b0 = c * C, nv = min(C, p.B - b0);
    const size_t ch = (size_t)c * g.VH + g.h;
    const __amdgpu_buffer_rsrc_t wr = blk_rsrc(p.W + ch * C * KD, C * KD);
    const __amdgpu_buffer_rsrc_t qr = blk_rsrc(p.post + (size_t)b0 * g.rows, (size_t)nv * g.rows);
    const __amdgpu_buffer_rsrc_t ur = blk_rsrc(p.U + ch * C * VD, C * VD);
    const __amdgpu_buffer_rsrc_t gr = blk_rsrc(p.gvec + ch * Q35_LIN_GVEC, Q35_LIN_GVEC);
#pragma unroll
    for (int u = 0; u < 8; u++) {
        st.w[u] = __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * lt, 4096 * u, 0);
        /* rows past the batch read the last row's q: q row t only feeds
         * output row t, which is not stored for those rows */
        const int r = min(8 * u + (lt >> 5), nv - 1);
        st.q[u] = __builtin_amdgcn_raw_buffer_load_b128(qr, (r * g.rows + g.kh * KD + (lt & 31) * 4) * 4, 0, 0);
    }
    st.u = __builtin_amdgcn_raw_buffer_load_b128(ur, ((lt >> 2) * VD + 16 * g.jb + (lt & 3) * 4) * 4, 0, 0);
    st.g = __builtin_amdgcn_raw_buffer_load_b128(gr, 16 * (lt & 15), 0, 0);
}

__device__ __forceinline__ void r1_store(const StageR1 &st, ScanLds &L, int lt) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int r = 8 * u + (lt >> 5), c4 = (lt & 31) * 4;
        *reinterpret_cast<u32x4_t *>(&L.W[r * XS + c4]) = st.w[u];
        *reinterpret_cast<u32x4_t *>(&L.Q[r * XS + c4]) = st.q[u];
    }
    *reinterpret_cast<u32x4_t *>(&L.U[(lt >> 2) * OS + (lt & 3) * 4]) = st.u;
    /* lanes lt and lt + 16k write the same four values */
    *reinterpret_cast<u32x4_t *>(&L.Gq[4 * (lt & 15)]) = st.g;
}

__device__ __forceinline__ void r2_load(StageR2 &st, const Q35LinPrefill &p, const ScanGeo &g,
                                        int c, int lt) {
    const size_t ch = (size_t)c * g.VH + g.h;
    const __amdgpu_buffer_rsrc_t pr = blk_rsrc(p.Pm + ch * C * C, C * C);
    const __amdgpu_buffer_rsrc_t kr = blk_rsrc(p.KdT + ch * KD * C, KD * C);
    const __amdgpu_buffer_rsrc_t gr = blk_rsrc(p.gvec + ch * Q35_LIN_GVEC, Q35_LIN_GVEC);
#pragma unroll
    for (int u = 0; u < 4; u++) st.pm[u] = __builtin_amdgcn_raw_buffer_load_b128(pr, 16 * lt, 4096 * u, 0);
#pragma unroll
    for (int u = 0; u < 8; u++) st.kd[u] = __builtin_amdgcn_raw_buffer_load_b128(kr, 16 * lt, 4096 * u, 0);
    st.gc = __builtin_amdgcn_raw_buffer_load_b128(gr, 2 * C * 4, 0, 0);
}

__device__ __forceinline__ void r2_store(const StageR2 &st, ScanLds &L, int lt) {
    const int c4 = (lt & 15) * 4;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int r = 16 * u + (lt >> 4);
        /* the chunk kernel leaves Pm's tiles above the diagonal unwritten */
        const u32x4_t z = {0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4_t *>(&L.P[r * AS + c4]) = (c4 >> 4) > u ? z : st.pm[u];
    }
#pragma unroll
    for (int u = 0; u < 8; u++)
        *reinterpret_cast<u32x4_t *>(&L.Kd[(16 * u + (lt >> 4)) * AS + c4]) = st.kd[u];
    *reinterpret_cast<u32x4_t *>(&L.Gc[0]) = st.gc;      /* all lanes: same value */
}

__global__ __launch_bounds__(SCAN_THREADS) void scan_kernel(Q35LinPrefill p) {
    const int n = blockIdx.x;
    ScanGeo g;
    g.h = (n & 7) + 8 * (n >> 6);
    g.jb = (n >> 3) & 7;
    g.kh = g.h >> 1;
    g.VH = p.v_heads;
    g.rows = 2 * p.k_heads * KD + p.v_heads * VD;
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int last = p.n_chunks - 1;

    __shared__ __align__(16) ScanLds L;
    float *state = p.state + ((size_t)g.h * VD + 16 * g.jb) * KD;

    if (wave >= 4) {
        /* ---- loader waves ---- */
        const int lt = t - 256;
        StageR1 s1;
        StageR2 s2;
        r1_load(s1, p, g, 0, lt);
        r2_load(s2, p, g, 0, lt);
        r1_store(s1, L, lt);
        r1_load(s1, p, g, min(1, last), lt);
        q35_lds_barrier();                                   /* B0 */
        /* the scheduling barriers keep each region's LDS writes ahead of
         * the loads that refill its registers: issued in the other order,
         * the loads go to fresh registers that must be copied back before
         * the loop repeats, which waits for them */
        for (int c = 0; c <= last; c++) {
            /* phase 1 of c runs: R2 is free */
            r2_store(s2, L, lt);
            __builtin_amdgcn_sched_barrier(0);
            r2_load(s2, p, g, min(c + 1, last), lt);
            q35_lds_barrier();                               /* B1(c) */
            /* phase 2 of c runs: R1 is free */
            r1_store(s1, L, lt);
            __builtin_amdgcn_sched_barrier(0);
            r1_load(s1, p, g, min(c + 2, last), lt);
            q35_lds_barrier();                               /* B2(c) */
        }
        return;
    }

    /* ---- compute waves ---- */
    const int w = wave, lane = t & 63, l16 = lane & 15, lq = lane >> 4;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int idx = u * 256 + t, j = idx >> 5, i4 = (idx & 31) * 4;
        *reinterpret_cast<float4 *>(&L.S[j * XS + i4]) =
            *reinterpret_cast<const float4 *>(state + (size_t)j * KD + i4);
    }
    q35_lds_barrier();                                       /* B0 */
    for (int c = 0; c <= last; c++) {
        const int b0 = c * C, nv = min(C, p.B - b0);

        /* phase 1: W S0 and Q S0 on rows 16w.. over all 128 key rows */
        f32x4_t aw = {0.f, 0.f, 0.f, 0.f}, aq = aw;
#pragma unroll
        for (int blk = 0; blk < 8; blk++) {
            const int k = 16 * blk + 4 * lq;
            const float4 sb = *reinterpret_cast<const float4 *>(&L.S[l16 * XS + k]);
            const float4 wa = *reinterpret_cast<const float4 *>(&L.W[(16 * w + l16) * XS + k]);
            const float4 qa = *reinterpret_cast<const float4 *>(&L.Q[(16 * w + l16) * XS + k]);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                aw = mfma4(el(wa, e), el(sb, e), aw);
                aq = mfma4(el(qa, e), el(sb, e), aq);
            }
        }
        f32x4_t ao;
        float4 dl;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 16 * w + 4 * lq + i;
            ao[i] = L.Gq[r] * aq[i];
            const float d = L.U[r * OS + l16] - aw[i];
            if (i == 0) dl.x = d;
            if (i == 1) dl.y = d;
            if (i == 2) dl.z = d;
            if (i == 3) dl.w = d;
        }
        *reinterpret_cast<float4 *>(&L.D[l16 * AS + 16 * w + 4 * lq]) = dl;
        q35_lds_barrier();                                   /* B1(c) */

        /* phase 2: O += Pm Delta (key blocks 0..w), S_end on key rows 32w.. */
        float4 db[4];
#pragma unroll
        for (int blk = 0; blk < 4; blk++)
            db[blk] = *reinterpret_cast<const float4 *>(&L.D[l16 * AS + 16 * blk + 4 * lq]);
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            if (blk <= w) {       /* w is wave-uniform: a scalar branch */
                const float4 pa = *reinterpret_cast<const float4 *>(&L.P[(16 * w + l16) * AS + 16 * blk + 4 * lq]);
#pragma unroll
                for (int e = 0; e < 4; e++) ao = mfma4(el(pa, e), el(db[blk], e), ao);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) L.O[(16 * w + 4 * lq + i) * OS + l16] = ao[i];
        const float gc = L.Gc[0];
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            float *sp = &L.S[l16 * XS + 16 * (2 * w + tt) + 4 * lq];
            const float4 s0 = *reinterpret_cast<const float4 *>(sp);
            f32x4_t acc = {gc * s0.x, gc * s0.y, gc * s0.z, gc * s0.w};
#pragma unroll
            for (int blk = 0; blk < 4; blk++) {
                const float4 ka = *reinterpret_cast<const float4 *>(
                    &L.Kd[(16 * (2 * w + tt) + l16) * AS + 16 * blk + 4 * lq]);
#pragma unroll
                for (int e = 0; e < 4; e++) acc = mfma4(el(ka, e), el(db[blk], e), acc);
            }
            *reinterpret_cast<float4 *>(sp) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        }
        q35_lds_barrier();                                   /* B2(c) */

        /* O rows of this chunk: one 16-byte store a lane, rows >= nv fall
         * outside the buffer range and are dropped by the hardware */
        {
            const int r = t >> 2, c4 = (t & 3) * 4;
            const float4 o = *reinterpret_cast<const float4 *>(&L.O[r * OS + c4]);
            const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
                p.out + (size_t)b0 * g.VH * VD, 0, nv * g.VH * VD * 4, Q35_BUF_DW3);
            const u32x4_t ov = {__float_as_uint(o.x), __float_as_uint(o.y), __float_as_uint(o.z),
                                __float_as_uint(o.w)};
            __builtin_amdgcn_raw_buffer_store_b128(ov, ors, ((r * g.VH + g.h) * VD + 16 * g.jb + c4) * 4, 0, 0);
        }
    }

#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int idx = u * 256 + t, j = idx >> 5, i4 = (idx & 31) * 4;
        *reinterpret_cast<float4 *>(state + (size_t)j * KD + i4) =
            *reinterpret_cast<const float4 *>(&L.S[j * XS + i4]);
    }
}

/* ---- 5. RMSNormGated per (token, value head), in place on out ----------- *
 * grid (VH / 4, B), wave w -> head 4*blockIdx.x + w, 2 columns a lane. */
__global__ __launch_bounds__(256) void gnorm_kernel(Q35LinPrefill p) {
    const int b = blockIdx.y;
    const int h = 4 * blockIdx.x + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const size_t off = ((size_t)b * p.v_heads + h) * VD + 2 * lane;
    const float2 o = *reinterpret_cast<const float2 *>(p.out + off);
    const float2 z = *reinterpret_cast<const float2 *>(p.z + off);
    const uint32_t nw = *reinterpret_cast<const uint32_t *>(p.norm_w + 2 * lane);
    double ss = (double)o.x * o.x + (double)o.y * o.y;
    ss = q35_wave_sum(ss);
    float2 y;
    {
#pragma clang fp contract(off)
        const float r = sqrtf((float)(ss / (double)VD) + 1e-6f);
        y.x = o.x / r * q35_bf2f((uint16_t)(nw & 0xffff)) * (z.x * q35_sigmoid(z.x));
        y.y = o.y / r * q35_bf2f((uint16_t)(nw >> 16)) * (z.y * q35_sigmoid(z.y));
    }
    *reinterpret_cast<float2 *>(p.out + off) = y;
}

inline dim3 grid_for(int64_t n, int bs) { return dim3((unsigned)((n + bs - 1) / bs)); }

}  // namespace

extern "C" void q35_lin_prefill_ws_bytes(int B, int k_heads, int v_heads, int with_post,
                                         size_t *bytes) {
    const size_t rows = (size_t)2 * k_heads * KD + (size_t)v_heads * VD;
    const size_t nc = ((size_t)B + C - 1) / C, vh = (size_t)v_heads;
    size_t n = 0;
    if (with_post) n += (size_t)B * rows;                       /* post */
    n += (size_t)B * vh * 2;                                    /* gates */
    n += nc * vh * C * KD * 2;                                  /* W, U */
    n += nc * vh * C * C;                                       /* Pm */
    n += nc * vh * KD * C;                                      /* KdT */
    n += nc * vh * Q35_LIN_GVEC;                                /* gvec */
    *bytes = n * sizeof(float) + 8 * 256;     /* + alignment of the 7 pieces */
}

extern "C" hipError_t q35_lin_prefill(const Q35LinPrefill *pin, hipStream_t stream) {
    const Q35LinPrefill &p = *pin;
    const int rows = 2 * p.k_heads * KD + p.v_heads * VD;
    if (p.B < 1 || p.t0 < 0 || p.v_heads != 2 * p.k_heads || p.v_heads % 8 != 0 ||
        rows % 512 != 0 || p.n_chunks != (p.B + C - 1) / C)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(conv_kernel, dim3(rows / 512, (p.B + CT - 1) / CT), dim3(256), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nr = p.B < 4 ? p.B : 4;
    hipLaunchKernelGGL(ring_kernel, grid_for((int64_t)nr * rows, 256), dim3(256), 0, stream, p, nr);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(chunk_kernel, dim3(p.n_chunks, p.v_heads), dim3(256), 0, stream, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(scan_kernel, dim3(p.v_heads * (VD / 16)), dim3(SCAN_THREADS), 0, stream, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(gnorm_kernel, dim3(p.v_heads / 4, p.B), dim3(256), 0, stream, p);
    return hipGetLastError();
}
