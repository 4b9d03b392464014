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
 * 4 waves; wave w owns chunk rows 16w..16w+15 of Delta / O and key rows
 * 32w..32w+31 of the state block.  Workgroup n runs head
 * (n & 7) + 8 (n >> 6), block (n >> 3) & 7: the 8 blocks of a head share an
 * XCD (workgroups are dealt round-robin over the 8 XCDs), so the chunk
 * operands they all read stay in one L2.  The operands of chunk c+1 (they
 * do not depend on the state) are loaded into a second register set while
 * chunk c computes. */
struct ScanOps {
    float4 wa[8], qa[8], pa[4], ka[2][4];
    float u[4], gq[4], gc;
};

struct ScanCtx {
    int h, jb, kh, w, l16, lq, rows, VH;
};

__device__ __forceinline__ void scan_load(ScanOps &o, const Q35LinPrefill &p, const ScanCtx &x,
                                          int c) {
    const int b0 = c * C, nv = min(C, p.B - b0);
    const size_t ch = (size_t)c * x.VH + x.h;
    const float *Wc = p.W + ch * C * KD, *Uc = p.U + ch * C * VD;
    const float *Pc = p.Pm + ch * C * C, *Kc = p.KdT + ch * KD * C;
    const float *gv = p.gvec + ch * Q35_LIN_GVEC;
    const int row = 16 * x.w + x.l16;
#pragma unroll
    for (int blk = 0; blk < 8; blk++)
        o.wa[blk] = *reinterpret_cast<const float4 *>(Wc + (size_t)row * KD + 16 * blk + 4 * x.lq);
    /* every load is unconditional, so the compiler can count the loads in
     * flight exactly and wait for this set only.  Rows past the batch read
     * the last row's q: q row t only feeds output row t, which is not
     * stored for those rows. */
    const float *qrow = p.post + (size_t)(b0 + min(row, nv - 1)) * x.rows + x.kh * KD + 4 * x.lq;
#pragma unroll
    for (int blk = 0; blk < 8; blk++) o.qa[blk] = *reinterpret_cast<const float4 *>(qrow + 16 * blk);
#pragma unroll
    for (int blk = 0; blk < 4; blk++)   /* key blocks past the diagonal: unused */
        o.pa[blk] = *reinterpret_cast<const float4 *>(Pc + (size_t)row * C + 16 * blk + 4 * x.lq);
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
#pragma unroll
        for (int blk = 0; blk < 4; blk++)
            o.ka[tt][blk] = *reinterpret_cast<const float4 *>(
                Kc + (size_t)(16 * (2 * x.w + tt) + x.l16) * C + 16 * blk + 4 * x.lq);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 16 * x.w + 4 * x.lq + i;
        o.u[i] = Uc[(size_t)r * VD + 16 * x.jb + x.l16];
        o.gq[i] = gv[r];
    }
    o.gc = gv[2 * C];
}

__device__ __forceinline__ void scan_step(const ScanOps &o, const Q35LinPrefill &p,
                                          const ScanCtx &x, int c, float *sS, float *sD) {
    const int b0 = c * C, nv = min(C, p.B - b0);
    const int w = x.w, l16 = x.l16, lq = x.lq;

    /* W S0 and Q S0 (rows 16w.., all 128 key rows of the block) */
    f32x4_t aw = {0.f, 0.f, 0.f, 0.f}, aq = aw;
#pragma unroll
    for (int blk = 0; blk < 8; blk++) {
        const float4 sb = *reinterpret_cast<const float4 *>(&sS[l16 * XS + 16 * blk + 4 * lq]);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            aw = mfma4(el(o.wa[blk], e), el(sb, e), aw);
            aq = mfma4(el(o.qa[blk], e), el(sb, e), aq);
        }
    }
    float4 dl;
    dl.x = o.u[0] - aw[0];
    dl.y = o.u[1] - aw[1];
    dl.z = o.u[2] - aw[2];
    dl.w = o.u[3] - aw[3];
    *reinterpret_cast<float4 *>(&sD[l16 * AS + 16 * w + 4 * lq]) = dl;
    f32x4_t ao;
#pragma unroll
    for (int i = 0; i < 4; i++) ao[i] = o.gq[i] * aq[i];
    q35_lds_barrier();

    float4 db[4];
#pragma unroll
    for (int blk = 0; blk < 4; blk++)
        db[blk] = *reinterpret_cast<const float4 *>(&sD[l16 * AS + 16 * blk + 4 * lq]);
    /* O += Pm Delta (causal: key blocks 0..w) */
#pragma unroll
    for (int blk = 0; blk < 4; blk++) {
        if (blk <= w) {
#pragma unroll
            for (int e = 0; e < 4; e++) ao = mfma4(el(o.pa[blk], e), el(db[blk], e), ao);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 16 * w + 4 * lq + i;
        if (r < nv) p.out[((size_t)(b0 + r) * x.VH + x.h) * VD + 16 * x.jb + l16] = ao[i];
    }

    /* S_end = exp(G_C) S0 + Kd^T Delta on key rows 32w..32w+31 */
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
        float *sp = &sS[l16 * XS + 16 * (2 * w + tt) + 4 * lq];
        const float4 s0 = *reinterpret_cast<const float4 *>(sp);
        f32x4_t acc = {o.gc * s0.x, o.gc * s0.y, o.gc * s0.z, o.gc * s0.w};
#pragma unroll
        for (int blk = 0; blk < 4; blk++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc = mfma4(el(o.ka[tt][blk], e), el(db[blk], e), acc);
        *reinterpret_cast<float4 *>(sp) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
    q35_lds_barrier();
}

__global__ __launch_bounds__(256) void scan_kernel(Q35LinPrefill p) {
    const int n = blockIdx.x;
    ScanCtx x;
    x.h = (n & 7) + 8 * (n >> 6);
    x.jb = (n >> 3) & 7;
    x.kh = x.h >> 1;
    const int t = threadIdx.x, lane = t & 63;
    x.w = t >> 6;
    x.l16 = lane & 15;
    x.lq = lane >> 4;
    x.VH = p.v_heads;
    x.rows = 2 * p.k_heads * KD + p.v_heads * VD;

    __shared__ __align__(16) float sS[16 * XS];   /* state block, [j][i] */
    __shared__ __align__(16) float sD[16 * AS];   /* Delta, [j][t] */

    float *state = p.state + ((size_t)x.h * VD + 16 * x.jb) * KD;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int idx = u * 256 + t, j = idx >> 5, i4 = (idx & 31) * 4;
        *reinterpret_cast<float4 *>(&sS[j * XS + i4]) =
            *reinterpret_cast<const float4 *>(state + (size_t)j * KD + i4);
    }
    ScanOps A, B;
    scan_load(A, p, x, 0);
    q35_lds_barrier();

    /* the prefetch is unconditional (past the end it reloads the last chunk,
     * unused): a conditional one would leave the compiler unable to count
     * the loads in flight, and it would wait for all of them */
    const int last = p.n_chunks - 1;
    for (int c = 0; c < p.n_chunks; c += 2) {
        scan_load(B, p, x, min(c + 1, last));
        scan_step(A, p, x, c, sS, sD);
        if (c + 1 > last) break;
        scan_load(A, p, x, min(c + 2, last));
        scan_step(B, p, x, c + 1, sS, sD);
    }

#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int idx = u * 256 + t, j = idx >> 5, i4 = (idx & 31) * 4;
        *reinterpret_cast<float4 *>(state + (size_t)j * KD + i4) =
            *reinterpret_cast<const float4 *>(&sS[j * XS + i4]);
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
    hipLaunchKernelGGL(scan_kernel, dim3(p.v_heads * (VD / 16)), dim3(256), 0, stream, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(gnorm_kernel, dim3(p.v_heads / 4, p.B), dim3(256), 0, stream, p);
    return hipGetLastError();
}
