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
 *   A      = strict_lower( beta_t exp(G_t - G_s) k_t.k_s ),  T = (I + A)^-1
 *   Delta  = T diag(beta) (V - diag(exp(G)) K S0)   (the chunk's delta_t rows)
 *   O      = diag(exp(G)) Q S0 + Pm Delta,  Pm = lower( exp(G_t - G_s) q_t.k_s )
 *   S_end  = exp(G_C) S0 + K^T diag(exp(G_C - G)) Delta
 * (Delta is the WY form's U - W S0 with W = T diag(beta exp(G)) K and
 * U = T diag(beta) V, applied without forming W and U.)  Every factor
 * exp(G_t - G_s) has s <= t, so none exceeds 1.
 *
 * Kernels, in stream order:
 *   conv_kernel  per token: conv1d + SiLU (ring taps for positions before
 *                t0), q/k RMS-normalisation, gates -> post [B][rows] (the
 *                reference's mutated qkv) and gates [B][VH][2]
 *   chunk_kernel per (chunk, key head), strided over 512 workgroups: K K^T and Q K^T
 *                on fp32 MFMA (shared by the key head's two value heads),
 *                then per value head A, Pm, the decay vectors and T by
 *                16x16 blocks (diagonal blocks by back substitution, the
 *                rest on fp32 MFMA); the last chunk's workgroups also write
 *                the last min(B, 4) raw rows into the conv ring
 *   scan_kernel  per (value head, 16-column block of vd), sequential over
 *                chunks: the state block stays in LDS; K S0, Q S0, Delta,
 *                O and S_end on fp32 MFMA (v_mfma_f32_16x16x4_f32); O
 *                unnormalised into out
 *   gnorm_kernel per (4 tokens, value head): RMSNormGated of out with z
 *                (src/attn_qwen.c:726-749)
 * All arithmetic is fp32 (MFMA fp32 products are exact, accumulation fp32);
 * the conv's SiLU and norm reciprocal, the chunk's decay factors and the
 * gated norm's sigmoid and reciprocal use the hardware exp / rcp (about
 * 1 ulp); the chunk-local cumulative log-decay is summed in double.
 */
#include "q35_device.h"
#include "q35_launch.h"

namespace {

constexpr int KD = 128, VD = 128, C = 64;

__device__ __forceinline__ f32x4_t mfma4(float a, float b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float el(const float4 &v, int e) {
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

/* ---- 1. conv + SiLU, q/k norms, gates ------------------------------------ *
 * grid (rows / 1024, ceil(B / CT)), 4 waves; wave w owns channels
 * 256 (4 blockIdx.x + w) .. +255, two 128-channel head groups (q heads,
 * then k heads, then v heads), one per half-wave, 4 channels a lane, for
 * CT = 6 consecutive tokens: the 9 raw rows they tap are loaded once (a
 * sliding window instead of 4 loads per output).  Of CT = 4, 6, 8, 12, 16,
 * 24, 32 tokens a workgroup, 6 is the fastest (rocprof at 4096 tokens:
 * 47.9, 46.6, 48.4, 51.6, 53.2, 55.8, 58.2 us): the window's re-read rows
 * are served by the cache, and more, smaller workgroups keep more waves
 * streaming.  The q / k norm of a
 * head is a half-wave sum.  Against the reference's per-element IEEE
 * divisions and double square sums, the SiLU uses v_exp_f32 / v_rcp_f32,
 * the norm one reciprocal per token (each about 1 ulp) and an fp32 square
 * sum (128 terms, at most 8e-6 relative, about 1e-7 in practice): the
 * kernel then runs at the HBM rate of its 2 x B x rows x 4 bytes. */
constexpr int CT = 6;
__global__ __launch_bounds__(256) void conv_kernel(Q35LinPrefill p) {
    const int bb = blockIdx.y * CT;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int KH = p.k_heads, VH = p.v_heads;
    const int rows = 2 * KH * KD + VH * VD;
    const int c0 = (4 * blockIdx.x + w) * 256 + 4 * lane;
    const int grp = c0 >> 7;                       /* 128-channel group */
    /* k_heads is even, so both groups of a wave are q, both k or both v */
    const bool normed = grp < 2 * KH;

    /* the conv weights first, then the raw rows of positions t0+bb-3 ..
     * t0+bb+CT-1 in order, all unconditional range-checked buffer loads
     * (rows past the batch and positions before 0, addressed at the ring
     * view's end, read as zero): loads
     * complete in issue order, so token j's outputs wait only for the rows
     * up to j + 3 and its stores go out while the later rows arrive.  The
     * row view starts at the block's first row at or after row 0, so its
     * 32-bit offsets cover any batch length. */
    const uint4 wa = *reinterpret_cast<const uint4 *>(p.conv_w + (size_t)c0 * 4);
    const uint4 wb = *reinterpret_cast<const uint4 *>(p.conv_w + (size_t)c0 * 4 + 8);
    const int r0 = max(bb - 3, 0);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<float *>(p.qkv) + (size_t)r0 * rows), 0,
        min(p.B - r0, CT + 3) * rows * 4, Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(p.ring), 0, 4 * rows * 4, Q35_BUF_DW3);
    float4 xr[CT + 3];
#pragma unroll
    for (int k = 0; k < CT + 3; k++) {
        const int b = bb - 3 + k, pp = p.t0 + b;     /* block-uniform */
        const __amdgpu_buffer_rsrc_t rs = b >= 0 ? rq : rr;
        const uint32_t off = b >= 0 ? (uint32_t)(((b - r0) * rows + c0) * 4)
                             : pp >= 0 ? (uint32_t)(((pp & 3) * rows + c0) * 4) : (uint32_t)(4 * rows * 4);
        xr[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
    const uint2 wt[4] = {make_uint2(wa.x, wa.y), make_uint2(wa.z, wa.w), make_uint2(wb.x, wb.y),
                         make_uint2(wb.z, wb.w)};
    const float scale = grp < KH ? 1.0f / (float)KD : 1.0f / sqrtf((float)KD);
#pragma unroll
    for (int j = 0; j < CT; j++) {
        const int b = bb + j, pos = p.t0 + b;
        if (b >= p.B) break;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float x[4] = {el(xr[j], e), el(xr[j + 1], e), el(xr[j + 2], e), el(xr[j + 3], e)};
            y[e] = q35_conv_silu_fast(x, wt[e], pos);
        }
        if (normed) {              /* q or k head: RMS norm (src/attn_qwen.c:522-538) */
#pragma clang fp contract(off)
            float ss = y[0] * y[0] + y[1] * y[1] + y[2] * y[2] + y[3] * y[3];
            ss = q35_half_sum(ss);
            const float r = sqrtf(ss * (1.0f / (float)KD) + 1e-6f), ri = 1.0f / r;
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = y[e] * ri * scale;
        }
        *reinterpret_cast<float4 *>(p.post + (size_t)b * rows + c0) = make_float4(y[0], y[1], y[2], y[3]);
    }

    /* gates of the block's tokens, spread over the row-group workgroups */
    {
        for (int i = threadIdx.x * gridDim.x + blockIdx.x; i < CT * VH; i += 256 * gridDim.x) {
            const int b = bb + i / VH, h = i % VH;
            if (b >= p.B) break;
            float g, beta;
            q35_lin_gates(p.a[(size_t)b * VH + h], p.b[(size_t)b * VH + h], p.A_log[h],
                          p.dt_bias[h], &g, &beta);
            *reinterpret_cast<float2 *>(p.gates + ((size_t)b * VH + h) * 2) = make_float2(g, beta);
        }
    }
}

/* float offset of (row r, column k) in a [rows][128] / [rows][64] tile
 * stored with granule swizzle g ^ (r % 16) */
__device__ __forceinline__ int sw128(int r, int k) { return r * KD + ((((k >> 2) ^ (r & 15))) << 2) + (k & 3); }
__device__ __forceinline__ int sw64(int r, int k) { return r * C + ((((k >> 2) ^ (r & 15))) << 2) + (k & 3); }

/* T and Pm leave the chunk kernel as the 10 16x16 blocks (a, b), b <= a, of a 64x64 lower triangle: block
 * a (a + 1) / 2 + b at 256 floats each, row r of a block 16 floats (the
 * scan's LDS image of a block holds its 16-byte granule g of row r at
 * g ^ ((r >> 2) & 3), so an operand read of the 16 rows of one granule
 * column covers all 64 banks) */
__host__ __device__ constexpr int tri_idx(int a, int b) { return a * (a + 1) / 2 + b; }
__device__ __forceinline__ int tri_off(int j, int r, int gr) { return j * 256 + r * 16 + 4 * (gr ^ ((r >> 2) & 3)); }

/* 16x16 blocks of a 64x64 triangle: index of block (a, c), a <= c, among the
 * 10 blocks on and above the diagonal */
__device__ __forceinline__ int blk_q(int a, int c) { return a * (9 - a) / 2 + (c - a); }
constexpr int BS = 20, BLK = 16 * BS;

/* ---- 3. per (chunk, key head): decay vectors, Pm and T = (I + A)^-1 ------ *
 * The two value heads 2kh, 2kh+1 of key head kh share K K^T and Q K^T; they
 * differ in the gates.  Outputs per (chunk, value head): gvec, and Pm and
 * T (lower triangular, unit diagonal) as their 10 blocks on and below the
 * diagonal, 1 KB each (tri_idx), in a [64][64]-sized slot.
 * Items (chunk, key head) = (it % n_chunks, it / n_chunks) are strided over
 * at most CHUNK_GRID workgroups (two a CU): a workgroup requests the next
 * item's K and Q rows into registers as soon as the current item's rows are
 * in LDS, so they stream in under the current item's MFMA phases instead of
 * every workgroup of a second round loading at once. */
constexpr int CHUNK_GRID = 512;

/* thread t's 16 float4s of an item's K and Q rows: float4 u * 256 + t is
 * row idx >> 5, columns 4 (idx & 31) ..; raw buffer loads over the chunk's
 * rows, so rows past the batch end read as zero */
struct ChunkRows {
    float4 k[8], q[8];
};
__device__ __forceinline__ void chunk_rows_load(ChunkRows &R, const Q35LinPrefill &p, int it, int rows) {
    const int c = it % p.n_chunks, kh = it / p.n_chunks;
    const int b0 = c * C, nv = min(C, p.B - b0);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<float *>(p.post) + (size_t)b0 * rows), 0, nv * rows * 4, Q35_BUF_DW3);
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int idx = u * 256 + t, r = idx >> 5, c4 = (idx & 31) * 4;
        const int ok = (r * rows + (p.k_heads + kh) * KD + c4) * 4, oq = (r * rows + kh * KD + c4) * 4;
        R.k[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok, 0, 0));
        R.q[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, oq, 0, 0));
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void chunk_kernel(Q35LinPrefill p) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __builtin_assume(w >= 0 && w < 4);     /* 256 threads: tile n = w + 4k is K K^T for k < 2, Q K^T for k > 2 */
    const int KH = p.k_heads, VH = p.v_heads;
    const int rows = 2 * KH * KD + VH * VD;
    const int n_items = p.n_chunks * KH;

    /* K and Q rows, later A^T of both value heads, later T of both */
    __shared__ __align__(16) float sbuf[2 * C * KD];
    float *sK = sbuf, *sQ = sbuf + C * KD;
    __shared__ __align__(16) double sG[2][C];
    __shared__ __align__(16) float sBeta[2][C];

    ChunkRows R;
    chunk_rows_load(R, p, blockIdx.x, rows);
    for (int it = blockIdx.x; it < n_items; it += gridDim.x) {
        /* the thread index as an opaque value per item: the LDS addresses
         * derived from it are then computed where they are used, not hoisted
         * out of the item loop into registers held across it */
        int t = threadIdx.x;
        asm volatile("" : "+v"(t));
        const int lane = t & 63, l16 = lane & 15, lq = lane >> 4;
        const int c = it % p.n_chunks, kh = it / p.n_chunks;
        const int b0 = c * C, nv = min(C, p.B - b0);

        /* the conv ring: slot pos % 4 <- raw row of pos for the last min(B, 4)
         * tokens, written by the last chunk's items (the conv kernel, which
         * reads the ring, has finished) */
        if (c == p.n_chunks - 1) {
            const int nr = min(p.B, 4), n4 = rows / 4;
            for (int i = kh * 256 + t; i < nr * n4; i += KH * 256) {
                const int b = p.B - nr + i / n4, c4 = 4 * (i % n4);
                *reinterpret_cast<float4 *>(p.ring + (size_t)((p.t0 + b) & 3) * rows + c4) =
                    *reinterpret_cast<const float4 *>(p.qkv + (size_t)b * rows + c4);
            }
        }

        /* gates and the chunk-local cumulative log-decay of value head 2kh + w
         * (pads: g = beta = 0) */
        if (w < 2) {
            const int h = 2 * kh + w;
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
            sG[w][lane] = G;
            sBeta[w][lane] = beta;
            const double Gc = __shfl(G, 63);
            float *gv = p.gvec + ((size_t)c * VH + h) * Q35_LIN_GVEC;
            gv[lane] = (float)exp(G);
            gv[C + lane] = (float)exp(Gc - G);
            gv[2 * C + lane] = beta;
            if (lane == 0) gv[3 * C] = (float)exp(Gc);
        }
        /* the item's K and Q rows into LDS (pad rows zero), then the next
         * item's requested into the same registers */
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int idx = u * 256 + t, r = idx >> 5, c4 = (idx & 31) * 4;
            *reinterpret_cast<float4 *>(&sK[sw128(r, c4)]) = R.k[u];
            *reinterpret_cast<float4 *>(&sQ[sw128(r, c4)]) = R.q[u];
        }
        q35_lds_barrier();
        if (it + (int)gridDim.x < n_items) chunk_rows_load(R, p, it + gridDim.x, rows);

        /* K K^T and Q K^T, the 10 lower 16x16 tiles of each: tile n (0..19),
         * wave w takes n = w, w+4, ..., w+16.  Lane l holds rows 4*(l/16)+i. */
        f32x4_t res[5];
#pragma unroll
        for (int k = 0; k < 5; k++) {
            const int n = w + 4 * k, m = n % 10;
            const int tr = m < 1 ? 0 : m < 3 ? 1 : m < 6 ? 2 : 3;
            const int tc = m - (tr * (tr + 1)) / 2;
            const float *X = n < 10 ? sK : sQ;
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int blk = 0; blk < KD / 16; blk++) {
                const float4 xa = *reinterpret_cast<const float4 *>(&X[sw128(16 * tr + l16, 16 * blk + 4 * lq)]);
                const float4 yb = *reinterpret_cast<const float4 *>(&sK[sw128(16 * tc + l16, 16 * blk + 4 * lq)]);
#pragma unroll
                for (int e = 0; e < 4; e++) acc = mfma4(el(xa, e), el(yb, e), acc);
            }
            res[k] = acc;
        }
        q35_lds_barrier();                       /* K and Q no longer read */

        /* T = (I + A)^-1 in 16x16 blocks.  With M = A^T (strictly upper,
         * M[s][r] = A[r][s]) and U = (I + M)^-1 = T^T, for blocks a <= b:
         *   U_aa = (I + M_aa)^-1                      (back substitution)
         *   U_ab = -U_aa W,  W = sum_{c=a+1..b} M_ac U_cb   (by increasing b - a)
         * so T_ba = U_ab^T = -W^T U_aa^T.  LDS (in the K / Q rows' space):
         * MB the 10 upper blocks of M per value head, TB the 10 lower blocks of
         * T, UD the diagonal blocks of U row-major; a block is 16 rows of BS
         * floats (row stride 20 = 4 x odd: conflict-free 16-byte operand reads). */
        float *MB = sbuf, *TB = sbuf + 2 * 10 * BLK, *UD = sbuf + 4 * 10 * BLK;

        /* M blocks from the K K^T tiles: tile (tr >= tc) holds A[r][s] for r in
         * block tr, s in block tc, i.e. M block (tc, tr), row s, columns r;
         * Pm[r][s] = exp(G_r - G_s) q_r.k_s (s <= r) straight to its buffer */
#pragma unroll
        for (int k = 0; k < 5; k++) {
            const int n = w + 4 * k, m = n % 10;
            const int tr = m < 1 ? 0 : m < 3 ? 1 : m < 6 ? 2 : 3;
            const int tc = m - (tr * (tr + 1)) / 2;
            const int s = 16 * tc + l16;
            const int r0 = 16 * tr + 4 * lq;
#pragma unroll
            for (int v = 0; v < 2; v++) {
                /* the lane's G_s, its four G_r and beta_r read up front, the
                 * masks as selects: no LDS read waits inside a branch */
                const double gs = sG[v][s];
                const double2 g01 = *reinterpret_cast<const double2 *>(&sG[v][r0]);
                const double2 g23 = *reinterpret_cast<const double2 *>(&sG[v][r0 + 2]);
                const float4 bt = *reinterpret_cast<const float4 *>(&sBeta[v][r0]);
                const double gr[4] = {g01.x, g01.y, g23.x, g23.y};
                const float br[4] = {bt.x, bt.y, bt.z, bt.w};
                float o[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = r0 + i;
                    const float dec = __expf((float)(gr[i] - gs));   /* v_exp_f32, ~1 ulp */
                    const float av = br[i] * dec * res[k][i], pv = dec * res[k][i];
                    o[i] = n < 10 ? (s < r ? av : 0.0f) : (s <= r ? pv : 0.0f);
                }
                if (n < 10) {
                    *reinterpret_cast<float4 *>(&MB[(v * 10 + blk_q(tc, tr)) * BLK + l16 * BS + 4 * lq]) =
                        make_float4(o[0], o[1], o[2], o[3]);
                } else {
                    float *Pm = p.Pm + ((size_t)c * VH + 2 * kh + v) * C * C + tri_idx(tr, tc) * 256;
#pragma unroll
                    for (int i = 0; i < 4; i++) Pm[(4 * lq + i) * 16 + l16] = o[i];
                }
            }
        }
        q35_lds_barrier();

        /* diagonal blocks: wave w inverts block a = w of both value heads,
         * column kc of U_aa on lane kc (+16 for head 1; lanes 32-63 repeat
         * lanes 0-31 and do not write) */
        {
            const int a = w, v = (lane >> 4) & 1, kc = lane & 15;
            const float *Md = MB + (v * 10 + blk_q(a, a)) * BLK;
            float u[16];
#pragma unroll
            for (int s = 15; s >= 0; s--) {
                float4 mrow[4];
#pragma unroll
                for (int q = 0; q < 4; q++) mrow[q] = *reinterpret_cast<const float4 *>(&Md[s * BS + 4 * q]);
                float acc = s == kc ? 1.0f : 0.0f;
#pragma unroll
                for (int r = s + 1; r < 16; r++) acc = fmaf(-el(mrow[r >> 2], r & 3), u[r], acc);
                u[s] = acc;
            }
            if (lane < 32) {
                float *Td = TB + (v * 10 + blk_q(a, a)) * BLK + kc * BS;     /* T_aa row kc */
#pragma unroll
                for (int q = 0; q < 4; q++)
                    *reinterpret_cast<float4 *>(&Td[4 * q]) = make_float4(u[4 * q], u[4 * q + 1], u[4 * q + 2], u[4 * q + 3]);
                float *Ud = UD + (v * 4 + a) * BLK;
#pragma unroll
                for (int s = 0; s < 16; s++) Ud[s * BS + kc] = u[s];
            }
        }
        q35_lds_barrier();

        /* off-diagonal blocks by distance d = b - a: jobs (head v, block a),
         * dealt round-robin over the waves; each is two 16x16x16 products */
#pragma unroll
        for (int d = 1; d < 4; d++) {
            for (int j = w; j < 2 * (4 - d); j += 4) {
                const int v = j / (4 - d), a = j % (4 - d), b = a + d;
                f32x4_t wacc = {0.f, 0.f, 0.f, 0.f};
                for (int cb = a + 1; cb <= b; cb++) {
                    /* X = M_ac row-major; Y = U_cb, read as its transpose T_bc */
                    const float4 xa = *reinterpret_cast<const float4 *>(&MB[(v * 10 + blk_q(a, cb)) * BLK + l16 * BS + 4 * lq]);
                    const float4 yb = *reinterpret_cast<const float4 *>(&TB[(v * 10 + blk_q(cb, b)) * BLK + l16 * BS + 4 * lq]);
#pragma unroll
                    for (int e = 0; e < 4; e++) wacc = mfma4(el(xa, e), el(yb, e), wacc);
                }
                /* T_ba = (-W^T) U_aa^T: this lane's W entries W[4lq+e][l16] are
                 * X[l16][4lq+e] of -W^T as they stand; Y^T = U_aa row-major */
                const float4 ud = *reinterpret_cast<const float4 *>(&UD[(v * 4 + a) * BLK + l16 * BS + 4 * lq]);
                f32x4_t tb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int e = 0; e < 4; e++) tb = mfma4(-wacc[e], el(ud, e), tb);
                float *Tt = TB + (v * 10 + blk_q(a, b)) * BLK;
#pragma unroll
                for (int i = 0; i < 4; i++) Tt[(4 * lq + i) * BS + l16] = tb[i];
            }
            q35_lds_barrier();
        }

        /* T out: 2 heads x the 10 lower blocks x 16 rows x 4 float4, each wave
         * instruction one whole 1 KB block */
#pragma unroll
        for (int u = 0; u < 5; u++) {
            const int idx = u * 256 + t, v = idx / 640, rem = idx % 640;
            const int j = rem >> 6, r = (rem >> 2) & 15, q4 = rem & 3;
            const int bb = j < 1 ? 0 : j < 3 ? 1 : j < 6 ? 2 : 3, ba = j - tri_idx(bb, 0);
            const float4 o = *reinterpret_cast<const float4 *>(&TB[(v * 10 + blk_q(ba, bb)) * BLK + r * BS + 4 * q4]);
            *reinterpret_cast<float4 *>(p.T + ((size_t)c * VH + 2 * kh + v) * C * C + j * 256 + r * 16 + 4 * q4) = o;
        }
        q35_lds_barrier();                       /* T read out: the next item may overwrite the LDS */
    }
}

/* ---- 4. sequential scan over chunks per (value head, 16-column block) ---- *
 * With S0 the state block entering the chunk (all 128 key rows, 16 value
 * columns j), per chunk:
 *   phase 1   K S0;  X = diag(beta) (V - diag(exp(G)) K S0)
 *   phase 1b  Delta = T X                       (= U - W S0)
 *   phase 2   O = diag(exp(G)) Q S0 + Pm Delta
 *             S_end = exp(G_C) S0 + K^T diag(exp(G_C - G)) Delta
 * Q S0 is not on the recurrence's path: its operands are read into
 * registers in phase 1 and its key blocks fill phases 1b and 2 (8 - w and
 * w of them), so that every wave issues 32, 36 and 48 MFMAs in the three
 * phases instead of 64 and up to 16 and 48 (one wave at the maximum of
 * each phase).
 * 8 waves in two roles.  Waves 0-3 compute from LDS only: wave w owns rows
 * 16w.. of X and Delta, rows 16(3-w).. of O (so the causal products are
 * balanced: 116 MFMAs a wave), and key rows 32w..32w+31 of the state
 * block.  Waves 4-7 copy the operands global -> LDS with direct-to-LDS
 * buffer loads (no register staging), each into the tile's LDS image, and
 * count their own loads (vmcnt) before the barrier that publishes a tile:
 *   K (double-buffered)          read in 1 and 2, copied for c + 1 in 1 of c
 *   Pm (double-buffered)         read in 2,       copied for c + 1 in 1 of c
 *   gates (double-buffered)      read in 1 and 2, copied for c + 1 in 1 of c
 *   Q, V                         read in 1,       copied for c + 1 in 1b of c
 *   T                            read in 1b,      copied for c + 1 in 2 of c
 * so every copy has at least two phases to land, and the loads are spread
 * over the phases: a copy wave reaches a barrier only once it has issued
 * its loads, and the 18 a wave once issued in phase 1b (72 a CU) held the
 * barrier after it about 500 cycles.  T and Pm hold only their 10 lower
 * 16x16 blocks (tri_off), which frees the LDS for the second Pm buffer.
 * K and Q rows sit in LDS with 16-byte granule g of row r at granule
 * g ^ (r % 16) (the copy's lanes fetch the granule their slot holds), as do
 * the state block, X and Delta: the MFMA operand reads of 16 consecutive
 * rows hit 16 distinct bank groups.  Workgroups are dealt
 * round-robin over the 8 XCDs (id mod 8): with 8 | key heads, workgroup n
 * runs key head (n & 7) + 8 (n >> 7), its value head (n >> 6) & 1 and
 * block (n >> 3) & 7, so the 16 workgroups of a key head (both value
 * heads, all blocks: they all read its Q and K rows) share one XCD and its
 * L2; otherwise head (n & 7) + 8 (n >> 6), block (n >> 3) & 7 (the 8 blocks
 * of a value head on one XCD). */
constexpr int SCAN_THREADS = 512;

struct ScanLds {
    float K[2][C * KD];                /* K rows [t][i], chunk c in K[c & 1] (sw128) */
    float Q[C * KD];                   /* Q rows [t][i] (sw128) */
    float V[C * 16];                   /* V slice [t][j] */
    float T[10 * 256];                 /* the 10 lower 16x16 blocks of T (tri_off) */
    float P[2][10 * 256];              /* the same of Pm, chunk c in P[c & 1] */
    float G[2][Q35_LIN_GVEC];          /* gate vectors, chunk c in G[c & 1] */
    float S[16 * KD];                  /* state block [j][i] (sw128) */
    float X[16 * C];                   /* X [j][t] (sw64) */
    float D[16 * C];                   /* Delta [j][t] (sw64) */
};
static_assert(Q35_LIN_GVEC == 256, "a gate vector is four 64-float quarters, one per copy wave");

/* LDS row of V slice row t: rows t and t ^ 1 swap where bit 2 of t is set,
 * so the X update's reads of rows r and r + 4 (one 32-lane half of a wave)
 * fall in the two different 16-bank halves (the map is its own inverse) */
__device__ __forceinline__ int v_row(int t) { return t ^ ((t >> 2) & 1); }

struct ScanGeo {
    int h, jb, kh, VH, KH, rows;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t blk_rsrc(const float *base, size_t n_floats) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, (int)(n_floats * 4), Q35_BUF_DW3);
}

/* The copy waves' loads.  dw = 0..3 is the copy wave; each issues its
 * share of a tile: 1 KB copies dw, dw + 4, ... (lane l -> LDS bytes
 * 16 l .. of the copy) and a quarter of a gate vector. */
struct ScanCopy {
    const float *post, *T, *Pm, *gvec;
    int B;
    ScanGeo g;
    int dw, lane;
    uint32_t lK, lQ, lV, lT, lP, lG;            /* LDS byte addresses (K[0], P[0], G[0]; [1] follows) */

    /* 8 copies of a [64][128] row tile (K or Q rows, channels ch0 ..) */
    /* the post rows of chunk c (rows at and past the batch end read as zero) */
    __device__ __forceinline__ __amdgpu_buffer_rsrc_t rows(int c) const {
        const int b0 = c * C, nv = min(C, B - b0);
        return blk_rsrc(q35_uniform_ptr(post + (size_t)b0 * g.rows), (size_t)nv * g.rows);
    }
    template <int I0 = 0, int I1 = 8>
    __device__ __forceinline__ void rows128(uint32_t lds, int c, int ch0) const {
        const __amdgpu_buffer_rsrc_t rs = rows(c);
#pragma unroll
        for (int i = I0; i < I1; i++) {
            const int d = dw + 4 * i, r = 2 * d + (lane >> 5), gr = (lane & 31) ^ (r & 15);
            q35_dma16(rs, __builtin_amdgcn_readfirstlane(lds + 1024 * d),
                      (uint32_t)((r * g.rows + ch0 + 4 * gr) * 4), 0);
        }
    }
    /* K rows of chunk c into K[buf] */
    __device__ __forceinline__ void k(int c, int buf) const { rows128(lK + buf * C * KD * 4, c, (g.KH + g.kh) * KD); }
    /* the first or second half of those copies */
    template <int H>
    __device__ __forceinline__ void k_half(int c, int buf) const {
        rows128<4 * H, 4 * H + 4>(lK + buf * C * KD * 4, c, (g.KH + g.kh) * KD);
    }
    __device__ __forceinline__ void q(int c) const { rows128(lQ, c, g.kh * KD); }
    /* one copy of the V slice (16 rows of 16 floats) */
    __device__ __forceinline__ void v(int c) const {
        const __amdgpu_buffer_rsrc_t rs = rows(c);
        const int r = v_row(16 * dw + (lane >> 2));      /* the row this lane's LDS slot holds */
        q35_dma16(rs, __builtin_amdgcn_readfirstlane(lV + 1024 * dw),
                  (uint32_t)((r * g.rows + 2 * g.KH * KD + g.h * VD + 16 * g.jb + 4 * (lane & 3)) * 4), 0);
    }
    /* 3 of the 10 blocks of chunk c's T or Pm (blocks dw, dw + 4, dw + 8,
     * the last block again past 9: copy waves 2 and 3 write block 9 a
     * second and third time, the same bytes, so every wave counts 3 loads),
     * each 1 KB contiguous in memory; lane l -> bytes 16 l of the block's
     * LDS image: row l / 4, stored granule l % 4 */
    __device__ __forceinline__ void tri(uint32_t lds, const float *base, int c) const {
        const size_t ch = (size_t)c * g.VH + g.h;
        const __amdgpu_buffer_rsrc_t rs = blk_rsrc(q35_uniform_ptr(base + ch * C * C), C * C);
        const int r = lane >> 2, gr = (lane & 3) ^ ((r >> 2) & 3);
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int j = min(dw + 4 * i, 9);
            q35_dma16(rs, __builtin_amdgcn_readfirstlane(lds + 1024 * j), (uint32_t)((j * 256 + r * 16 + 4 * gr) * 4), 0);
        }
    }
    __device__ __forceinline__ void t(int c) const { tri(lT, T, c); }
    __device__ __forceinline__ void pm(int c, int buf) const { tri(lP + buf * 10 * 1024, Pm, c); }
    /* a quarter of chunk c's gate vector */
    __device__ __forceinline__ void gv(uint32_t lds, int c) const {
        const size_t ch = (size_t)c * g.VH + g.h;
        const __amdgpu_buffer_rsrc_t rs = blk_rsrc(q35_uniform_ptr(gvec + ch * Q35_LIN_GVEC), Q35_LIN_GVEC);
        q35_dma4(rs, __builtin_amdgcn_readfirstlane(lds + 256 * dw), (uint32_t)((64 * dw + lane) * 4), 0);
    }
};

/* an empty volatile asm that claims to change v: the MFMAs that use v stay
 * after the barrier before it (pure register operations are otherwise free
 * to move across it, and the compiler moved Q S0 back into phase 1) */
__device__ __forceinline__ void after_barrier(f32x4_t &v) { asm volatile("" : "+v"(v)); }

/* The compute waves' chunk loop, one instance per wave index W: the
 * wave-dependent block counts become compile-time, so each phase is one
 * basic block in which the scheduler interleaves the LDS reads with the
 * MFMAs (rocprof, 4096 tokens: scan 198.5 -> 193.9 us on one box) */
template <int W>
__device__ __forceinline__ void scan_chunks(ScanLds &L, const Q35LinPrefill &p, const ScanGeo &g,
                                            int last, int lane) {
    constexpr int w = W, rx = 16 * W, ro = 16 * (3 - W);
    const int l16 = lane & 15, lq = lane >> 4;
    for (int c = 0; c <= last; c++) {
        const int b0 = c * C, nv = min(C, p.B - b0);
        const float *Kc = L.K[c & 1], *Gc = L.G[c & 1], *Pc = L.P[c & 1];

        /* phase 1: K S0 on rows rx over all 128 key rows; the state block and
         * the Q rows ro of the 8 key blocks stay in registers for Q S0, which
         * runs in phases 1b and 2 (blocks 0..7-w and 8-w..7): every wave then
         * issues 32, 36 and 48 MFMAs in the three phases */
        f32x4_t ak = {0.f, 0.f, 0.f, 0.f}, aq = ak;
        float4 sbv[8], qav[8];
#pragma unroll
        for (int blk = 0; blk < 8; blk++) {
            const int k = 16 * blk + 4 * lq;
            sbv[blk] = *reinterpret_cast<const float4 *>(&L.S[sw128(l16, k)]);
            const float4 ka = *reinterpret_cast<const float4 *>(&Kc[sw128(rx + l16, k)]);
            qav[blk] = *reinterpret_cast<const float4 *>(&L.Q[sw128(ro + l16, k)]);
#pragma unroll
            for (int e = 0; e < 4; e++) ak = mfma4(el(ka, e), el(sbv[blk], e), ak);
        }
        float xr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = rx + 4 * lq + i;
            xr[i] = Gc[2 * C + r] * (L.V[v_row(r) * 16 + l16] - Gc[r] * ak[i]);
        }
        *reinterpret_cast<float4 *>(&L.X[sw64(l16, rx + 4 * lq)]) = make_float4(xr[0], xr[1], xr[2], xr[3]);
        q35_lds_barrier();                                   /* B1(c) */
        after_barrier(aq);

        /* phase 1b: Q S0 blocks 0..7-w from registers (under the T and X
         * reads), then Delta = T X on rows rx (key blocks 0..w) */
        f32x4_t ad = {0.f, 0.f, 0.f, 0.f};
        float4 ta[4], xb[4];
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            if (blk <= w) {       /* compile-time in each instance */
                ta[blk] = *reinterpret_cast<const float4 *>(&L.T[tri_off(tri_idx(w, blk), l16, lq)]);
                xb[blk] = *reinterpret_cast<const float4 *>(&L.X[sw64(l16, 16 * blk + 4 * lq)]);
            }
        }
#pragma unroll
        for (int blk = 0; blk < 8; blk++) {
            if (blk <= 7 - w) {
#pragma unroll
                for (int e = 0; e < 4; e++) aq = mfma4(el(qav[blk], e), el(sbv[blk], e), aq);
            }
        }
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            if (blk <= w) {
#pragma unroll
                for (int e = 0; e < 4; e++) ad = mfma4(el(ta[blk], e), el(xb[blk], e), ad);
            }
        }
        *reinterpret_cast<float4 *>(&L.D[sw64(l16, rx + 4 * lq)]) = make_float4(ad[0], ad[1], ad[2], ad[3]);
        q35_lds_barrier();                                   /* B2(c) */
        after_barrier(aq);

        /* phase 2: Q S0 blocks 8-w..7, then O = exp(G) Q S0 + Pm Delta on
         * rows ro (key blocks 0..3-w); exp(G) from the phase-2 gate copy */
        float4 db[4], pa[4];
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            db[blk] = *reinterpret_cast<const float4 *>(&L.D[sw64(l16, 16 * blk + 4 * lq)]);
            if (blk <= 3 - w)
                pa[blk] = *reinterpret_cast<const float4 *>(&Pc[tri_off(tri_idx(3 - w, blk), l16, lq)]);
        }
        const float4 eg = *reinterpret_cast<const float4 *>(&Gc[ro + 4 * lq]);
#pragma unroll
        for (int blk = 0; blk < 8; blk++) {
            if (blk > 7 - w) {
#pragma unroll
                for (int e = 0; e < 4; e++) aq = mfma4(el(qav[blk], e), el(sbv[blk], e), aq);
            }
        }
        f32x4_t ao = {eg.x * aq[0], eg.y * aq[1], eg.z * aq[2], eg.w * aq[3]};
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            if (blk <= 3 - w) {
#pragma unroll
                for (int e = 0; e < 4; e++) ao = mfma4(el(pa[blk], e), el(db[blk], e), ao);
            }
        }
        {
            /* rows >= nv fall outside the buffer range: the hardware drops them */
            const __amdgpu_buffer_rsrc_t ors = blk_rsrc(p.out + (size_t)b0 * g.VH * VD, (size_t)nv * g.VH * VD);
#pragma unroll
            for (int i = 0; i < 4; i++)
                __builtin_amdgcn_raw_buffer_store_b32(
                    __float_as_uint(ao[i]), ors, (((ro + 4 * lq + i) * g.VH + g.h) * VD + 16 * g.jb + l16) * 4, 0, 0);
        }
        /* S_end on key rows 32w..32w+31: A = K^T (one LDS dword per lane
         * and MFMA), B = exp(G_C - G_s) Delta */
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            const float4 gk = *reinterpret_cast<const float4 *>(&Gc[C + 16 * blk + 4 * lq]);
            db[blk].x *= gk.x;
            db[blk].y *= gk.y;
            db[blk].z *= gk.z;
            db[blk].w *= gk.w;
        }
        const float gc = Gc[3 * C];
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const int i0 = 16 * (2 * w + tt);
            float *sp = &L.S[sw128(l16, i0 + 4 * lq)];
            const float4 s0 = *reinterpret_cast<const float4 *>(sp);
            f32x4_t acc = {gc * s0.x, gc * s0.y, gc * s0.z, gc * s0.w};
#pragma unroll
            for (int blk = 0; blk < 4; blk++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    acc = mfma4(Kc[sw128(16 * blk + 4 * lq + e, i0 + l16)], el(db[blk], e), acc);
            *reinterpret_cast<float4 *>(sp) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        }
        q35_lds_barrier();                                   /* B3(c) */
    }
}

__global__ __launch_bounds__(SCAN_THREADS) void scan_kernel(Q35LinPrefill p) {
    const int n = blockIdx.x;
    ScanGeo g;
    if ((p.k_heads & 7) == 0) {
        g.h = 2 * ((n & 7) + 8 * (n >> 7)) + ((n >> 6) & 1);
    } else {
        g.h = (n & 7) + 8 * (n >> 6);
    }
    g.jb = (n >> 3) & 7;
    g.kh = g.h >> 1;
    g.VH = p.v_heads;
    g.KH = p.k_heads;
    g.rows = 2 * p.k_heads * KD + p.v_heads * VD;
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int last = p.n_chunks - 1;

    __shared__ __align__(16) ScanLds L;
    float *state = p.state + ((size_t)g.h * VD + 16 * g.jb) * KD;

    if (wave >= 4) {
        /* ---- copy waves: loads counted per wave (12 in step 1, 9 in
         * step 2, 3 in step 3 of every chunk) ---- */
        ScanCopy cp;
        cp.post = p.post;
        cp.T = p.T;
        cp.Pm = p.Pm;
        cp.gvec = p.gvec;
        cp.B = p.B;
        cp.g = g;
        cp.dw = wave - 4;
        cp.lane = t & 63;
        cp.lK = q35_lds_addr(L.K[0]);
        cp.lQ = q35_lds_addr(L.Q);
        cp.lV = q35_lds_addr(L.V);
        cp.lT = q35_lds_addr(L.T);
        cp.lP = q35_lds_addr(L.P[0]);
        cp.lG = q35_lds_addr(L.G[0]);
        cp.k(0, 0);
        cp.q(0);
        cp.v(0);
        cp.gv(cp.lG, 0);
        cp.t(0);
        cp.pm(0, 0);
        q35_wait_vm<0>();
        q35_lds_barrier();                                   /* B0 */
        for (int c = 0; c <= last; c++) {
            const int c1 = min(c + 1, last);
            /* step 1 (phase 1 of c): K, Pm and gates of c + 1, each into
             * the buffer phase 2 of c - 1 read */
            cp.k(c1, (c + 1) & 1);
            cp.pm(c1, (c + 1) & 1);
            cp.gv(cp.lG + ((c + 1) & 1) * 1024, c1);
            q35_wait_vm<12>();                               /* T of c (and Pm of c) */
            q35_lds_barrier();                               /* B1(c) */
            /* step 2 (phase 1b of c): Q, V of c + 1 */
            cp.q(c1);
            cp.v(c1);
            q35_lds_barrier();                               /* B2(c) */
            /* step 3 (phase 2 of c): T of c + 1 */
            cp.t(c1);
            q35_wait_vm<3>();                                /* K, Pm, gates, Q, V of c + 1 */
            q35_lds_barrier();                               /* B3(c) */
        }
        q35_wait_vm<0>();
        return;
    }

    /* ---- compute waves ---- */
    const int w = wave, lane = t & 63;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int idx = u * 256 + t, jj = idx >> 5, i4 = (idx & 31) * 4;
        *reinterpret_cast<float4 *>(&L.S[sw128(jj, i4)]) =
            *reinterpret_cast<const float4 *>(state + (size_t)jj * KD + i4);
    }
    q35_lds_barrier();                                       /* B0 */
    switch (w) {
    case 0: scan_chunks<0>(L, p, g, last, lane); break;
    case 1: scan_chunks<1>(L, p, g, last, lane); break;
    case 2: scan_chunks<2>(L, p, g, last, lane); break;
    default: scan_chunks<3>(L, p, g, last, lane); break;
    }

#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int idx = u * 256 + t, jj = idx >> 5, i4 = (idx & 31) * 4;
        *reinterpret_cast<float4 *>(state + (size_t)jj * KD + i4) =
            *reinterpret_cast<const float4 *>(&L.S[sw128(jj, i4)]);
    }
}

/* ---- 5. RMSNormGated per (4 tokens, value head), in place on out ------- *
 * grid (VH / 4, ceil(B / GTT)), wave w -> head 4*blockIdx.x + w of GTT
 * consecutive tokens, 2 columns a lane.  Every token's o and z rows are
 * requested before the first is used (GTT = 4 against one token a wave:
 * 35.7 -> 30.9 us at 4096 tokens, the kernel then at the HBM copy rate).
 * The reference's operation order (src/attn_qwen.c:726-749) with an fp32
 * square sum, x times 1 / r and the sigmoid on v_exp / v_rcp (about 1 ulp
 * each; the prefill outputs are checked to 2e-3). */
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

constexpr int GTT = 4;
template <int TT>
__global__ __launch_bounds__(256) void gnorm_kernel(Q35LinPrefill p) {
    const int h = 4 * blockIdx.x + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int b0 = blockIdx.y * TT;
    const uint32_t nw = *reinterpret_cast<const uint32_t *>(p.norm_w + 2 * lane);
    float2 oa[TT], za[TT];
#pragma unroll
    for (int k = 0; k < TT; k++) {
        const int b = min(b0 + k, p.B - 1);
        const size_t off = ((size_t)b * p.v_heads + h) * VD + 2 * lane;
        oa[k] = *reinterpret_cast<const float2 *>(p.out + off);
        za[k] = *reinterpret_cast<const float2 *>(p.z + off);
    }
#pragma unroll
    for (int k = 0; k < TT; k++) {
        const int b = b0 + k;
        if (b >= p.B) break;
        const size_t off = ((size_t)b * p.v_heads + h) * VD + 2 * lane;
        const float2 o = oa[k], z = za[k];
        float ss = o.x * o.x + o.y * o.y;
        ss = q35_wave_sum(ss);
        float2 y;
        {
#pragma clang fp contract(off)
            const float r = sqrtf(ss * (1.0f / (float)VD) + 1e-6f), ri = 1.0f / r;
            y.x = o.x * ri * q35_bf2f((uint16_t)(nw & 0xffff)) * (z.x * q35_sigmoid_fast(z.x));
            y.y = o.y * ri * q35_bf2f((uint16_t)(nw >> 16)) * (z.y * q35_sigmoid_fast(z.y));
        }
        if (!p.xw) {
            *reinterpret_cast<float2 *>(p.out + off) = y;
            continue;
        }
        q35_f16_guard(p.status, Q35_STATUS_GEMM_F16, q35_f16_over(y.x) || q35_f16_over(y.y));
        /* The chunk GEMM's X operand instead: quad lanes 4k..4k+3 hold word k
         * of the head's 16 (values 2i, 2i + 1 in quad lane i); every lane of the
         * quad gathers the word, lane 0 stores its hi granule, lane 1 its lo.
         * The group sums (64 columns = one half wave) add the same hi + lo. */
        float w8[8];
        w8[0] = q35_dpp<0x00>(y.x), w8[1] = q35_dpp<0x00>(y.y);
        w8[2] = q35_dpp<0x55>(y.x), w8[3] = q35_dpp<0x55>(y.y);
        w8[4] = q35_dpp<0xAA>(y.x), w8[5] = q35_dpp<0xAA>(y.y);
        w8[6] = q35_dpp<0xFF>(y.x), w8[7] = q35_dpp<0xFF>(y.y);
        f16x8 hi, lo;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v = w8[q35_xw_perm(j)];
            hi[j] = (_Float16)v;
            lo[j] = (_Float16)(v - (float)hi[j]);
        }
        const _Float16 hx = (_Float16)y.x, hy = (_Float16)y.y;
        float s = ((float)hx + (float)(_Float16)(y.x - (float)hx)) + ((float)hy + (float)(_Float16)(y.y - (float)hy));
        s = q35_half_sum(s);
        const int G = p.v_heads * VD / 64, v = h * (VD / 8) + (lane >> 2);
        uint8_t *gr = reinterpret_cast<uint8_t *>(p.xw) + q35_xw_granule(b, v, G);
        if ((lane & 3) == 0) *reinterpret_cast<f16x8 *>(gr) = hi;
        if ((lane & 3) == 1) *reinterpret_cast<f16x8 *>(gr + Q35_XW_BLK) = lo;
        if ((lane & 31) == 0) p.xsum[(size_t)(v >> 3) * p.mpad + b] = s;
    }
}


}  // namespace

extern "C" void q35_lin_prefill_ws_bytes(int B, int k_heads, int v_heads, int with_post,
                                         size_t *bytes) {
    const size_t rows = (size_t)2 * k_heads * KD + (size_t)v_heads * VD;
    const size_t nc = ((size_t)B + C - 1) / C, vh = (size_t)v_heads;
    size_t n = 0;
    if (with_post) n += (size_t)B * rows;                       /* post */
    n += (size_t)B * vh * 2;                                    /* gates */
    n += nc * vh * C * C * 2;                                   /* T, Pm */
    n += nc * vh * Q35_LIN_GVEC;                                /* gvec */
    *bytes = n * sizeof(float) + 6 * 256;     /* + alignment of the 5 pieces */
}

extern "C" hipError_t q35_lin_prefill(const Q35LinPrefill *pin, hipStream_t stream) {
    const Q35LinPrefill &p = *pin;
    const int rows = 2 * p.k_heads * KD + p.v_heads * VD;
    if (p.B < 1 || p.t0 < 0 || p.v_heads != 2 * p.k_heads || p.v_heads % 8 != 0 ||
        p.k_heads % 2 != 0 || rows % 1024 != 0 || p.n_chunks != (p.B + C - 1) / C)
        return hipErrorInvalidValue;
    /* checked before any launch: the kernels advance the ring and state in place */
    if (p.xw && (p.mpad < p.B || p.mpad % Q35_XW_ROWS != 0 || !p.xsum)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(conv_kernel, dim3(rows / 1024, (p.B + CT - 1) / CT), dim3(256), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(chunk_kernel, dim3(min(p.n_chunks * p.k_heads, CHUNK_GRID)), dim3(256), 0, stream, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(scan_kernel, dim3(p.v_heads * (VD / 16)), dim3(SCAN_THREADS), 0, stream, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(gnorm_kernel<GTT>, dim3(p.v_heads / 4, (p.B + GTT - 1) / GTT), dim3(256), 0, stream, p);
    return hipGetLastError();
}

/* ---- the workspace of the no-allocation entry point ---------------------
 * One file-scope device array: every GPU the library runs on holds its own
 * copy until the process ends, and every no-allocation call on that GPU
 * uses it (its contents are the last call's; each call writes every part
 * it reads before reading it, so nothing needs clearing).  In host code the
 * name `scratch` is a host-side stand-in, not a device address: the device
 * address comes from hipGetSymbolAddress, taken once per device with that
 * device current (q35_lin_scratch_init, called by the plugin's init) and
 * kept per device in scratch_dev. */
static __device__ __align__(256) unsigned char scratch[Q35_LIN_SCRATCH_BYTES];

namespace {
constexpr int SCRATCH_MAX_DEV = 64;
void *scratch_dev[SCRATCH_MAX_DEV];
}  // namespace

extern "C" hipError_t q35_lin_scratch_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= SCRATCH_MAX_DEV) return hipErrorInvalidDevice;
    if (scratch_dev[dev]) return hipSuccess;
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    scratch_dev[dev] = ptr;
    return hipSuccess;
}

extern "C" void *q35_lin_scratch(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_MAX_DEV) return nullptr;
    return scratch_dev[dev];
}
