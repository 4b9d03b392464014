/*
 * gqa_decode.hip -- one decode token of a full-GQA layer on gfx950:
 * split-K flash-decode over the bf16 KV cache.
 *
 * Replaces gqa_body's per-token work (src/attn_qwen.c:279-396): q_norm /
 * k_norm, half-split partial RoPE, cache write of the new k / v, softmax
 * attention of 16 q heads over 2 kv heads, sigmoid output gate.
 *
 * Kernel 1 (split): grid = (P chunks, kv heads), 512 threads (8 waves, one
 * q head's norm / RoPE each).  A workgroup streams `chunk` cached positions
 * of one kv head and serves all 8 q heads of that kv head from the same K/V
 * bytes; wave w takes the 16-position tiles w, w + 8, ...:
 *   scores  S[16 pos][16 col] = K[16 pos][256] * Q^T on 16x16x32 bf16 MFMA,
 *           columns 0-7 holding the bf16 "hi" part of the 8 q heads and
 *           columns 8-15 the "lo" remainder (q = hi + lo to ~2^-16), so the
 *           fp32 q is used at near-fp32 precision; hi + lo are summed with
 *           one DPP lane exchange;
 *   values  O^T[16 dim][16 col] += V^T[16 dim][16 pos] * P^T on 16x16x16
 *           bf16 MFMA, P split the same way (hi | lo columns);
 *   online softmax per wave, the 8 waves merged in LDS (wave w merges
 *   head w), one partial (max, sum, O[8][256]) written per workgroup.
 * The new token (position `token`) is attended in fp32 from registers (as
 * the reference does with its fp32 cache) by the last chunk's workgroup,
 * which also writes the bf16 cache row.
 * Kernel 2 (merge): rescales and sums the P partials of each q head and
 * applies the gate, one wave per (head, 16 dims) with wave reductions only.
 *
 * Every global input of the prologue is loaded up front so the workgroup
 * pays one memory round trip before its main loop, not one per element.
 */
#include "q35_device.h"
#include "q35_launch.h"

namespace {

constexpr int D = Q35_GQA_D, G = Q35_GQA_GROUP, RD = Q35_ROPE_DIMS;
constexpr int NW = 8, NT = 64 * NW;   /* waves per workgroup, threads */
constexpr int HPW = G / NW;           /* q heads normed per wave in the prologue */
constexpr int MAX_CHUNKS = 256;
constexpr int OS = D + 4;             /* sO head stride: the 8 heads' 16-byte stores of a dim block start 4 banks apart */
static_assert(NW == G, "wave w merges q head w of the kv head");
constexpr float SCALE = 0.0625f;      /* 1/sqrtf(256), src/attn_qwen.c:334 */
struct KTile { bf16x8_t k[8]; };
struct VTile { s16x4_t v[16]; };

/* Tile loads are raw buffer loads over the workgroup's own chunk: `off` is
 * the tile's byte offset (8192 bytes a tile) plus the lane's; a tile past
 * the chunk's end lies outside the resource's range, and the hardware
 * returns zeros for it without a memory access.  Nontemporal: the KV is
 * streamed once, and the delta-rule states stay cache-resident. */
__device__ __forceinline__ void load_k(KTile &kt, __amdgpu_buffer_rsrc_t rs, int off) {
    /* lane: block kk at +kk*1024 bytes, row lane & 15 (+64 B), 8 dims at
     * (lane >> 4) * 16 B */
#pragma unroll
    for (int kk = 0; kk < 8; kk++)
        kt.k[kk] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off + kk * 1024, 0, 2));
}
__device__ __forceinline__ void load_v(VTile &vt, __amdgpu_buffer_rsrc_t rs, int off) {
    /* lane: dim row 16dt + (lane & 15) (+32 B a row), 4 tokens at
     * (lane >> 4) * 8 B; dim block dt at +dt*512 bytes */
#pragma unroll
    for (int dt = 0; dt < 16; dt++)
        vt.v[dt] = __builtin_bit_cast(s16x4_t, __builtin_amdgcn_raw_buffer_load_b64(rs, off + dt * 512, 0, 2));
}

/* max of v over lanes l and l ^ 16 (l ^ 32): gfx950's row-swap moves.  With
 * both operands v, permlane16_swap returns v's even rows in both rows of a
 * row pair in one result and its odd rows in the other (permlane32_swap
 * the same for the two halves), so the max of v and both results is the
 * pair's max, with no LDS permute. */
__device__ __forceinline__ float pair_max16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(fmaxf(v, __uint_as_float(r[0])), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_max32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(fmaxf(v, __uint_as_float(r[0])), __uint_as_float(r[1]));
}
/* q_norm + RoPE of one q head, as q35_norm_rope_head but with an fp32
 * square sum and the hardware reciprocal square root (about 1 ulp against
 * the double sum and IEEE division): q feeds the hi / lo bf16 split and
 * the scores only, while the new k row, which the cache stores, keeps the
 * reference's operation order. */
__device__ __forceinline__ float4 norm_rope_fast(float4 x, uint2 w, float4 c, float4 s, int lane) {
    const float ri = __builtin_amdgcn_rsqf(q35_wave_sum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w) * (1.0f / D) + 1e-6f);
    float v[4] = {x.x, x.y, x.z, x.w};
    const uint16_t wt[4] = {(uint16_t)(w.x & 0xffff), (uint16_t)(w.x >> 16),
                            (uint16_t)(w.y & 0xffff), (uint16_t)(w.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = v[e] * ri * q35_bf2f(wt[e]);
    const float cc[4] = {c.x, c.y, c.z, c.w}, sn[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float pr = q35_xor8(v[e]);
        if (lane < RD / 8)
            v[e] = v[e] * cc[e] - pr * sn[e];
        else if (lane < RD / 4)
            v[e] = pr * sn[e] + v[e] * cc[e];
    }
    return make_float4(v[0], v[1], v[2], v[3]);
}
/* One 16-position sub-tile: scores on MFMA, online-softmax update, P split
 * into hi | lo columns, P*V on MFMA into acc.  next_k(kt) runs as soon as
 * the score MFMAs have read the K registers, so the next tile's K loads go
 * out under this tile's softmax and P*V (op at 32K 15.8 -> 15.5 us in the
 * stack graph, against issuing them with the V loads after P*V). */
template <typename NextK>
__device__ __forceinline__ void attend_tile(KTile &kt, VTile &vt, const bf16x8_t *sqb,
                                            int lane, int base, int c1, int grp, bool is_lo,
                                            float &m_run, float &l_run, f32x4_t (&acc)[16],
                                            NextK next_k) {
    f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 8; kk++)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt.k[kk], sqb[kk * 64 + lane], sc, 0, 0, 0);
    next_k(kt);   /* the K registers are free: the next tile's K goes out now */
    /* lane holds S[pos 4grp+i][col n]; add the partner column (hi<->lo) */
    float sv[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float v = sc[i] + q35_xor8(sc[i]);
        const int pos = base + 4 * grp + i;
        v = (pos < c1) ? v * SCALE : -INFINITY;
        sv[i] = v;
        tmax = fmaxf(tmax, v);
    }
    tmax = pair_max16(tmax);     /* max over lanes l, l ^ 16, l ^ 32, l ^ 48 */
    tmax = pair_max32(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = q35_exp(m_run - m_new);   /* m_run = -inf -> 0 */
    const bool rescale = __any(m_new != m_run && m_run != -INFINITY);
    m_run = m_new;
    s16x4_t pb;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float pv = q35_exp(sv[i] - m_new);
        psum += pv;
        uint16_t hi, lo;
        q35_split_bf16(pv, hi, lo);
        pb[i] = (short)(is_lo ? lo : hi);
    }
    l_run = l_run * alpha + psum;
    if (rescale) {   /* wave-uniform: skipped while no running max moves */
#pragma unroll
        for (int dt = 0; dt < 16; dt++) acc[dt] *= alpha;
    }
    if (base + 16 > c1) {
        /* partial tail tile: zero V of masked positions (0 * junk) */
        const int valid = c1 - base;   /* 1..15 */
#pragma unroll
        for (int dt = 0; dt < 16; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++) vt.v[dt][i] = (4 * grp + i >= valid) ? 0 : vt.v[dt][i];
    }
#pragma unroll
    for (int dt = 0; dt < 16; dt++)
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt.v[dt], pb, acc[dt], 0, 0, 0);
}

/* The arguments are scalars, not the struct, so that the first nine (14
 * dwords: what the prologue and the first K/V tiles need) are preloaded
 * into SGPRs at wave launch (-amdgpu-kernarg-preload-count=9 for this
 * file); the rest load while those loads are in flight. */
__global__ __launch_bounds__(NT) void gqa_split_kernel(int token, int t_tiles, int chunk, int n_chunks,
                                                       const float *q_gate, const uint16_t *qn_w,
                                                       const float *rope, uint16_t *kt, uint16_t *vt,
                                                       const float *k_new, const float *v_new,
                                                       const uint16_t *kn_w, float *part_o, float *part_ml,
                                                       float *k_post, int heads, int kv_heads) {
    Q35GqaDecode p;
    p.token = token, p.t_tiles = t_tiles, p.chunk = chunk, p.n_chunks = n_chunks;
    p.q_gate = q_gate, p.qn_w = qn_w, p.rope = rope, p.kt = kt, p.vt = vt;
    p.k_new = k_new, p.v_new = v_new, p.kn_w = kn_w, p.part_o = part_o, p.part_ml = part_ml;
    p.k_post = k_post, p.heads = heads, p.kv_heads = kv_heads, p.attn_out = nullptr;
    const int c = blockIdx.x, g = blockIdx.y;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int n_past = p.token;
    const int c0 = c * p.chunk;
    const int c1 = min(c0 + p.chunk, n_past);
    const bool last = (c == p.n_chunks - 1);
    const int d0 = lane * 4;

    /* this wave's first K/V tile is requested right after the prologue's
     * own loads (loads complete in issue order, so the prologue's waits do
     * not cover it), and its HBM latency runs under the q norm / RoPE work */
    const int n_sub = (c1 > c0) ? (c1 - c0 + 15) >> 4 : 0;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(p.kt + (size_t)g * p.t_tiles * (D / 32) * 512 +
                                                (size_t)(c0 >> 4) * (D / 32) * 512)),
        0, n_sub * 8192, Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(p.vt + (size_t)g * p.t_tiles * D * 16 + (size_t)(c0 >> 4) * D * 16)),
        0, n_sub * 8192, Q35_BUF_DW3);
    const int wv = __builtin_amdgcn_readfirstlane(w);
    const int koff = (lane & 15) * 64 + (lane >> 4) * 16, voff = (lane & 15) * 32 + (lane >> 4) * 8;

    __shared__ __align__(16) float sQ[G][D];
    __shared__ bf16x8_t sQb[8 * 64];
    __shared__ __align__(16) float sO[NW][G * OS];
    __shared__ float sM[NW + 1][G], sL[NW + 1][G];
    __shared__ __align__(16) float sKn[D], sVn[D];

    /* ---- prologue: every input in flight at once ---- */
    float4 xq[HPW];
#pragma unroll
    for (int hh = 0; hh < HPW; hh++)
        xq[hh] = *reinterpret_cast<const float4 *>(p.q_gate + (size_t)(g * G + HPW * w + hh) * 2 * D +
                                                   d0);
    const uint2 wq = *reinterpret_cast<const uint2 *>(p.qn_w + d0);
    float4 rc = make_float4(1.f, 1.f, 1.f, 1.f), rs = make_float4(0.f, 0.f, 0.f, 0.f);
    if (lane < RD / 4) {
        rc = *reinterpret_cast<const float4 *>(p.rope + (d0 & (RD / 2 - 1)));
        rs = *reinterpret_cast<const float4 *>(p.rope + RD / 2 + (d0 & (RD / 2 - 1)));
    }
    const bool newtok = last && w == 0;
    float4 xk = make_float4(0.f, 0.f, 0.f, 0.f), xv = xk;
    uint2 wk = make_uint2(0, 0);
    if (newtok) {
        xk = *reinterpret_cast<const float4 *>(p.k_new + (size_t)g * D + d0);
        xv = *reinterpret_cast<const float4 *>(p.v_new + (size_t)g * D + d0);
        wk = *reinterpret_cast<const uint2 *>(p.kn_w + d0);
    }
    KTile ka;
    VTile va;
    load_k(ka, krs, wv * 8192 + koff);
    load_v(va, vrs, wv * 8192 + voff);

    /* q of heads HPW*w .. HPW*w+HPW-1 (of this kv head): norm + RoPE, then straight into
     * the MFMA B-operand layout: entry [kk][lane'] holds 8 bf16 of column
     * n = lane'&15 (head n&7, hi if n<8 else lo) for dims 32kk + 8*(lane'>>4).
     * This lane's dims 4l..4l+3 are half of one such entry. */
    const int kk0 = d0 >> 5, gp0 = (d0 >> 3) & 3, half = (d0 >> 2) & 1;
#pragma unroll
    for (int hh = 0; hh < HPW; hh++) {
        const int qh = HPW * w + hh;
        const float4 y = norm_rope_fast(xq[hh], wq, rc, rs, lane);
        *reinterpret_cast<float4 *>(&sQ[qh][d0]) = y;
        const float yy[4] = {y.x, y.y, y.z, y.w};
        s16x4_t hv, lv;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint16_t hi, lo;
            q35_split_bf16(yy[e], hi, lo);
            hv[e] = (short)hi;
            lv[e] = (short)lo;
        }
        s16x4_t *dst_hi = reinterpret_cast<s16x4_t *>(&sQb[kk0 * 64 + qh + 16 * gp0]) + half;
        s16x4_t *dst_lo = reinterpret_cast<s16x4_t *>(&sQb[kk0 * 64 + qh + 8 + 16 * gp0]) + half;
        *dst_hi = hv;
        *dst_lo = lv;
    }
    if (newtok) {
        /* the new token: k_norm + RoPE in fp32, cache row write (bf16) */
        const float4 y = q35_norm_rope_head(xk, wk, rc, rs, lane);
        *reinterpret_cast<float4 *>(&sKn[d0]) = y;
        *reinterpret_cast<float4 *>(&sVn[d0]) = xv;
        if (p.k_post) *reinterpret_cast<float4 *>(p.k_post + (size_t)g * D + d0) = y;
        const float ky[4] = {y.x, y.y, y.z, y.w}, vy[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            p.kt[q35_k_index(g, p.token, d0 + e, p.t_tiles)] = q35_f2bf(ky[e]);
            p.vt[q35_v_index(g, p.token, d0 + e, p.t_tiles)] = q35_f2bf(vy[e]);
        }
    }
    q35_lds_barrier();

    /* ---- main loop over 16-position sub-tiles w, w+4, ... of the chunk ---- */
    const int n = lane & 15, grp = lane >> 4, hq = n & 7;
    const bool is_lo = n >= 8;
    float m_run = -INFINITY, l_run = 0.0f;
    f32x4_t acc[16];
#pragma unroll
    for (int dt = 0; dt < 16; dt++) acc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    /* tiles wv, wv + NW, ...: each one's K loads are issued as soon as the
     * previous tile's scores are done, its V loads once the previous tile's
     * P*V has read the V registers.  The last tile requests nothing: a
     * load past the chunk reads zeros without a memory access, but the wave
     * still waits for it before it can retire (measured: 1.1 us a call at
     * 32768 positions). */
    const int n_mine = (n_sub > wv) ? (n_sub - wv + NW - 1) / NW : 0;
    for (int i = 0; i < n_mine; i++) {
        const int s0 = wv + i * NW;
        const bool more = i + 1 < n_mine;
        attend_tile(ka, va, sQb, lane, c0 + 16 * s0, c1, grp, is_lo, m_run, l_run, acc, [&](KTile &kt) {
            if (more) load_k(kt, krs, (s0 + NW) * 8192 + koff);
        });
        if (more) load_v(va, vrs, (s0 + NW) * 8192 + voff);
    }

    /* ---- per-wave partial: l over the 4 lane groups; O hi + lo columns ---- */
    l_run = q35_psum16(l_run);
    l_run = q35_psum32(l_run);
    /* lane (n < 8, grp) holds dims 16dt + 4grp .. +3 of head n: one 16-byte
     * LDS store per dim block */
#pragma unroll
    for (int dt = 0; dt < 16; dt++) {
        float4 o4;
        o4.x = acc[dt][0] + q35_xor8(acc[dt][0]);
        o4.y = acc[dt][1] + q35_xor8(acc[dt][1]);
        o4.z = acc[dt][2] + q35_xor8(acc[dt][2]);
        o4.w = acc[dt][3] + q35_xor8(acc[dt][3]);
        if (!is_lo) *reinterpret_cast<float4 *>(&sO[w][hq * OS + 16 * dt + 4 * grp]) = o4;
    }
    if (lane < G) {
        sM[w][lane] = m_run;
        sL[w][lane] = l_run;
    }
    if (last && w == 1) {
        /* the new token's score for the 8 heads, fp32 dot products */
        const float4 kn = *reinterpret_cast<const float4 *>(&sKn[d0]);
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
            const float4 q = *reinterpret_cast<const float4 *>(&sQ[hh][d0]);
            float d = q.x * kn.x + q.y * kn.y + q.z * kn.z + q.w * kn.w;
            d = q35_wave_sum(d);
            if (lane == hh) {
                sM[NW][hh] = d * SCALE;
                sL[NW][hh] = 1.0f;
            }
        }
    }
    q35_lds_barrier();

    /* ---- merge the waves (and the new token) ---- *
     * wave w merges head w: every lane reads the 8 waves' (max, sum) of the
     * head (broadcast LDS reads), forms the factors itself, and sums its 4
     * dims of the 8 partial rows; lane 0 stores the head's (max, sum). */
    float *po = p.part_o + ((size_t)(g * p.n_chunks + c) * G) * D;
    float *pml = p.part_ml + ((size_t)(g * p.n_chunks + c) * G) * 2;
    {
        const int hh = w, d4 = 4 * lane;
        float ms[NW];
        const float mnew = last ? sM[NW][hh] : -INFINITY;
        float M = mnew;
#pragma unroll
        for (int s2 = 0; s2 < NW; s2++) {
            ms[s2] = sM[s2][hh];
            M = fmaxf(M, ms[s2]);
        }
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < NW; s2++) {
            const float f = (ms[s2] == -INFINITY) ? 0.0f : q35_exp(ms[s2] - M);
            const float4 v = *reinterpret_cast<const float4 *>(&sO[s2][hh * OS + d4]);
            L = fmaf(sL[s2][hh], f, L);
            o.x = fmaf(v.x, f, o.x);
            o.y = fmaf(v.y, f, o.y);
            o.z = fmaf(v.z, f, o.z);
            o.w = fmaf(v.w, f, o.w);
        }
        if (last) {
            const float f = q35_exp(mnew - M);
            const float4 v = *reinterpret_cast<const float4 *>(&sVn[d4]);
            L = fmaf(sL[NW][hh], f, L);
            o.x = fmaf(v.x, f, o.x);
            o.y = fmaf(v.y, f, o.y);
            o.z = fmaf(v.z, f, o.z);
            o.w = fmaf(v.w, f, o.w);
        }
        const __amdgpu_buffer_rsrc_t ors =
            __builtin_amdgcn_make_buffer_rsrc(q35_uniform_ptr(po), 0, G * D * 4, Q35_BUF_DW3);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, o), ors, (hh * D + d4) * 4, 0,
                                               Q35_ST_SC1);
        if (lane == 0) {
            const __amdgpu_buffer_rsrc_t mrs =
                __builtin_amdgcn_make_buffer_rsrc(q35_uniform_ptr(pml), 0, G * 2 * 4, Q35_BUF_DW3);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M), mrs, hh * 8, 0, Q35_ST_SC1);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(L), mrs, hh * 8 + 4, 0, Q35_ST_SC1);
        }
    }
}

/* merge: one wave per (q head, 16 output dims), grid (heads, D/16).  Lane l
 * takes the chunks l, l + 64, ... (at most MCH a lane: 2 for the split's
 * usual P <= 128, whose instance carries no dead chunk slots, else
 * MAX_CHUNKS / 64) and loads their (max, sum) and 16 output dims in one
 * memory round trip; the maximum and the weighted sum are wave reductions
 * on DPP lanes and the 16 dim totals one transposing reduction, with no LDS
 * and no barrier. */
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, q35_dpp<0xB1>(v));
    v = fmaxf(v, q35_dpp<0x4E>(v));
    v = fmaxf(v, q35_dpp<0x141>(v));
    v = fmaxf(v, q35_dpp<0x140>(v));
    return pair_max32(pair_max16(v));
}
template <int MCH>
__global__ __launch_bounds__(64) void gqa_merge_kernel(int n_chunks, int heads, const float *part_ml,
                                                       const float *part_o, const float *q_gate,
                                                       float *attn_out) {
    Q35GqaDecode p;
    p.n_chunks = n_chunks, p.heads = heads, p.part_ml = const_cast<float *>(part_ml);
    p.part_o = const_cast<float *>(part_o), p.q_gate = q_gate, p.attn_out = attn_out;
    const int h = blockIdx.x, g = h / G, hh = h % G, d0 = 16 * blockIdx.y;
    const int lane = threadIdx.x;
    const int P = p.n_chunks;
    float mc[MCH], lc[MCH];
    float4 oc[MCH][4];
#pragma unroll
    for (int j = 0; j < MCH; j++) {
        const int c = lane + 64 * j;
        const bool valid = c < P;
        const size_t row = (size_t)(g * P + (valid ? c : 0)) * G + hh;
        const float2 ml = valid ? *reinterpret_cast<const float2 *>(p.part_ml + row * 2)
                                : make_float2(-INFINITY, 0.0f);
        mc[j] = ml.x;
        lc[j] = ml.y;
#pragma unroll
        for (int q = 0; q < 4; q++)
            oc[j][q] = valid ? *reinterpret_cast<const float4 *>(p.part_o + row * D + d0 + 4 * q)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float gate = lane < 16 ? p.q_gate[(size_t)h * 2 * D + D + d0 + lane] : 0.0f;

    float M = mc[0];
#pragma unroll
    for (int j = 1; j < MCH; j++) M = fmaxf(M, mc[j]);
    M = wave_max(M);
    float wgt[MCH], ls = 0.0f;
#pragma unroll
    for (int j = 0; j < MCH; j++) {
        wgt[j] = (mc[j] == -INFINITY) ? 0.0f : q35_exp(mc[j] - M);
        ls = fmaf(lc[j], wgt[j], ls);
    }
    const float L = q35_wave_sum(ls);
    float v[16];
#pragma unroll
    for (int d = 0; d < 16; d++) {
        v[d] = 0.0f;
#pragma unroll
        for (int j = 0; j < MCH; j++) {
            const float4 o4 = oc[j][d >> 2];
            const float od = (d & 3) == 0 ? o4.x : (d & 3) == 1 ? o4.y : (d & 3) == 2 ? o4.z : o4.w;
            v[d] = fmaf(od, wgt[j], v[d]);
        }
    }
    /* the 16 dim totals over the wave as a transposing reduction: in each
     * 16-lane row, four pairings (lane i with 15 - i, with its mirror in
     * the 8-lane half, with i ^ 2, with i ^ 1) each flip one bit of i; a
     * lane keeps the half of its dims whose index bit matches its own and
     * adds the partner's copy of that half, so lane i ends with its row's
     * total of dim i; the four rows are then summed with two row swaps */
    const int li = lane & 15;
    float a8[8], a4[4], a2[2];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const bool hi = li & 8;
        a8[j] = (hi ? v[j + 8] : v[j]) + q35_dpp<0x140>(hi ? v[j] : v[j + 8]);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const bool hi = li & 4;
        a4[j] = (hi ? a8[j + 4] : a8[j]) + q35_dpp<0x141>(hi ? a8[j] : a8[j + 4]);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const bool hi = li & 2;
        a2[j] = (hi ? a4[j + 2] : a4[j]) + q35_dpp<0x4E>(hi ? a4[j] : a4[j + 2]);
    }
    float tot = ((li & 1) ? a2[1] : a2[0]) + q35_dpp<0xB1>((li & 1) ? a2[0] : a2[1]);
    tot = q35_psum16(tot);
    tot = q35_psum32(tot);
    if (lane < 16)
        __builtin_amdgcn_raw_buffer_store_b32(
            __float_as_uint(tot * __builtin_amdgcn_rcpf(L) * q35_sigmoid_fast(gate)),
            __builtin_amdgcn_make_buffer_rsrc(q35_uniform_ptr(p.attn_out), 0, p.heads * D * 4, Q35_BUF_DW3),
            (h * D + d0 + lane) * 4, 0, Q35_ST_SC1);
}

}  // namespace

extern "C" void q35_gqa_split(int n_past, int *chunk, int *n_chunks) {
    /* about 128 chunks per kv head (256 workgroups); chunks are multiples of
     * 64 positions (4 sub-tiles per wave at least) */
    const int target = 128;
    int per = (n_past + target - 1) / target;
    int ch = ((per + 63) / 64) * 64;
    if (ch < 64) ch = 64;
    int P = (n_past + ch - 1) / ch;
    if (P < 1) P = 1;
    *chunk = ch;
    *n_chunks = P;
}

extern "C" int q35_gqa_max_chunks(void) { return MAX_CHUNKS; }

extern "C" hipError_t q35_gqa_decode(const Q35GqaDecode *p, hipStream_t stream) {
    if (p->heads != p->kv_heads * G || p->n_chunks < 1 || p->n_chunks > MAX_CHUNKS)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gqa_split_kernel, dim3(p->n_chunks, p->kv_heads), dim3(NT), 0, stream, p->token,
                       p->t_tiles, p->chunk, p->n_chunks, p->q_gate, p->qn_w, p->rope, p->kt, p->vt, p->k_new,
                       p->v_new, p->kn_w, p->part_o, p->part_ml, p->k_post, p->heads, p->kv_heads);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p->n_chunks <= 128)
        hipLaunchKernelGGL(gqa_merge_kernel<2>, dim3(p->heads, D / 16), dim3(64), 0, stream, p->n_chunks,
                           p->heads, p->part_ml, p->part_o, p->q_gate, p->attn_out);
    else
        hipLaunchKernelGGL(gqa_merge_kernel<MAX_CHUNKS / 64>, dim3(p->heads, D / 16), dim3(64), 0, stream,
                           p->n_chunks, p->heads, p->part_ml, p->part_o, p->q_gate, p->attn_out);
    return hipGetLastError();
}
