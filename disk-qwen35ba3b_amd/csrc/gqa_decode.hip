/*
 * gqa_decode.hip -- one decode token of a full-GQA layer on gfx950:
 * split-K flash-decode over the bf16 KV cache.
 *
 * Replaces gqa_body's per-token work (src/attn_qwen.c:279-396): q_norm /
 * k_norm, half-split partial RoPE, cache write of the new k / v, softmax
 * attention of 16 q heads over 2 kv heads, sigmoid output gate.
 *
 * Kernel 1 (split): grid = (P chunks, kv heads), 256 threads.  A workgroup
 * streams `chunk` cached positions of one kv head and serves all 8 q heads
 * of that kv head from the same K/V bytes:
 *   scores  S[16 pos][16 col] = K[16 pos][256] * Q^T on 16x16x32 bf16 MFMA,
 *           with columns 0-7 holding the bf16 "hi" part of the 8 q heads and
 *           columns 8-15 the "lo" remainder (q = hi + lo to ~2^-16), so the
 *           fp32 q is used at near-fp32 precision; hi + lo are summed with
 *           one lane exchange;
 *   values  O^T[16 dim][16 col] += V^T[16 dim][16 pos] * P^T on 16x16x16
 *           bf16 MFMA, P split the same way (hi | lo columns);
 *   online softmax per wave, the 4 waves merged in LDS, one partial
 *   (max, sum, O[8][256]) written per workgroup.
 * The new token (position `token`) is attended in fp32 from registers (as
 * the reference does with its fp32 cache) by the last chunk's workgroup,
 * which also writes the bf16 cache row.
 * Kernel 2 (merge): rescales and sums the P partials of each q head and
 * applies the gate.
 */
#include "q35_device.h"
#include "q35_launch.h"

namespace {

constexpr int D = Q35_GQA_D, G = Q35_GQA_GROUP, RD = Q35_ROPE_DIMS;
constexpr int NT = 256, NW = 4;
constexpr int MAX_CHUNKS = 128;
constexpr float SCALE = 0.0625f;   /* 1/sqrtf(256), src/attn_qwen.c:334 */

/* q_norm (RMSNorm, double sum, eps on the mean) + half-split RoPE of one
 * head held as 4 dims per lane (dims 4l..4l+3); returns the 4 values. */
__device__ __forceinline__ float4 norm_rope_head(float4 x, const uint16_t *w, const float *rope,
                                                 int lane) {
#pragma clang fp contract(off)
    double ss = (double)x.x * x.x + (double)x.y * x.y + (double)x.z * x.z + (double)x.w * x.w;
    ss = q35_wave_sum(ss);
    float r = sqrtf((float)(ss / (double)D) + 1e-6f);
    const int d0 = lane * 4;
    float v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = v[e] / r * q35_bf2f(w[d0 + e]);
    /* RoPE pairs (i, i+32), i < 32: lanes 0..7 hold i, lanes 8..15 hold i+32 */
    float pr[4];
#pragma unroll
    for (int e = 0; e < 4; e++) pr[e] = __shfl_xor(v[e], 8);
    if (lane < RD / 4) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            int i = (d0 + e) & (RD / 2 - 1);
            float c = rope[i], s = rope[RD / 2 + i];
            if (lane < RD / 8)
                v[e] = v[e] * c - pr[e] * s;        /* x0*c - x1*s */
            else
                v[e] = pr[e] * s + v[e] * c;        /* x0*s + x1*c */
        }
    }
    return make_float4(v[0], v[1], v[2], v[3]);
}

struct KTile { bf16x8_t k[8]; };
struct VTile { s16x4_t v[16]; };

__device__ __forceinline__ void load_k(KTile &kt, const uint16_t *base, int lane) {
    /* base: the 16-token tile's first 16x32 block; block kk at +kk*512 */
    const int m = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 8; kk++)
        kt.k[kk] = *reinterpret_cast<const bf16x8_t *>(base + kk * 512 + m * 32 + grp * 8);
}
__device__ __forceinline__ void load_v(VTile &vt, const uint16_t *base, int lane) {
    /* base: the tile's [256 dim][16 tok] block; dims 16dt.. at +dt*256 */
    const int m = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int dt = 0; dt < 16; dt++)
        vt.v[dt] = *reinterpret_cast<const s16x4_t *>(base + (dt * 16 + m) * 16 + grp * 4);
}

__global__ __launch_bounds__(NT) void gqa_split_kernel(Q35GqaDecode p) {
    const int c = blockIdx.x, g = blockIdx.y;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int n_past = p.token;
    const int c0 = c * p.chunk;
    const int c1 = min(c0 + p.chunk, n_past);
    const bool last = (c == p.n_chunks - 1);

    __shared__ float sQ[G][D];
    __shared__ float sO[NW][G][D];
    __shared__ float sM[NW + 1][G], sL[NW + 1][G];
    __shared__ float sKn[D], sVn[D];

    /* q of heads 8g+2w, 8g+2w+1: norm + RoPE */
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const int qh = 2 * w + hh;
        const float4 x = *reinterpret_cast<const float4 *>(p.q_gate + (size_t)(g * G + qh) * 2 * D +
                                                           lane * 4);
        const float4 y = norm_rope_head(x, p.qn_w, p.rope, lane);
        *reinterpret_cast<float4 *>(&sQ[qh][lane * 4]) = y;
    }
    if (last && w == 0) {
        /* the new token: k_norm + RoPE in fp32, cache row write (bf16) */
        const float4 x = *reinterpret_cast<const float4 *>(p.k_new + (size_t)g * D + lane * 4);
        const float4 y = norm_rope_head(x, p.kn_w, p.rope, lane);
        const float4 vv = *reinterpret_cast<const float4 *>(p.v_new + (size_t)g * D + lane * 4);
        *reinterpret_cast<float4 *>(&sKn[lane * 4]) = y;
        *reinterpret_cast<float4 *>(&sVn[lane * 4]) = vv;
        if (p.k_post) *reinterpret_cast<float4 *>(p.k_post + (size_t)g * D + lane * 4) = y;
        const float ky[4] = {y.x, y.y, y.z, y.w}, vy[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            p.kt[q35_k_index(g, p.token, lane * 4 + e, p.t_tiles)] = q35_f2bf(ky[e]);
            p.vt[q35_v_index(g, p.token, lane * 4 + e, p.t_tiles)] = q35_f2bf(vy[e]);
        }
    }
    __syncthreads();

    /* Q as the MFMA B operand: column n = lane&15 (head n&7, hi if n<8 else
     * lo), k-step kk covers dims 32kk + 8*grp .. +8 */
    const int n = lane & 15, grp = lane >> 4, hq = n & 7;
    const bool is_lo = n >= 8;
    bf16x8_t qb[8];
#pragma unroll
    for (int kk = 0; kk < 8; kk++) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            uint16_t hi, lo;
            q35_split_bf16(sQ[hq][32 * kk + 8 * grp + e], hi, lo);
            qb[kk][e] = q35_as_bf16(is_lo ? lo : hi);
        }
    }

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4_t acc[16];
#pragma unroll
    for (int dt = 0; dt < 16; dt++) acc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int n_sub = (c1 > c0) ? (c1 - c0 + 15) >> 4 : 0;
    const size_t kv_head_k = (size_t)g * p.t_tiles * (D / 32) * 512;
    const size_t kv_head_v = (size_t)g * p.t_tiles * D * 16;
    for (int s = w; s < n_sub; s += NW) {
        const int base = c0 + 16 * s;
        const int tile = base >> 4;
        KTile kt;
        VTile vt;
        load_k(kt, p.kt + kv_head_k + (size_t)tile * (D / 32) * 512, lane);
        load_v(vt, p.vt + kv_head_v + (size_t)tile * D * 16, lane);

        f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 8; kk++)
            sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt.k[kk], qb[kk], sc, 0, 0, 0);
        /* lane holds S[pos 4grp+i][col n]; add the partner column (hi<->lo) */
        float sv[4];
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v = sc[i] + __shfl_xor(sc[i], 8);
            const int pos = base + 4 * grp + i;
            v = (pos < c1) ? v * SCALE : -INFINITY;
            sv[i] = v;
            tmax = fmaxf(tmax, v);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = expf(m_run - m_new);   /* m_run = -inf -> 0 */
        m_run = m_new;
        s16x4_t pb;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float pv = expf(sv[i] - m_new);
            psum += pv;
            uint16_t hi, lo;
            q35_split_bf16(pv, hi, lo);
            pb[i] = (short)(is_lo ? lo : hi);
        }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < 16; dt++) acc[dt] *= alpha;
        if (base + 16 > c1) {
            /* partial tail tile: zero V of masked positions (0 * junk) */
            const int valid = c1 - base;   /* 1..15 */
#pragma unroll
            for (int dt = 0; dt < 16; dt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (4 * grp + i >= valid) vt.v[dt][i] = 0;
        }
#pragma unroll
        for (int dt = 0; dt < 16; dt++)
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt.v[dt], pb, acc[dt], 0, 0, 0);
    }

    /* per-wave partial: reduce l over the 4 lane groups; O hi + lo columns */
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
#pragma unroll
    for (int dt = 0; dt < 16; dt++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float o = acc[dt][i] + __shfl_xor(acc[dt][i], 8);
            if (!is_lo) sO[w][hq][16 * dt + 4 * grp + i] = o;
        }
    }
    if (lane < G) {
        sM[w][lane] = m_run;
        sL[w][lane] = l_run;
    }
    if (last && w == 1) {
        /* the new token's score for the 8 heads, fp32 dot products */
        const float4 kn = *reinterpret_cast<const float4 *>(&sKn[lane * 4]);
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
            const float4 q = *reinterpret_cast<const float4 *>(&sQ[hh][lane * 4]);
            float d = q.x * kn.x + q.y * kn.y + q.z * kn.z + q.w * kn.w;
            d = q35_wave_sum(d);
            if (lane == hh) {
                sM[NW][hh] = d * SCALE;
                sL[NW][hh] = 1.0f;
            }
        }
    }
    __syncthreads();

    /* merge the waves (and the new token) of this workgroup */
    const int nsrc = last ? NW + 1 : NW;
    float *po = p.part_o + ((size_t)(g * p.n_chunks + c) * G) * D;
    float *pml = p.part_ml + ((size_t)(g * p.n_chunks + c) * G) * 2;
    for (int e = t; e < G * D; e += NT) {
        const int hh = e / D, d = e % D;
        float M = -INFINITY;
        for (int s2 = 0; s2 < nsrc; s2++) M = fmaxf(M, sM[s2][hh]);
        float o = 0.0f, L = 0.0f;
        for (int s2 = 0; s2 < nsrc; s2++) {
            const float f = (sM[s2][hh] == -INFINITY) ? 0.0f : expf(sM[s2][hh] - M);
            const float src = (s2 < NW) ? sO[s2][hh][d] : sVn[d];
            o += src * f;
            L += sL[s2][hh] * f;
        }
        po[e] = o;
        if (d == 0) {
            pml[hh * 2] = M;
            pml[hh * 2 + 1] = L;
        }
    }
}

/* merge: grid (heads, D/64), 256 threads = 4 chunk groups x 64 dims */
__global__ __launch_bounds__(256) void gqa_merge_kernel(Q35GqaDecode p) {
    const int h = blockIdx.x, g = h / G, hh = h % G;
    const int t = threadIdx.x, cg = t >> 6, d = blockIdx.y * 64 + (t & 63);
    __shared__ float sM[4], sL[4], sO[4][64];
    const float *pml = p.part_ml + ((size_t)g * p.n_chunks * G + hh) * 2;
    const float *po = p.part_o + ((size_t)g * p.n_chunks * G + hh) * D + d;

    float M = -INFINITY;
    for (int c = cg; c < p.n_chunks; c += 4) M = fmaxf(M, pml[(size_t)c * G * 2]);
    M = fmaxf(M, __shfl_xor(M, 1));   /* uniform within the group already */
    if ((t & 63) == 0) sM[cg] = M;
    __syncthreads();
    M = fmaxf(fmaxf(sM[0], sM[1]), fmaxf(sM[2], sM[3]));
    float o = 0.0f, L = 0.0f;
    for (int c = cg; c < p.n_chunks; c += 4) {
        const float mc = pml[(size_t)c * G * 2];
        const float f = (mc == -INFINITY) ? 0.0f : expf(mc - M);
        L += pml[(size_t)c * G * 2 + 1] * f;
        o += po[(size_t)c * G * D] * f;
    }
    __syncthreads();
    if ((t & 63) == 0) sL[cg] = L;
    sO[cg][t & 63] = o;
    __syncthreads();
    if (cg == 0) {
        const float Lt = (sL[0] + sL[1]) + (sL[2] + sL[3]);
        const float ot = (sO[0][t] + sO[1][t]) + (sO[2][t] + sO[3][t]);
        const float gate = p.q_gate[(size_t)h * 2 * D + D + d];
        p.attn_out[(size_t)h * D + d] = (ot / Lt) * q35_sigmoid(gate);
    }
}

}  // namespace

extern "C" void q35_gqa_split(int n_past, int *chunk, int *n_chunks) {
    int per = (n_past + MAX_CHUNKS - 1) / MAX_CHUNKS;
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
    if (p->ev_begin) {
        hipError_t e0 = hipEventRecord(p->ev_begin, stream);
        if (e0 != hipSuccess) return e0;
    }
    hipLaunchKernelGGL(gqa_split_kernel, dim3(p->n_chunks, p->kv_heads), dim3(NT), 0, stream, *p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p->ev_end) {
        e = hipEventRecord(p->ev_end, stream);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(gqa_merge_kernel, dim3(p->heads, D / 64), dim3(256), 0, stream, *p);
    return hipGetLastError();
}
