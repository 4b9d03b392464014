/*
 * mlx4.hip -- MLX 4-bit affine matvec on gfx950: y = W x for the
 * [R x C] weight of src/kernels.c:104-219 (ds4f_mlx4_matvec) and its
 * batched form (the routed-expert jobs of ds4f_gpu_mlx4_batch,
 * include/ds4f/gpu.h:29-54).
 *
 * Format: U32 words of 8 nibbles, low nibble first; element k = r*C + c
 * of the flattened matrix is nibble k%8 of word k/8; a BF16 scale and bias
 * per 64 elements (group k/64, which may straddle rows); w = q*scale+bias.
 *
 * One wave per 4 / NCH rows (NCH = 2048-column chunks of x; 1 at 8192), their loads
 * and the next rows' issued together; lane l takes 32 consecutive elements
 * (one 16-byte word load) of each 2048-column chunk.
 * With C % 32 == 0 those 32 elements start 32-aligned in the flattened
 * index, so they lie in one group: the lane computes
 *     scale * sum_e q_e x_e + bias * sum_e x_e
 * with x and its per-lane sums held in registers for every row the wave
 * visits.  The products are fp32 FMAs on the exact nibble values, the
 * sums fp32; the summation order differs from the reference's per-element
 * q*s+b accumulation, a float32 rounding difference (gpu.h:13-18).
 * The row's partial sums meet in a DPP wave reduction.  HBM-bound: R*C/2
 * bytes of nibbles plus R*C/16 bytes of scales and biases per matvec.
 * Fused around it for the attention layer steps: the input RMSNorm of x
 * and the residual add into y.  x is read, normalised and scaled once per
 * workgroup into LDS, from where every wave takes its lanes' columns (a
 * per-wave copy cost each wave 32 divisions a lane and 12 KiB of L2 reads:
 * 11.4 -> 8.6 us for a delta layer's 12352 x 2048 projections).
 */
#include "q35_device.h"
#include "q35_launch.h"

namespace {

constexpr int NT = 256;
constexpr int CHUNK = 2048;            /* columns per 64 lanes x 32 */
constexpr int MAXCH = 4;               /* C <= 8192 */

struct Mlx4Job {
    const uint32_t *vals;
    const uint16_t *scales, *biases;
    const float *x;
    float *y;
    int R;
};

/* 32 nibble products of one lane: 4 words, 8 nibbles each, against x[32].
 * Masking a word with 0x0F0F0F0F leaves one nibble per byte; a byte q < 16
 * read as an fp8 e4m3 number is q * 2^-9 exactly (exponent field 0 or 1,
 * where e4m3 is linear), so v_cvt_pk_f32_fp8 turns two nibbles into two
 * exact floats in one instruction.  x is held pre-multiplied by the
 * inverse of that unit, a power of two, so each product is q * x exactly
 * as with an integer conversion.  Byte b of the low mask is nibble 2b,
 * of the high mask nibble 2b+1. */
__device__ __forceinline__ float nib_dot(u32x4_t w, const float (&x)[32]) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int lo = (int)(w[i] & 0x0F0F0F0Fu), hi = (int)((w[i] >> 4) & 0x0F0F0F0Fu);
        const auto l0 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);   /* nibbles 0, 2 */
        const auto l1 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);    /* nibbles 4, 6 */
        const auto h0 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);   /* nibbles 1, 3 */
        const auto h1 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);    /* nibbles 5, 7 */
        a0 = fmaf(l0[0], x[8 * i + 0], a0);
        a1 = fmaf(h0[0], x[8 * i + 1], a1);
        a0 = fmaf(l0[1], x[8 * i + 2], a0);
        a1 = fmaf(h0[1], x[8 * i + 3], a1);
        a0 = fmaf(l1[0], x[8 * i + 4], a0);
        a1 = fmaf(h1[0], x[8 * i + 5], a1);
        a0 = fmaf(l1[1], x[8 * i + 6], a0);
        a1 = fmaf(h1[1], x[8 * i + 7], a1);
    }
    return a0 + a1;
}

/* rows a wave takes per iteration: 4 2048-column chunks' worth of loads
 * (one row at 8192 columns).  Measured against 8 and 2 on the 40-layer
 * step and the 248320-row head: 4 is faster on both (a layer's 12352
 * projection rows then give 3088 waves, 3 workgroups a CU, instead of
 * 1.5) */
template <int NCH>
constexpr int rows_per_wave() { return NCH >= 4 ? 1 : 4 / NCH; }

/* The arguments are scalars, not the struct, so that the first nine (14
 * dwords: the row count, width, accumulate flag and the x, job table,
 * norm weight, word and scale pointers) are preloaded into SGPRs at launch
 * (-amdgpu-kernarg-preload-count=9 for this file): the job table and x go
 * out with no argument load before them. */
template <int NCH, bool NORM>
__global__ __launch_bounds__(NT) void mlx4_kernel(int R_, int C_, int accumulate, const float *x,
                                                  const Q35Mlx4Job *jobs, const uint16_t *x_norm,
                                                  const uint32_t *vals, const uint16_t *scales,
                                                  const uint16_t *biases, float *y) {
    Q35Mlx4 p;
    p.R = R_, p.C = C_, p.accumulate = accumulate, p.x = x, p.y = y, p.jobs = jobs;
    p.x_norm = x_norm, p.vals = vals, p.scales = scales, p.biases = biases;
    constexpr int RP = rows_per_wave<NCH>();
    Mlx4Job j;
    if (p.jobs) {
        const Q35Mlx4Job &d = p.jobs[blockIdx.y];
        j = {d.vals, d.scales, d.biases, d.x ? d.x : p.x, d.y, d.R ? d.R : p.R};
    } else {
        j = {p.vals, p.scales, p.biases, p.x, p.y, p.R};
    }
    const int R = j.R, C = p.C, lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (NT / 64) + (threadIdx.x >> 6), nwaves = gridDim.x * (NT / 64);
    /* a shorter job of a batch: no rows for this workgroup (uniform, so no
     * wave leaves before the prologue's barriers) */
    if (RP * (NT / 64) * (int)blockIdx.x >= R) return;

    bool live[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) live[ch] = ch * CHUNK + 32 * lane < C;

    /* range-checked views: rows at and past R read zero */
    const size_t nel = (size_t)R * C;
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint32_t *>(j.vals)), 0, (int)(nel / 2), Q35_BUF_DW3);
    const int ng = (int)((nel + 63) / 64);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(j.scales)), 0, 2 * ng, Q35_BUF_DW3);
    const bool has_b = j.biases != nullptr;
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(has_b ? j.biases : j.scales)), 0, has_b ? 2 * ng : 0, Q35_BUF_DW3);

    /* the nibble words, scales and biases of RP rows; rows at and past R
     * (and dead lanes) point past the buffers and read zero, so every load
     * is unconditional.  Nontemporal: a decode step reads each weight once,
     * and streaming them through the cache would evict the delta-rule
     * states and the cache rows the cores read next (40 whole layers at
     * 32768 context: 1249 -> 1329 tokens/s) */
    struct Rows {
        u32x4_t w[RP][NCH];
        uint32_t sc[RP][NCH], bi[RP][NCH];
    };
    auto load_rows = [&](int r0, Rows &q) {
#pragma unroll
        for (int u = 0; u < RP; u++)
#pragma unroll
            for (int ch = 0; ch < NCH; ch++) {
                const int64_t k0 = (int64_t)(r0 + u) * C + ch * CHUNK + 32 * lane;
                const bool in = live[ch] && r0 + u < R;
                const int kk = in ? (int)(k0 >> 3) : (int)(nel / 8);
                const int gg = in ? (int)(k0 >> 6) : ng;
                q.w[u][ch] = __builtin_amdgcn_raw_buffer_load_b128(vr, 4 * kk, 0, 2);
                q.sc[u][ch] = __builtin_amdgcn_raw_buffer_load_b16(sr, 2 * gg, 0, 2);
                q.bi[u][ch] = __builtin_amdgcn_raw_buffer_load_b16(br, 2 * gg, 0, 2);
            }
    };
    /* x, and with x_norm its RMSNorm, once per workgroup: thread t holds
     * float4s t, t + NT, ... of x (range-checked loads: columns past C read
     * zero), the fp32 square sum meets over the workgroup, and x times
     * rsq(mean + 1e-6) times w (src/attn_qwen.c:142-157 computes the sum in
     * double and divides by the square root: about 1 ulp apart here, and
     * 40 whole layers at 32768 context 1370 -> 1422 tokens/s, the norm being
     * on the projection launch's dependent path).  The result, scaled by the
     * inverse fp8 nibble unit, goes to LDS laid out [chunk][q][lane] (float4 q
     * of lane l's 32 columns), so each lane's reads below are conflict-free
     * 16-byte rows.  Every slot is written, zeros past C. */
    constexpr int XQ = NCH * CHUNK / 4 / NT;
    __shared__ float4 sx[NCH * CHUNK / 4];
    __shared__ float sredf[NT / 64];
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<float *>(j.x)), 0, 4 * C, Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t nrs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(NORM ? p.x_norm : reinterpret_cast<const uint16_t *>(j.x))),
        0, NORM ? 2 * C : 0, Q35_BUF_DW3);
    float xv[XQ][4];
    uint32_t nw[XQ][2];
#pragma unroll
    for (int q = 0; q < XQ; q++) {
        const int c = 4 * ((int)threadIdx.x + NT * q);
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(xrs, 4 * c, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) xv[q][e] = __uint_as_float(v[e]);
        if (NORM) {
            const auto n2 = __builtin_amdgcn_raw_buffer_load_b64(nrs, 2 * c, 0, 0);
            nw[q][0] = n2[0];
            nw[q][1] = n2[1];
        }
    }
    /* the first rows' weights go out right after x: loads return in issue
     * order, so the prologue below waits for x alone and runs while the
     * weights stream in (issued first, they would hold x's wait until the
     * wave's whole weight tile had arrived).  The scheduler barriers keep
     * that order and keep the weight loads above the norm's reduction. */
    __builtin_amdgcn_sched_barrier(0);
    Rows cur;
    load_rows(RP * wave, cur);
    __builtin_amdgcn_sched_barrier(0);
    if (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int q = 0; q < XQ; q++)
#pragma unroll
            for (int e = 0; e < 4; e++) ss = fmaf(xv[q][e], xv[q][e], ss);
        ss = q35_wave_sum(ss);
        if (lane == 0) sredf[threadIdx.x >> 6] = ss;
        q35_lds_barrier();
        float tot = sredf[0];
#pragma unroll
        for (int i = 1; i < NT / 64; i++) tot += sredf[i];
        const float ri = __builtin_amdgcn_rsqf(tot * (1.0f / (float)C) + 1e-6f);
#pragma unroll
        for (int q = 0; q < XQ; q++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float w = q35_bf2f((uint16_t)(nw[q][e >> 1] >> (16 * (e & 1))));
                xv[q][e] = xv[q][e] * ri * w;
            }
    }
    const float unit = __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0], xsc = 1.0f / unit;
#pragma unroll
    for (int q = 0; q < XQ; q++) {
        const int c = 4 * ((int)threadIdx.x + NT * q);
        sx[(c >> 11) * (CHUNK / 4) + ((c & 31) >> 2) * 64 + ((c & (CHUNK - 1)) >> 5)] =
            make_float4(xv[q][0] * xsc, xv[q][1] * xsc, xv[q][2] * xsc, xv[q][3] * xsc);
    }
    q35_lds_barrier();

    /* this lane's 32 columns of each chunk, and their plain sums (the scaled
     * sum times the unit, a power of two: exact) */
    float xr[NCH][32], xs[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) {
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float4 v = sx[ch * (CHUNK / 4) + q * 64 + lane];
            xr[ch][4 * q] = v.x;
            xr[ch][4 * q + 1] = v.y;
            xr[ch][4 * q + 2] = v.z;
            xr[ch][4 * q + 3] = v.w;
            s += (v.x + v.y) + (v.z + v.w);
        }
        xs[ch] = s * unit;
    }

    /* y of the rows for the residual add, lane u < RP holding row r0 + u (a
     * view of length 0 reads zeros when the launch does not accumulate) */
    const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(j.y), 0, p.accumulate ? 4 * R : 0, Q35_BUF_DW3);
    for (int r0 = RP * wave; r0 < R; r0 += RP * nwaves) {
        /* the next rows and these rows' y are requested before these rows
         * are consumed.  A wave's last rows request nothing more: loads past
         * R read zeros without a memory access, but the wave would still wait
         * for them before it retires. */
        const float yv = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(yrs, lane < RP ? 4 * (r0 + lane) : 4 * R, 0, 0));
        const bool more = r0 + RP * nwaves < R;
        Rows nxt;
        if (more) load_rows(r0 + RP * nwaves, nxt);
        float part[RP];
#pragma unroll
        for (int u = 0; u < RP; u++) {
            float acc = 0.0f;
#pragma unroll
            for (int ch = 0; ch < NCH; ch++) {
                const float sc = q35_bf2f((uint16_t)cur.sc[u][ch]);
                const float bi = q35_bf2f((uint16_t)cur.bi[u][ch]);
                acc = fmaf(sc, nib_dot(cur.w[u][ch], xr[ch]), fmaf(bi, xs[ch], acc));
            }
            part[u] = acc;
        }
        /* row u's total lands in every lane; lane u stores it */
        float t = 0.0f;
#pragma unroll
        for (int u = 0; u < RP; u++) {
            const float tu = q35_wave_sum(part[u]);
            t = lane == u ? tu : t;
        }
        if (lane < RP && r0 + lane < R) j.y[r0 + lane] = p.accumulate ? yv + t : t;
        if (more) cur = nxt;
    }
}

template <int NCH>
void launch(const Q35Mlx4 *p, dim3 grid, hipStream_t stream) {
    if (p->x_norm)
        hipLaunchKernelGGL((mlx4_kernel<NCH, true>), grid, dim3(NT), 0, stream, p->R, p->C, p->accumulate,
                           p->x, p->jobs, p->x_norm, p->vals, p->scales, p->biases, p->y);
    else
        hipLaunchKernelGGL((mlx4_kernel<NCH, false>), grid, dim3(NT), 0, stream, p->R, p->C, p->accumulate,
                           p->x, p->jobs, p->x_norm, p->vals, p->scales, p->biases, p->y);
}

}  // namespace

extern "C" int q35_mlx4_supported(int R, int C) {
    return R >= 1 && C >= 32 && C % 32 == 0 && C <= MAXCH * CHUNK &&
           (int64_t)R * C / 2 < ((int64_t)1 << 31);
}

extern "C" hipError_t q35_mlx4_matvec(const Q35Mlx4 *p, int njobs, hipStream_t stream) {
    if (!q35_mlx4_supported(p->R, p->C) || njobs < 1 || (njobs > 1 && !p->jobs))
        return hipErrorInvalidValue;
    /* one wave per group of rows_per_wave rows, grid-strided beyond 2048
     * workgroups */
    const int nch = (p->C + CHUNK - 1) / CHUNK;
    const int rp = nch == 1 ? rows_per_wave<1>() : nch == 2 ? rows_per_wave<2>() : rows_per_wave<4>();
    const int64_t waves = ((int64_t)p->R + rp - 1) / rp;
    int64_t blocks = (waves + NT / 64 - 1) / (NT / 64);
    if (blocks > 2048) blocks = 2048;
    const dim3 grid((unsigned)blocks, (unsigned)njobs);
    if (nch == 1)
        launch<1>(p, grid, stream);
    else if (nch == 2)
        launch<2>(p, grid, stream);
    else
        launch<4>(p, grid, stream);
    return hipGetLastError();
}
