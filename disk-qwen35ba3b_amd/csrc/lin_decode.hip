/*
 * lin_decode.hip -- one decode token of a gated delta-rule layer on gfx950.
 *
 * Replaces lin_body's per-token work (src/attn_qwen.c:470-764): causal
 * depthwise conv1d (k = 4) + SiLU over the ring, q/k RMS-normalisation,
 * decay / beta gates, the gated delta rule on the 128x128 fp32 state of
 * every value head, and the RMSNormGated epilogue.
 *
 * One workgroup owns one value head: 1024 threads, 16 waves; wave w holds
 * value columns 8w..8w+7 of the value-major state (4 KiB, contiguous).  Its
 * u-th 16-byte load and store cover kilobyte u of that range: lane l holds
 * column 8w + 2u + (l >> 5), key rows 4(l & 31)..+3, so each instruction
 * moves 1 KiB of whole cache lines (a column-per-8-lanes layout would have
 * each instruction touch 32 lines partially, four times the requests).  The
 * state is the dominant traffic (64 KiB read and 64 KiB written per head);
 * the per-column sums over key rows are 32-lane reductions.  The state loads
 * are issued after the prologue's few loads (returns are counted in order,
 * so the conv does not wait for the state) and before its arithmetic.
 * Owning a whole head keeps the RMSNormGated reduction (over all 128 value
 * columns) inside the workgroup, so the layer is one launch with no
 * cross-workgroup handshake: splitting a head over workgroups would need an
 * agent-scope release / acquire per head, which costs more on this GPU than
 * the per-CU state traffic it spreads.  Inside the workgroup, each norm is
 * one wave's sum: waves 0 / 1 / 2 convolve the head's q / k / v channels, two
 * a lane (so the q and k norms need no cross-wave step), and wave 3 computes
 * the gates and, at the end, the gated norm of all 128 outputs; the kernel
 * has two barriers (conv results to the delta rule, outputs to the norm).
 *
 * Arithmetic: fp32 with FMA in the state update (the reference sums i in
 * ascending order without FMA; the difference is fp32 rounding).  The
 * gates keep the reference's operation order (their decay error would
 * compound over the state's lifetime).  The SiLU and the output gate's
 * sigmoid use the hardware exp / reciprocal, and the three RMS norms an
 * fp32 square sum times the hardware reciprocal square root (about 1 ulp
 * each against the reference's double sums and IEEE divisions): the gated
 * norm is the kernel's tail and the conv the head of its dependent chain.
 */
#include "q35_device.h"
#include "q35_launch.h"

namespace {

constexpr int KD = 128, VD = 128, NT = 1024;

/* The arguments are scalars, not the struct, so that the first nine (14
 * dwords: everything the conv inputs and the state loads need) are
 * preloaded into SGPRs at wave launch (-amdgpu-kernarg-preload-count=9 for
 * this file): the kernel's first global loads wait for no argument load. */
__global__ __launch_bounds__(NT) void lin_decode_kernel(int token, int rows, int k_heads, int v_heads,
                                                        const float *qkv, float *ring,
                                                        const uint16_t *conv_w, float *state,
                                                        const float *a, const float *b,
                                                        const float *A_log, const uint16_t *dt_bias,
                                                        const float *z, const uint16_t *norm_w, float *out,
                                                        float *qkv_post) {
    Q35LinDecode p;
    p.token = token, p.k_heads = k_heads, p.v_heads = v_heads;
    p.qkv = qkv, p.ring = ring, p.conv_w = conv_w, p.state = state, p.a = a, p.b = b;
    p.A_log = A_log, p.dt_bias = dt_bias, p.z = z, p.norm_w = norm_w, p.out = out, p.qkv_post = qkv_post;
    const int h = blockIdx.x;      /* value head */
    const int kh = h >> 1;         /* its key head (src/attn_qwen.c:658) */
    const int t = threadIdx.x;
    const int tok = p.token;

    /* ---- every global input in flight at once ---- */
    /* state: wave w's columns 8w..8w+7; load u is kilobyte u of them */
    const int w = t >> 6, l = t & 63, half = l >> 5, r0 = 4 * (l & 31);
    float4 *sp = reinterpret_cast<float4 *>(p.state + ((size_t)h * VD + 8 * w) * KD) + l;
    float4 s[4];
    /* conv inputs: wave 0 the head's q channels, wave 1 its k channels,
     * wave 2 its v channels, two adjacent channels a lane, so that each
     * q / k norm is a sum over one wave */
    const int kind = w < 3 ? w : -1;
    int ch = 0;
    if (kind == 0)
        ch = kh * KD + 2 * l;
    else if (kind == 1)
        ch = p.k_heads * KD + kh * KD + 2 * l;
    else if (kind == 2)
        ch = 2 * p.k_heads * KD + h * VD + 2 * l;
    float2 xin[4];
    uint4 wv = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int k = 0; k < 4; k++) xin[k] = make_float2(0.f, 0.f);
    if (kind >= 0) {
#pragma unroll
        for (int k = 0; k < 3; k++)
            if (tok - 3 + k >= 0)
                xin[k] = *reinterpret_cast<const float2 *>(p.ring + (size_t)((tok - 3 + k) & 3) * rows + ch);
        xin[3] = *reinterpret_cast<const float2 *>(p.qkv + ch);
        wv = *reinterpret_cast<const uint4 *>(p.conv_w + (size_t)ch * 4);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) s[u] = sp[64 * u];
    /* the gated norm's inputs: wave 3 owns the head's 128 outputs, 2 a lane */
    float2 zv = make_float2(0.f, 0.f);
    uint32_t nw = 0;
    if (w == 3) {
        zv = *reinterpret_cast<const float2 *>(p.z + h * VD + 2 * l);
        nw = *reinterpret_cast<const uint32_t *>(p.norm_w + 2 * l);
    }
    /* the head's gate inputs, at addresses uniform over the workgroup: read
     * by every thread as scalar loads, which the vector-load waits do not
     * cover (dt_bias as the 4-byte-aligned word that holds it: the scalar
     * unit reads whole dwords).  Loaded in the gate lane's branch, dt_bias
     * was a vector load whose bf16 conversion the compiler placed in the
     * branch, so wave 3 waited for all of its loads before requesting its
     * state, one memory round trip late. */
    const float ga = p.a[h], gb = p.b[h], gal = p.A_log[h];
    const int dt_hi = (int)((reinterpret_cast<uintptr_t>(p.dt_bias + h) >> 1) & 1);
    const uint16_t gdt = (uint16_t)(*reinterpret_cast<const uint32_t *>(p.dt_bias + h - dt_hi) >> (16 * dt_hi));
    __shared__ float sq[KD], sk[KD], sv[VD], so[VD];
    __shared__ float sgate[2];

    /* ---- prologue: conv + SiLU, ring update, q/k norms, gates ---- */
    if (kind >= 0) {
        const float xa[4] = {xin[0].x, xin[1].x, xin[2].x, xin[3].x};
        const float xb[4] = {xin[0].y, xin[1].y, xin[2].y, xin[3].y};
        const float ya = q35_conv_silu_fast(xa, make_uint2(wv.x, wv.y), tok);
        const float yb = q35_conv_silu_fast(xb, make_uint2(wv.z, wv.w), tok);
        /* ring slot token%4 takes the raw row; q/k channels are shared by
         * the two value heads of a key head, the even one writes them */
        if (kind == 2 || (h & 1) == 0)
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, xin[3]),
                __builtin_amdgcn_make_buffer_rsrc(q35_uniform_ptr(p.ring), 0, 4 * rows * 4, Q35_BUF_DW3),
                ((tok & 3) * rows + ch) * 4, 0, Q35_ST_SC1);
        float2 y = make_float2(ya, yb);
        if (kind < 2) {
            const float ri = __builtin_amdgcn_rsqf(q35_wave_sum(ya * ya + yb * yb) * (1.0f / KD) + 1e-6f);
            if (kind == 0) {
                y.x = ya * ri * (1.0f / (float)KD);
                y.y = yb * ri * (1.0f / (float)KD);
                *reinterpret_cast<float2 *>(&sq[2 * l]) = y;
            } else {
                y.x = ya * ri * (1.0f / sqrtf((float)KD));
                y.y = yb * ri * (1.0f / sqrtf((float)KD));
                *reinterpret_cast<float2 *>(&sk[2 * l]) = y;
            }
            if (p.qkv_post && (h & 1) == 0) *reinterpret_cast<float2 *>(p.qkv_post + ch) = y;
        } else {
            *reinterpret_cast<float2 *>(&sv[2 * l]) = y;
            if (p.qkv_post) *reinterpret_cast<float2 *>(p.qkv_post + ch) = y;
        }
    }
    if (t == 3 * 64) {
        float g, beta;
        q35_lin_gates(ga, gb, gal, gdt, &g, &beta);
        sgate[0] = expf(g);
        sgate[1] = beta;
    }
    q35_lds_barrier();

    /* ---- gated delta rule (src/attn_qwen.c:666-690), four columns per lane ---- */
    const float dec = sgate[0], beta = sgate[1];
    const float4 kk = *reinterpret_cast<const float4 *>(sk + r0);
    const float4 qq = *reinterpret_cast<const float4 *>(sq + r0);
    float mem[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        s[u].x *= dec; s[u].y *= dec; s[u].z *= dec; s[u].w *= dec;
        float m = s[u].x * kk.x;
        m = fmaf(s[u].y, kk.y, m);
        m = fmaf(s[u].z, kk.z, m);
        m = fmaf(s[u].w, kk.w, m);
        mem[u] = m;
    }
#pragma unroll
    for (int u = 0; u < 4; u++) mem[u] = q35_half_sum(mem[u]);   /* the column's 32 lanes */
    float o[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const float delta = (sv[8 * w + 2 * u + half] - mem[u]) * beta;
        s[u].x = fmaf(kk.x, delta, s[u].x);
        s[u].y = fmaf(kk.y, delta, s[u].y);
        s[u].z = fmaf(kk.z, delta, s[u].z);
        s[u].w = fmaf(kk.w, delta, s[u].w);
        float a = s[u].x * qq.x;
        a = fmaf(s[u].y, qq.y, a);
        a = fmaf(s[u].z, qq.z, a);
        a = fmaf(s[u].w, qq.w, a);
        o[u] = a;
    }
    {
        const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
            q35_uniform_ptr(p.state + (size_t)h * VD * KD), 0, VD * KD * 4, Q35_BUF_DW3);
#pragma unroll
        for (int u = 0; u < 4; u++)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, s[u]), srs,
                                                   ((8 * w * KD) + 4 * (l + 64 * u)) * 4, 0, Q35_ST_SC1);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) o[u] = q35_half_sum(o[u]);
    if ((l & 31) == 0) {
#pragma unroll
        for (int u = 0; u < 4; u++) so[8 * w + 2 * u + half] = o[u];
    }
    q35_lds_barrier();

    /* ---- RMSNormGated over the head's 128 outputs (src/attn_qwen.c:726-749),
     * wave 3, two outputs a lane ---- */
    if (w == 3) {
        const float2 ov = *reinterpret_cast<const float2 *>(&so[2 * l]);
        const float ri = __builtin_amdgcn_rsqf(q35_wave_sum(ov.x * ov.x + ov.y * ov.y) * (1.0f / VD) + 1e-6f);
        float2 y;
        y.x = ov.x * ri * (zv.x * q35_sigmoid_fast(zv.x) * q35_bf2f((uint16_t)(nw & 0xffff)));
        y.y = ov.y * ri * (zv.y * q35_sigmoid_fast(zv.y) * q35_bf2f((uint16_t)(nw >> 16)));
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, y),
            __builtin_amdgcn_make_buffer_rsrc(q35_uniform_ptr(p.out), 0, p.v_heads * VD * 4, Q35_BUF_DW3),
            (h * VD + 2 * l) * 4, 0, Q35_ST_SC1);
    }
}

}  // namespace

extern "C" hipError_t q35_lin_decode(const Q35LinDecode *p, hipStream_t stream) {
    hipLaunchKernelGGL(lin_decode_kernel, dim3(p->v_heads), dim3(NT), 0, stream, p->token,
                       2 * p->k_heads * KD + p->v_heads * VD, p->k_heads, p->v_heads, p->qkv, p->ring,
                       p->conv_w, p->state, p->a, p->b, p->A_log, p->dt_bias, p->z, p->norm_w, p->out,
                       p->qkv_post);
    return hipGetLastError();
}
