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
 * the per-CU state traffic it spreads.
 *
 * Arithmetic: fp32 with FMA in the state update (the reference sums i in
 * ascending order without FMA; the difference is fp32 rounding).  The
 * conv, norms and gates keep the reference's operation order.
 */
#include "q35_device.h"
#include "q35_launch.h"

namespace {

constexpr int KD = 128, VD = 128, NT = 1024;

__global__ __launch_bounds__(NT) void lin_decode_kernel(Q35LinDecode p) {
    const int h = blockIdx.x;      /* value head */
    const int kh = h >> 1;         /* its key head (src/attn_qwen.c:658) */
    const int t = threadIdx.x;
    const int rows = 2 * p.k_heads * KD + p.v_heads * VD;
    const int tok = p.token;

    /* ---- every global input in flight at once ---- */
    /* state: wave w's columns 8w..8w+7; load u is kilobyte u of them */
    const int w = t >> 6, l = t & 63, half = l >> 5, r0 = 4 * (l & 31);
    float4 *sp = reinterpret_cast<float4 *>(p.state + ((size_t)h * VD + 8 * w) * KD) + l;
    float4 s[4];
    /* conv inputs of this head's q (t<128), k (t<256), v (t<384) channels */
    int ch = -1, kind = -1;
    if (t < KD) {
        ch = kh * KD + t;
        kind = 0;
    } else if (t < 2 * KD) {
        ch = p.k_heads * KD + kh * KD + (t - KD);
        kind = 1;
    } else if (t < 2 * KD + VD) {
        ch = 2 * p.k_heads * KD + h * VD + (t - 2 * KD);
        kind = 2;
    }
    float xin[4] = {0.f, 0.f, 0.f, 0.f};
    uint2 wv = make_uint2(0, 0);
    if (ch >= 0) {
#pragma unroll
        for (int k = 0; k < 3; k++)
            if (tok - 3 + k >= 0) xin[k] = p.ring[(size_t)((tok - 3 + k) & 3) * rows + ch];
        xin[3] = p.qkv[ch];
        wv = *reinterpret_cast<const uint2 *>(p.conv_w + (size_t)ch * 4);
    }
    float zv = 0.0f;
    uint16_t nw = 0;
    if (t < VD) {
        zv = p.z[h * VD + t];
        nw = p.norm_w[t];
    }
    float ga = 0.f, gb = 0.f, gal = 0.f;
    uint16_t gdt = 0;
    if (t == 2 * KD + VD) {
        ga = p.a[h];
        gb = p.b[h];
        gal = p.A_log[h];
        gdt = p.dt_bias[h];
    }

#pragma unroll
    for (int u = 0; u < 4; u++) s[u] = sp[64 * u];
    __shared__ float sq[KD], sk[KD], sv[VD], so[VD];
    __shared__ double sred[4];
    __shared__ float sgate[2];

    /* ---- prologue: conv + SiLU, ring update, q/k norms, gates ---- */
    float x = 0.0f;
    if (ch >= 0) {
        x = q35_conv_silu(xin, wv, tok);
        /* ring slot token%4 takes the raw row; q/k channels are shared by
         * the two value heads of a key head, the even one writes them */
        if (kind == 2 || (h & 1) == 0) p.ring[(size_t)(tok & 3) * rows + ch] = xin[3];
    }
    double ss = (kind == 0 || kind == 1) ? (double)x * x : 0.0;
    ss = q35_wave_sum(ss);
    if ((t & 63) == 0 && t < 2 * KD) sred[t >> 6] = ss;
    if (t == 2 * KD + VD) {
        float g, beta;
        q35_lin_gates(ga, gb, gal, gdt, &g, &beta);
        sgate[0] = expf(g);
        sgate[1] = beta;
    }
    q35_lds_barrier();
    if (kind == 0 || kind == 1) {
#pragma clang fp contract(off)
        double tot = kind == 0 ? sred[0] + sred[1] : sred[2] + sred[3];
        float r = sqrtf((float)(tot / (double)KD) + 1e-6f);
        float y;
        if (kind == 0) {
            y = x / r * (1.0f / (float)KD);
            sq[t] = y;
        } else {
            y = x / r * (1.0f / sqrtf((float)KD));
            sk[t - KD] = y;
        }
        if (p.qkv_post && (h & 1) == 0) p.qkv_post[ch] = y;
    } else if (kind == 2) {
        sv[t - 2 * KD] = x;
        if (p.qkv_post) p.qkv_post[ch] = x;
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
#pragma unroll
    for (int u = 0; u < 4; u++) sp[64 * u] = s[u];
#pragma unroll
    for (int u = 0; u < 4; u++) o[u] = q35_half_sum(o[u]);
    if ((l & 31) == 0) {
#pragma unroll
        for (int u = 0; u < 4; u++) so[8 * w + 2 * u + half] = o[u];
    }
    q35_lds_barrier();

    /* ---- RMSNormGated over the head's 128 outputs (src/attn_qwen.c:726-749) ---- */
    if (t < VD) {
        double o2 = (double)so[t] * so[t];
        o2 = q35_wave_sum(o2);
        if ((t & 63) == 0) sred[t >> 6] = o2;
    }
    q35_lds_barrier();
    if (t < VD) {
#pragma clang fp contract(off)
        float r = sqrtf((float)((sred[0] + sred[1]) / (double)VD) + 1e-6f);
        float sg = q35_sigmoid(zv);
        p.out[h * VD + t] = so[t] / r * q35_bf2f(nw) * (zv * sg);
    }
}

}  // namespace

extern "C" hipError_t q35_lin_decode(const Q35LinDecode *p, hipStream_t stream) {
    hipLaunchKernelGGL(lin_decode_kernel, dim3(p->v_heads), dim3(NT), 0, stream, *p);
    return hipGetLastError();
}
