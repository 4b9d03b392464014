/*
 * mlx4_gemm.hip -- the batched MLX 4-bit projections of a prefill chunk on
 * gfx950 MFMA: Y[M tokens][N] = X[M][K] W^T for the [N x K] affine 4-bit
 * weight of src/kernels.c:104-219, the GEMM form of ds4f_mlx4_matvec_batch
 * (src/kernels.c:581-619) that ds4f_attn_gqa_chunk / ds4f_attn_linear_chunk
 * call on their B normed token rows (src/attn_qwen.c:1199-1221).
 *
 * Exactness.  With w = q s + b (q in 0..15, s and b the BF16 scale and
 * bias of the 64-element group), and G the groups along K,
 *     y[m][n] = sum_g s[n,g] sum_{k in g} (1024 + q) x  +  b'[n,g] xsum[m,g],
 *     b' = b - 1024 s,  xsum[m,g] = sum_{k in g} x.
 * 1024 + q is exact in fp16, x is carried as an fp16 hi + lo pair (about
 * 22 bits), each MFMA product is exact in fp32, and the group partial is
 * scaled by s in fp32 after its 8 MFMAs (4 k-steps x hi / lo); xsum is the
 * sum of the same hi + lo values, so the 1024 terms cancel to fp32
 * rounding.  The result differs from the reference's fp32 dot products by
 * fp32 rounding of the group sums.
 *
 * Layouts (written by xprep_kernel):
 *   xh, xl  fp16 [Mpad][K]: 8 consecutive k (one nibble word's worth) kept
 *           in the order 0,4,1,5,2,6,3,7, the order in which a word's
 *           nibbles become fp16 pairs ((w >> 4j) & 0x000F000F | 0x64006400
 *           gives 1024 + q_j and 1024 + q_{j+4});
 *   xsum    fp32 [G][Mpad].
 * In a group (8 words), MFMA k-step ks of lane half h is word 4h + ks: a
 * lane's weight operand for a whole group is one 16-byte load.
 *
 * gemm_kernel: 256 threads, a 64-token x 256-feature tile; wave w owns
 * features 64w..64w+63 as 2 x 2 blocks of v_mfma_f32_32x32x16_f16 (A = X
 * from LDS, B = W^T converted in registers).  X tiles of one group (hi, lo,
 * xsum) are staged through LDS, double-buffered, the next group's X and
 * weights in registers meanwhile.
 */
#include "q35_device.h"
#include "q35_launch.h"

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;

namespace {

constexpr int NT = 256;
constexpr int MT = 64;                 /* tokens a tile */
constexpr int NTILE = 256;             /* features a tile, 64 a wave */
constexpr int XROW = 144;              /* LDS bytes of one token row of a group: 128 + 16 pad */
constexpr float OFFSET = 1024.0f;      /* fp16 0x6400 */

/* the word's order of k inside a group: slot j of word v holds k = 8v + PERM[j] */
__device__ __forceinline__ int perm8(int j) { return (j >> 1) + 4 * (j & 1); }

/* x rows -> (optional RMSNorm) -> fp16 hi / lo in word order, and the
 * group sums of hi + lo.  One workgroup per token row (rows >= M: zeros);
 * thread t takes words t, t + 256, ... of the row. */
__global__ __launch_bounds__(NT) void xprep_kernel(Q35Mlx4Xprep p) {
    const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const int nw = p.K / 8;
    const bool live = m < p.M;
    const float *x = p.x + (size_t)m * p.ldx;
    __shared__ double sred[NT / 64];

    float r = 1.0f;
    if (p.norm_w) {
        double ss = 0.0;
        for (int v = t; v < nw; v += NT) {
            if (!live) break;
            const float4 a = *reinterpret_cast<const float4 *>(x + 8 * v);
            const float4 b = *reinterpret_cast<const float4 *>(x + 8 * v + 4);
            const float e[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 8; j++) ss += (double)e[j] * e[j];
        }
        ss = q35_wave_sum(ss);
        if (lane == 0) sred[t >> 6] = ss;
        q35_lds_barrier();
        ss = (sred[0] + sred[1]) + (sred[2] + sred[3]);
        r = sqrtf((float)(ss / (double)p.K) + 1e-6f);
    }
    for (int v = t; v < nw; v += NT) {
        float e[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (live) {
            const float4 a = *reinterpret_cast<const float4 *>(x + 8 * v);
            const float4 b = *reinterpret_cast<const float4 *>(x + 8 * v + 4);
            e[0] = a.x, e[1] = a.y, e[2] = a.z, e[3] = a.w;
            e[4] = b.x, e[5] = b.y, e[6] = b.z, e[7] = b.w;
            if (p.norm_w) {
                const uint4 wb = *reinterpret_cast<const uint4 *>(p.norm_w + 8 * v);
                const uint32_t ww[4] = {wb.x, wb.y, wb.z, wb.w};
#pragma unroll
                for (int j = 0; j < 8; j++)
                    e[j] = e[j] / r * q35_bf2f((uint16_t)(ww[j >> 1] >> (16 * (j & 1))));
            }
        }
        f16x8_t hi, lo;
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v8 = e[perm8(j)];
            const _Float16 h = (_Float16)v8;
            const _Float16 l = (_Float16)(v8 - (float)h);
            hi[j] = h;
            lo[j] = l;
            s += (float)h + (float)l;
        }
        *reinterpret_cast<f16x8_t *>(p.xh + (size_t)m * p.K + 8 * v) = hi;
        *reinterpret_cast<f16x8_t *>(p.xl + (size_t)m * p.K + 8 * v) = lo;
        /* the group's 8 words are 8 consecutive threads of a wave */
        s = q35_sum8(s);
        if ((v & 7) == 0) p.xsum[(size_t)(v >> 3) * p.Mpad + m] = s;
    }
}

/* (s, b - 1024 s) per (row, group) of a weight, from its BF16 scales and
 * biases (biases may be NULL) */
__global__ void sb_kernel(const uint16_t *scales, const uint16_t *biases, Q35Mlx4SB *sb, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float s = q35_bf2f(scales[i]);
    const float b = biases ? q35_bf2f(biases[i]) : 0.0f;
    sb[i] = Q35Mlx4SB{s, b - OFFSET * s};
}

/* a word's 8 nibbles as the fp16 B operand 1024 + q, in word order */
__device__ __forceinline__ f16x8_t nib_f16(uint32_t w) {
    u32x4_t u;
#pragma unroll
    for (int j = 0; j < 4; j++) u[j] = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
    return __builtin_bit_cast(f16x8_t, u);
}

__global__ __launch_bounds__(NT, 2) void gemm_kernel(Q35Mlx4Gemm p) {
    const Q35Mlx4GemmJob J = p.jobs[blockIdx.z];
    float *const Y = p.y[blockIdx.z];
    const int ldy = p.ldy[blockIdx.z];
    const int n0 = blockIdx.x * NTILE, m0 = blockIdx.y * MT;
    if (n0 >= J.N) return;                       /* a narrower job of the launch */
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int h = lane >> 5, c = lane & 31;
    const int G = p.K / 64;

    __shared__ __align__(16) uint8_t sx[2][2][MT * XROW];   /* [buffer][hi, lo] */
    __shared__ __align__(16) float sxs[2][MT];

    /* weights: lane's rows n = n0 + 64w + 32nb + c, range-checked (rows past N
     * read zero); group g of row n is 8 words at n * K / 8 + 8g, the lane's
     * 4 at + 4h */
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint32_t *>(J.vals)), 0, (int)((size_t)J.N * p.K / 2), Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<Q35Mlx4SB *>(J.sb)), 0, (int)((size_t)J.N * G * 8), Q35_BUF_DW3);
    int nrow[2];
#pragma unroll
    for (int nb = 0; nb < 2; nb++) nrow[nb] = n0 + 64 * w + 32 * nb + c;
    auto load_w = [&](int g, u32x4_t (&wq)[2], uint32_t (&sbv)[2][2]) {
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
            const int n = nrow[nb] < J.N ? nrow[nb] : J.N;      /* J.N: past the buffer */
            wq[nb] = __builtin_amdgcn_raw_buffer_load_b128(wr, ((n * (p.K / 8) + 8 * g + 4 * h) * 4), 0, 0);
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(sr, (n * G + g) * 8, 0, 0);
            sbv[nb][0] = v[0];
            sbv[nb][1] = v[1];
        }
    };
    /* X of a group: thread t moves 32 bytes of hi and of lo of token row t / 4 */
    const int xr = t >> 2, xq = t & 3;
    const __amdgpu_buffer_rsrc_t xhr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(p.xh)), 0, (int)((size_t)p.Mpad * p.K * 2), Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t xlr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(p.xl)), 0, (int)((size_t)p.Mpad * p.K * 2), Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t xsr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<float *>(p.xsum)), 0, (int)((size_t)G * p.Mpad * 4), Q35_BUF_DW3);
    const int xoff = ((m0 + xr) * p.K) * 2 + xq * 32;
    auto load_x = [&](int g, u32x4_t (&xv)[4], uint32_t &xs) {
        xv[0] = __builtin_amdgcn_raw_buffer_load_b128(xhr, xoff + g * 128, 0, 0);
        xv[1] = __builtin_amdgcn_raw_buffer_load_b128(xhr, xoff + g * 128 + 16, 0, 0);
        xv[2] = __builtin_amdgcn_raw_buffer_load_b128(xlr, xoff + g * 128, 0, 0);
        xv[3] = __builtin_amdgcn_raw_buffer_load_b128(xlr, xoff + g * 128 + 16, 0, 0);
        xs = __builtin_amdgcn_raw_buffer_load_b32(xsr, (g * p.Mpad + m0 + (t & 63)) * 4, 0, 0);
    };
    auto store_x = [&](int buf, const u32x4_t (&xv)[4], uint32_t xs) {
        uint8_t *hb = &sx[buf][0][xr * XROW + xq * 32];
        uint8_t *lb = &sx[buf][1][xr * XROW + xq * 32];
        *reinterpret_cast<u32x4_t *>(hb) = xv[0];
        *reinterpret_cast<u32x4_t *>(hb + 16) = xv[1];
        *reinterpret_cast<u32x4_t *>(lb) = xv[2];
        *reinterpret_cast<u32x4_t *>(lb + 16) = xv[3];
        if (t < MT) sxs[buf][t] = __uint_as_float(xs);
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int mb = 0; mb < 2; mb++)
#pragma unroll
        for (int nb = 0; nb < 2; nb++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[mb][nb][i] = 0.0f;

    u32x4_t wq[2], xv[4];
    uint32_t sbv[2][2], xs;
    load_w(0, wq, sbv);
    load_x(0, xv, xs);
    store_x(0, xv, xs);
    q35_lds_barrier();

    for (int g = 0; g < G; g++) {
        const int buf = g & 1;
        /* this group's operands in registers, the next group's requested */
        f16x8_t bf[2][4];
        float sc[2], bp[2];
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) bf[nb][ks] = nib_f16(wq[nb][ks]);
            sc[nb] = __uint_as_float(sbv[nb][0]);
            bp[nb] = __uint_as_float(sbv[nb][1]);
        }
        const int gn = g + 1 < G ? g + 1 : g;
        load_w(gn, wq, sbv);
        load_x(gn, xv, xs);

        f32x16_t tmp[2][2];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            f16x8_t ah[2], al[2];
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const int off = (32 * mb + c) * XROW + (4 * h + ks) * 16;
                ah[mb] = *reinterpret_cast<const f16x8_t *>(&sx[buf][0][off]);
                al[mb] = *reinterpret_cast<const f16x8_t *>(&sx[buf][1][off]);
            }
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int nb = 0; nb < 2; nb++) {
                    if (ks == 0) {
                        f32x16_t z;
#pragma unroll
                        for (int i = 0; i < 16; i++) z[i] = 0.0f;
                        tmp[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mb], bf[nb][ks], z, 0, 0, 0);
                    } else {
                        tmp[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mb], bf[nb][ks], tmp[mb][nb], 0, 0, 0);
                    }
                    tmp[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[mb], bf[nb][ks], tmp[mb][nb], 0, 0, 0);
                }
        }
        /* acc += s * partial + b' * xsum; lane rows 32mb + 8(i/4) + 4h + i%4 */
#pragma unroll
        for (int mb = 0; mb < 2; mb++) {
            float xsv[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 v = *reinterpret_cast<const float4 *>(&sxs[buf][32 * mb + 8 * q + 4 * h]);
                xsv[4 * q] = v.x, xsv[4 * q + 1] = v.y, xsv[4 * q + 2] = v.z, xsv[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int nb = 0; nb < 2; nb++)
#pragma unroll
                for (int i = 0; i < 16; i++)
                    acc[mb][nb][i] = fmaf(sc[nb], tmp[mb][nb][i], fmaf(bp[nb], xsv[i], acc[mb][nb][i]));
        }
        /* the next group's X into the other buffer (its last readers passed
         * the previous barrier) */
        store_x(buf ^ 1, xv, xs);
        q35_lds_barrier();
    }

    /* y[m][n] (+= with accumulate): lanes 0..31 of a row write 32
     * consecutive features */
#pragma unroll
    for (int mb = 0; mb < 2; mb++)
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
            const int n = nrow[nb];
            if (n >= J.N) continue;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = m0 + 32 * mb + 8 * (i >> 2) + 4 * h + (i & 3);
                if (m < p.M) {
                    float *dst = Y + (size_t)m * ldy + n;
                    *dst = p.accumulate ? *dst + acc[mb][nb][i] : acc[mb][nb][i];
                }
            }
        }
}

}  // namespace

extern "C" hipError_t q35_mlx4_sb(const uint16_t *scales, const uint16_t *biases, Q35Mlx4SB *sb, int64_t n,
                                  hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(sb_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, scales, biases, sb,
                       n);
    return hipGetLastError();
}

extern "C" hipError_t q35_mlx4_xprep(const Q35Mlx4Xprep *p, hipStream_t stream) {
    if (p->K % 64 != 0 || p->K > 8192 || p->Mpad % MT != 0 || p->M > p->Mpad || p->M < 1)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(xprep_kernel, dim3(p->Mpad), dim3(NT), 0, stream, *p);
    return hipGetLastError();
}

extern "C" hipError_t q35_mlx4_gemm(const Q35Mlx4Gemm *p, int njobs, int max_n, hipStream_t stream) {
    if (p->K % 64 != 0 || p->Mpad % MT != 0 || p->M > p->Mpad || njobs < 1 ||
        njobs > Q35_GEMM_MAX_JOBS || max_n < 1 ||
        (int64_t)max_n * p->K / 2 >= ((int64_t)1 << 31) || (int64_t)p->Mpad * p->K * 2 >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((max_n + NTILE - 1) / NTILE), (unsigned)(p->Mpad / MT), (unsigned)njobs);
    hipLaunchKernelGGL(gemm_kernel, grid, dim3(NT), 0, stream, *p);
    return hipGetLastError();
}

extern "C" int q35_mlx4_gemm_mtile(void) { return MT; }
