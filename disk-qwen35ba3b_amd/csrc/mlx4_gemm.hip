/*
 * mlx4_gemm.hip -- the batched MLX 4-bit projections of a prefill chunk on
 * gfx950 MFMA: Y[M tokens][N] = X[M][K] W^T for the [N x K] affine 4-bit
 * weight of src/kernels.c:104-219, the GEMM form of ds4f_mlx4_matvec_batch
 * (src/kernels.c:581-619) that ds4f_attn_gqa_chunk / ds4f_attn_linear_chunk
 * call on their B normed token rows (src/attn_qwen.c:1199-1221).
 *
 * Exactness.  With w = q s + b (q in 0..15, s and b the BF16 scale and
 * bias of the 64-element group), and G the groups along K,
 *     y[m][n] = sum_g s'[n,g] sum_{k in g} (1 + q/16) x  +  b'[n,g] xsum[m,g],
 *     s' = 16 s,  b' = b - 16 s,  xsum[m,g] = sum_{k in g} x.
 * 1 + q/16 is exact in fp16 (the nibble in mantissa bits 6..9 under the
 * exponent of 1), x is carried as an fp16 hi + lo pair (about 22 bits),
 * each MFMA product is exact in fp32, and the group partial is scaled by
 * s' in fp32 after its 8 MFMAs (4 k-steps x hi / lo); xsum is the sum of
 * the same hi + lo values.  The offset 1 is at most about twice the q/16
 * part, so the cancellation against b' xsum costs about a bit, and the
 * result differs from the reference's fp32 dot products by fp32 rounding
 * of the group sums.
 *
 * Layouts:
 *   xw      (xprep_kernel) per 64-token tile mt and group g, a 16 KB block
 *           at ((mt G + g) 2 + {0: hi, 1: lo}) 8 KB: 64 rows of 128 bytes,
 *           fp16, 8 consecutive k (one nibble word's worth) kept in the
 *           order 0,4,1,5,2,6,3,7, the order in which a word's nibbles become
 *           fp16 pairs (nibbles j and j + 4 moved to bits 6..9 and 22..25,
 *           ORed into 0x3C003C00, give 1 + q_j / 16 and 1 + q_{j+4} / 16);
 *           word j of row r at 16-byte slot
 *           j ^ (r & 7) ^ ((r >> 3) & 1), so that the MFMA operand reads
 *           (32 rows, one word each) hit distinct LDS banks;
 *   xsum    fp32 [G][Mpad];
 *   sb      (sb_kernel) (16 s, b - 16 s) as [G][Npad], Npad = N rounded up
 *           to 256, zeros past N;
 *   wt      (wt_kernel) the weight words re-laid out once per weight: per
 *           256-feature tile and group an 8 KB block that is the LDS image
 *           of the stage (16-byte position p = row p / 2, half
 *           wslot(row, p % 2)), rows past N zero; staging it is a plain
 *           copy, 1 KB a wave load.
 * In a group (8 words), MFMA k-step ks of lane half h is word 4h + ks: a
 * lane's weight operand for a whole group is one 16-byte read.
 *
 * gemm_kernel: 256 threads, a 64-token x 256-feature tile; wave w owns
 * features 64w..64w+63 as 2 x 2 blocks of v_mfma_f32_32x32x16_f16 (A = X,
 * B = W^T converted in registers).  Every global load is a direct-to-LDS
 * load into a ring of three stages, one group each (X hi and lo 16 KB,
 * the tile's weight words 8 KB, (s, b') 2 KB, xsum 256 B), issued two
 * groups ahead (every stage load a contiguous 1 KB); each wave waits for
 * its own loads of the next group
 * before the one barrier a group.  Two workgroups fit a CU (157.5 KB of
 * LDS), two waves a SIMD.
 */
#include "q35_device.h"
#include "q35_launch.h"

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;

namespace {

constexpr int NT = 256;
constexpr int MT = 64;                 /* tokens a tile */
constexpr int NTILE = 256;             /* features a tile, 64 a wave */
constexpr int XBLK = Q35_XW_BLK;       /* bytes of a tile's hi (or lo) X of one group */
static_assert(MT == Q35_XW_ROWS, "the X tiles are the GEMM's token tiles");
constexpr int WBLK = NTILE * 32;       /* bytes of a tile's weight words of one group */
constexpr int SBLK = NTILE * 8;        /* bytes of a tile's (s, b') of one group */
constexpr int OFF_W = 2 * XBLK, OFF_SB = OFF_W + WBLK, OFF_XS = OFF_SB + SBLK;
constexpr int STAGE = OFF_XS + MT * 4; /* 26880 bytes */
constexpr int NSTAGE = 3;
constexpr float QSTEP = 16.0f;         /* B = 1 + q / QSTEP */

/* q35_xw_slot: the 16-byte slot of word j of tile row r in its 128-byte X
 * row is distinct over any 8 consecutive rows and, with the row's 128-byte
 * half, over any 16: the operand reads are free of bank conflicts whether
 * the LDS serves 8 lanes over 32 banks or 16 lanes over 64 banks a cycle */
/* slot of half h (words 4h..4h+3) of tile feature row r in its 32-byte
 * weight row, by the same argument over 4 and 8 consecutive rows */
__device__ __forceinline__ int wslot(int r, int h) { return h ^ (((r >> 2) ^ (r >> 3)) & 1); }

/* x rows -> (optional RMSNorm) -> fp16 hi / lo in word order, tiled, and
 * the group sums of hi + lo.  One workgroup per token row (rows >= M: zeros);
 * thread t takes words t, t + 256, ... of the row, XW of them: the
 * instance is picked by K (1 at 2048, the input projections; 2 at 4096, the
 * GQA output projection; 4 up to 8192), so no thread issues loads past the
 * row (at K = 2048 an instance for 8192 issued nine dead loads a thread:
 * range-checked, they read no memory, but each is still issued and waited
 * for).  The norm is an fp32
 * square sum times the hardware rsq (about 1 ulp from the reference's double
 * sum and division, src/attn_qwen.c:142-157, far below the hi / lo split's
 * 22 bits). */
template <int XW>
__global__ __launch_bounds__(NT) void xprep_kernel(Q35Mlx4Xprep p) {
    const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const int nw = p.K / 8;
    const bool live = m < p.M;
    __shared__ float sred[NT / 64];

    /* the thread's words of the row and of the norm weight, all requested
     * at once as range-checked buffer loads (rows past M, words past K and
     * an absent norm weight read as zeros): the norm and the conversion
     * then work from registers, one memory round trip a workgroup */
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<float *>(live ? p.x + (size_t)m * p.ldx : p.x)), 0, live ? p.K * 4 : 0,
        Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(p.norm_w)), 0, p.norm_w ? p.K * 2 : 0, Q35_BUF_DW3);
    float4 xa[XW], xb[XW];
    uint4 wv[XW];
#pragma unroll
    for (int i = 0; i < XW; i++) {
        const int v = t + i * NT;
        xa[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xrs, 32 * v, 0, 0));
        xb[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xrs, 32 * v + 16, 0, 0));
        wv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrs, 16 * v, 0, 0));
    }

    float ri = 1.0f;
    if (p.norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XW; i++) {
            const float e[8] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w, xb[i].x, xb[i].y, xb[i].z, xb[i].w};
#pragma unroll
            for (int j = 0; j < 8; j++) ss = fmaf(e[j], e[j], ss);
        }
        ss = q35_wave_sum(ss);
        if (lane == 0) sred[t >> 6] = ss;
        q35_lds_barrier();
        ss = (sred[0] + sred[1]) + (sred[2] + sred[3]);
        ri = __builtin_amdgcn_rsqf(ss * (1.0f / (float)p.K) + 1e-6f);
    }
#pragma unroll
    for (int i = 0; i < XW; i++) {
        const int v = t + i * NT;
        if (v >= nw) break;   /* nw is a multiple of 8: the 8 lanes of a group (q35_sum8) leave together */
        float e[8] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w, xb[i].x, xb[i].y, xb[i].z, xb[i].w};
        if (p.norm_w) {
            const uint32_t ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
            for (int j = 0; j < 8; j++)
                e[j] = e[j] * ri * q35_bf2f((uint16_t)(ww[j >> 1] >> (16 * (j & 1))));
        }
        bool over = false;
#pragma unroll
        for (int j = 0; j < 8; j++) over = over || q35_f16_over(e[j]);
        q35_f16_guard(p.status, Q35_STATUS_GEMM_F16, over);
        f16x8_t hi, lo;
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v8 = e[q35_xw_perm(j)];
            const _Float16 h = (_Float16)v8;
            const _Float16 l = (_Float16)(v8 - (float)h);
            hi[j] = h;
            lo[j] = l;
            s += (float)h + (float)l;
        }
        uint8_t *blk = reinterpret_cast<uint8_t *>(p.xw) + q35_xw_granule(m, v, p.K / 64);
        *reinterpret_cast<f16x8_t *>(blk) = hi;
        *reinterpret_cast<f16x8_t *>(blk + XBLK) = lo;
        /* the group's 8 words are 8 consecutive threads of a wave */
        s = q35_sum8(s);
        if ((v & 7) == 0) p.xsum[(size_t)(v >> 3) * p.Mpad + m] = s;
    }
}

/* (16 s, b - 16 s) of a weight's rows and groups as [G][npad] (zeros for
 * rows past N), from its BF16 scales and biases [N][G] (biases may be
 * NULL) */
__global__ void sb_kernel(const uint16_t *scales, const uint16_t *biases, Q35Mlx4SB *sb, int N, int G,
                          int npad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)G * npad) return;
    const int g = (int)(i / npad), n = (int)(i % npad);
    float sv = 0.0f, bv = 0.0f;
    if (n < N) {
        const float s = q35_bf2f(scales[(size_t)n * G + g]);
        const float b = biases ? q35_bf2f(biases[(size_t)n * G + g]) : 0.0f;
        sv = QSTEP * s;
        bv = b - sv;
    }
    sb[i] = Q35Mlx4SB{sv, bv};
}

/* the weight words [N][K/8] as wt blocks [npad/256][G][512 granules of
 * 16 bytes]: granule p of block (tile, g) = words 4 wslot(r, p % 2) ..
 * +3 of group g of row tile * 256 + r, r = p / 2; zeros past N */
__global__ void wt_kernel(const uint32_t *vals, u32x4_t *wt, int N, int K, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int G = K / 64;
    const int p = (int)(i & 511);
    const int64_t blk = i >> 9;
    const int g = (int)(blk % G), tile = (int)(blk / G);
    const int r = p >> 1, row = tile * NTILE + r;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (row < N)
        v = *reinterpret_cast<const u32x4_t *>(vals + (size_t)row * (K / 8) + 8 * g + 4 * wslot(r, p & 1));
    wt[i] = v;
}

/* a word's 8 nibbles as the fp16 B operand 1 + q / 16, in word order:
 * pair j (nibbles j and j + 4, bits 4j and 16 + 4j) shifted to bits 6 and
 * 22, masked, ORed into the exponent of 1.  The mask and the exponent bits
 * are held in registers (an SGPR and a VGPR) so that each pair is one
 * shift and one v_and_or_b32. */
__device__ __forceinline__ f16x8_t nib_f16(uint32_t w, uint32_t mask, uint32_t one) {
    u32x4_t u;
    u[0] = ((w << 6) & mask) | one;
    u[1] = ((w << 2) & mask) | one;
    u[2] = ((w >> 2) & mask) | one;
    u[3] = ((w >> 6) & mask) | one;
    return __builtin_bit_cast(f16x8_t, u);
}

__device__ __forceinline__ int ntiles(int N) { return (N + NTILE - 1) / NTILE; }

/* One workgroup per (job, 256-feature tile, 64-token tile), numbered with
 * the token tile fastest over the jobs' feature tiles in order.  Work-
 * groups are handed to the 8 XCDs in turn, so with 8 | token tiles an XCD
 * holds token tiles of one residue mod 8 over consecutive feature tiles:
 * about 8 x 8 tiles at once, sharing X and weight tiles in its L2. */
__global__ __launch_bounds__(NT, 2) void gemm_kernel(Q35Mlx4Gemm p) {
    const int ntm = p.Mpad / MT;
    const int mt = blockIdx.x % ntm;
    int nt = blockIdx.x / ntm;
    /* the job of feature tile nt (uniform selects: the job array is kernel
     * arguments, not indexed memory) */
    Q35Mlx4GemmJob J = p.jobs[0];
#pragma unroll
    for (int j = 1; j < Q35_GEMM_MAX_JOBS; j++) {
        const int prev = ntiles(J.N);
        if (j < p.njobs && nt >= prev) {
            nt -= prev;
            J = p.jobs[j];
        }
    }
    float *const Y = J.y;
    const int ldy = J.ldy;
    const int n0 = nt * NTILE, m0 = mt * MT;
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int h = lane >> 5, c = lane & 31;
    const int G = p.K / 64;
    const int npad = (J.N + NTILE - 1) / NTILE * NTILE;

    __shared__ __align__(16) uint8_t smem[NSTAGE * STAGE];
    const uint32_t lds0 = q35_lds_addr(smem);

    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint16_t *>(p.xw)), 0, (int)((size_t)p.Mpad * p.K * 4), Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<uint32_t *>(J.vals)), 0, (int)((size_t)npad * p.K / 2), Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<Q35Mlx4SB *>(J.sb)), 0, (int)((size_t)G * npad * 8), Q35_BUF_DW3);
    const __amdgpu_buffer_rsrc_t ssr = __builtin_amdgcn_make_buffer_rsrc(
        q35_uniform_ptr(const_cast<float *>(p.xsum)), 0, (int)((size_t)G * p.Mpad * 4), Q35_BUF_DW3);

    /* group g into stage st: X 16 loads, weights 8, (s, b') 2, xsum 1 (a
     * dword load); waves 0-2 issue 7 of them, wave 3 issues 6 */
    auto issue = [&](int g, int st) {
        const uint32_t sb = lds0 + (uint32_t)(st * STAGE);
        const uint32_t xb = (uint32_t)(mt * G + g) * (2 * XBLK);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int i = w + 4 * q;
            q35_dma16(xr, sb + i * 1024, lane * 16, xb + i * 1024);
        }
        const uint32_t wb = (uint32_t)(nt * G + g) * WBLK;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int i = w + 4 * q;
            q35_dma16(wr, sb + OFF_W + i * 1024, lane * 16, wb + i * 1024);
        }
        if (w < 2)
            q35_dma16(sr, sb + OFF_SB + w * 1024, lane * 16, (uint32_t)(g * npad + n0) * 8 + w * 1024);
        else if (w == 2)
            q35_dma4(ssr, sb + OFF_XS, lane * 4, (uint32_t)(g * p.Mpad + m0) * 4);
    };
    /* this wave's loads of the group before the last issued have landed */
    auto wait_prev = [&]() {
        if (w == 3)
            q35_wait_vm<6>();
        else
            q35_wait_vm<7>();
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int mb = 0; mb < 2; mb++)
#pragma unroll
        for (int nb = 0; nb < 2; nb++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[mb][nb][i] = 0.0f;

    issue(0, 0);
    if (G > 1) {
        issue(1, 1);
        wait_prev();
    } else {
        q35_wait_vm<0>();
    }
    q35_lds_barrier();

    /* a wave whose 64 features all lie past N (a narrow job) only stages */
    const bool idle = n0 + 64 * w >= J.N;
    uint32_t mask, one;
    asm("s_mov_b32 %0, 0x03c003c0" : "=s"(mask));
    asm("v_mov_b32 %0, 0x3c003c00" : "=v"(one));

    int st = 0;
    for (int g = 0; g < G; g++) {
        if (g + 2 < G) issue(g + 2, st == 0 ? 2 : st - 1);
        if (!idle) {
            const uint8_t *S = smem + st * STAGE;
            /* the weight operand: this lane's words 4h..4h+3 of rows
             * 64w + 32nb + c, and their (s, b') */
            f16x8_t bf[2][4];
            float sc[2], bp[2];
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                const int r = 64 * w + 32 * nb + c;
                const u32x4_t wq = *reinterpret_cast<const u32x4_t *>(S + OFF_W + r * 32 + wslot(r, h) * 16);
#pragma unroll
                for (int ks = 0; ks < 4; ks++) bf[nb][ks] = nib_f16(wq[ks], mask, one);
                const float2 v = *reinterpret_cast<const float2 *>(S + OFF_SB + r * 8);
                sc[nb] = v.x;
                bp[nb] = v.y;
            }

            /* acc += b' * xsum first: it does not wait for the MFMAs, so it
             * runs while the previous wave's MFMAs hold the pipe */
            {
                const float *xs0 = reinterpret_cast<const float *>(S + OFF_XS);
#pragma unroll
                for (int mb = 0; mb < 2; mb++) {
                    float xsv[16];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 v = *reinterpret_cast<const float4 *>(xs0 + 32 * mb + 8 * q + 4 * h);
                        xsv[4 * q] = v.x, xsv[4 * q + 1] = v.y, xsv[4 * q + 2] = v.z, xsv[4 * q + 3] = v.w;
                    }
#pragma unroll
                    for (int nb = 0; nb < 2; nb++)
#pragma unroll
                        for (int i = 0; i < 16; i++) acc[mb][nb][i] = fmaf(bp[nb], xsv[i], acc[mb][nb][i]);
                }
            }
            /* the group's MFMAs at raised wave priority, so that the SIMD's
             * other wave does its VALU work around them rather than
             * competing for the issue slot (output GEMM 126 -> 116 us) */
            __builtin_amdgcn_s_setprio(1);
            f32x16_t tmp[2][2];
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                f16x8_t ah[2], al[2];
#pragma unroll
                for (int mb = 0; mb < 2; mb++) {
                    const int r = 32 * mb + c;
                    const int off = r * 128 + q35_xw_slot(r, 4 * h + ks) * 16;
                    ah[mb] = *reinterpret_cast<const f16x8_t *>(S + off);
                    al[mb] = *reinterpret_cast<const f16x8_t *>(S + XBLK + off);
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
                            tmp[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mb], bf[nb][ks],
                                                                                 tmp[mb][nb], 0, 0, 0);
                        }
                        tmp[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[mb], bf[nb][ks], tmp[mb][nb], 0, 0, 0);
                    }
            }
            __builtin_amdgcn_s_setprio(0);
            /* acc += s' * partial; lane rows 32mb + 8(i/4) + 4h + i%4 */
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[mb][nb][i] = fmaf(sc[nb], tmp[mb][nb][i], acc[mb][nb][i]);
        }
        /* the next group's stage is complete for every wave; this one is
         * free for the load issued next iteration */
        if (g + 2 < G)
            wait_prev();
        else
            q35_wait_vm<0>();
        q35_lds_barrier();
        st = st == 2 ? 0 : st + 1;
    }

    int nrow[2];
#pragma unroll
    for (int nb = 0; nb < 2; nb++) nrow[nb] = n0 + 64 * w + 32 * nb + c;
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

extern "C" hipError_t q35_mlx4_sb(const uint16_t *scales, const uint16_t *biases, Q35Mlx4SB *sb, int N,
                                  int G, hipStream_t stream) {
    if (N < 1 || G < 1) return hipErrorInvalidValue;
    const int64_t n = (int64_t)G * q35_mlx4_sb_npad(N);
    hipLaunchKernelGGL(sb_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, scales, biases, sb,
                       N, G, q35_mlx4_sb_npad(N));
    return hipGetLastError();
}

extern "C" int q35_mlx4_sb_npad(int N) { return (N + NTILE - 1) / NTILE * NTILE; }

extern "C" hipError_t q35_mlx4_wt(const uint32_t *vals, uint32_t *wt, int N, int K, hipStream_t stream) {
    if (N < 1 || K < 64 || K % 64 != 0) return hipErrorInvalidValue;
    const int64_t n = (int64_t)q35_mlx4_sb_npad(N) * (K / 64) * 2;   /* granules */
    hipLaunchKernelGGL(wt_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, vals,
                       reinterpret_cast<u32x4_t *>(wt), N, K, n);
    return hipGetLastError();
}

extern "C" hipError_t q35_mlx4_xprep(const Q35Mlx4Xprep *p, hipStream_t stream) {
    if (p->K % 64 != 0 || p->K > 8192 || p->Mpad % MT != 0 || p->M > p->Mpad || p->M < 1)
        return hipErrorInvalidValue;
    const int words = p->K / 8;           /* words of a row, NT a thread-step */
    if (words <= NT)
        hipLaunchKernelGGL(xprep_kernel<1>, dim3(p->Mpad), dim3(NT), 0, stream, *p);
    else if (words <= 2 * NT)
        hipLaunchKernelGGL(xprep_kernel<2>, dim3(p->Mpad), dim3(NT), 0, stream, *p);
    else
        hipLaunchKernelGGL(xprep_kernel<4>, dim3(p->Mpad), dim3(NT), 0, stream, *p);
    return hipGetLastError();
}

extern "C" hipError_t q35_mlx4_gemm(const Q35Mlx4Gemm *p, hipStream_t stream) {
    if (p->K < 64 || p->K % 64 != 0 || p->Mpad % MT != 0 || p->M > p->Mpad || p->M < 1 || p->njobs < 1 ||
        p->njobs > Q35_GEMM_MAX_JOBS || (int64_t)p->Mpad * p->K * 4 >= ((int64_t)1 << 31) ||
        (int64_t)(p->K / 64) * p->Mpad * 4 >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;
    /* buffer offsets are 32-bit: each weight and its (s, b') table below 2 GB */
    int64_t tiles = 0;
    for (int j = 0; j < p->njobs; j++) {
        const Q35Mlx4GemmJob *J = &p->jobs[j];
        if (J->N < 1 || !J->vals || !J->sb || !J->y || J->ldy < J->N ||
            (int64_t)q35_mlx4_sb_npad(J->N) * p->K / 2 >= ((int64_t)1 << 31) ||
            (int64_t)(p->K / 64) * q35_mlx4_sb_npad(J->N) * 8 >= ((int64_t)1 << 31))
            return hipErrorInvalidValue;
        tiles += (J->N + NTILE - 1) / NTILE;
    }
    tiles *= p->Mpad / MT;
    if (tiles >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_kernel, dim3((unsigned)tiles), dim3(NT), 0, stream, *p);
    return hipGetLastError();
}

extern "C" int q35_mlx4_gemm_mtile(void) { return MT; }
