/*
 * q35_device.h -- device helpers shared by the gfx950 kernels.
 */
#ifndef Q35_DEVICE_H
#define Q35_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2_t;

/* A pointer every lane holds the same value of, moved to scalar registers.
 * A buffer resource must be uniform; built from an address the compiler
 * computed in vector registers (64-bit products are VALU work on gfx9), it
 * would be wrapped in a readfirstlane loop at every load. */
template <typename T>
__device__ __forceinline__ T *q35_uniform_ptr(T *ptr) {
    const uint64_t v = (uint64_t)ptr;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T *)(((uint64_t)hi << 32) | lo);
}

/* dword 3 of a raw buffer resource on gfx9-family GPUs (no format
 * conversion, range checking against num_records: loads outside the range
 * return zero, stores outside it are dropped) */
constexpr int Q35_BUF_DW3 = 0x00020000;

#define Q35_GQA_D 256       /* GQA head dim */
#define Q35_GQA_GROUP 8     /* q heads per kv head */
#define Q35_ROPE_DIMS 64    /* rotary dims: head_dim * 0.25 */

__device__ __forceinline__ float q35_bf2f(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

/* float -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950). */
__device__ __forceinline__ uint16_t q35_f2bf(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

/* hi + lo split of a float into two bf16 (hi = rne(x), lo = rne(x - hi)). */
__device__ __forceinline__ void q35_split_bf16(float x, uint16_t &hi, uint16_t &lo) {
    hi = q35_f2bf(x);
    lo = q35_f2bf(x - q35_bf2f(hi));
}

__device__ __forceinline__ __bf16 q35_as_bf16(uint16_t h) {
    return __builtin_bit_cast(__bf16, h);
}

/* DPP lane moves (VALU-latency, no LDS round trip).  Controls used:
 * quad_perm [1,0,3,2] = 0xB1 (lane ^ 1), quad_perm [2,3,0,1] = 0x4E
 * (lane ^ 2), row_half_mirror = 0x141 (i <-> 7-i in each 8 lanes),
 * row_mirror = 0x140 (i <-> 15-i in each 16 lanes), row_ror:8 = 0x128. */
template <int CTRL>
__device__ __forceinline__ float q35_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ double q35_dpp(double x) {
    const long long b = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_mov_dpp((int)(b & 0xffffffff), CTRL, 0xF, 0xF, true);
    const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), CTRL, 0xF, 0xF, true);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

/* value of lane (l ^ 8) inside each 16-lane row */
__device__ __forceinline__ float q35_xor8(float x) { return q35_dpp<0x128>(x); }

/* sum over each aligned group of 8 lanes, the total in every lane of it */
template <typename T>
__device__ __forceinline__ T q35_sum8(T v) {
    v += q35_dpp<0xB1>(v);
    v += q35_dpp<0x4E>(v);
    v += q35_dpp<0x141>(v);
    return v;
}

__device__ __forceinline__ float q35_readlane(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double q35_readlane(double v, int l) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffff), l);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

/* Sums across 16-lane rows on gfx950's row swaps.  With both operands v,
 * permlane16_swap returns, for each pair of rows (0, 1) and (2, 3), the
 * even row's values in both rows of one result and the odd row's in both
 * rows of the other (permlane32_swap: the lower and the upper half), so the
 * sum of the two results is the pair's sum, in the same order in every lane
 * of the pair.  No LDS permute and no scalar round trip. */
__device__ __forceinline__ float q35_psum16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float q35_psum32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ double q35_psum16(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)b, hi = (uint32_t)(b >> 32);
    const auto rl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return __longlong_as_double((long long)(((uint64_t)rh[0] << 32) | rl[0])) +
           __longlong_as_double((long long)(((uint64_t)rh[1] << 32) | rl[1]));
}
__device__ __forceinline__ double q35_psum32(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)b, hi = (uint32_t)(b >> 32);
    const auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    return __longlong_as_double((long long)(((uint64_t)rh[0] << 32) | rl[0])) +
           __longlong_as_double((long long)(((uint64_t)rh[1] << 32) | rl[1]));
}

/* sum over the 64 lanes of a wave, the total in every lane (all 64 lanes
 * active): 16-lane row totals on DPP, then the two row swaps */
template <typename T>
__device__ __forceinline__ T q35_wave_sum(T v) {
    v = q35_sum8(v);
    v += q35_dpp<0x140>(v);
    return q35_psum32(q35_psum16(v));
}

/* sum over each 32-lane half of a wave, the half's total in each of its
 * lanes (all 64 lanes active) */
template <typename T>
__device__ __forceinline__ T q35_half_sum(T v) {
    v = q35_sum8(v);
    v += q35_dpp<0x140>(v);
    return q35_psum16(v);
}

/* The chunk GEMM's tiled X operand (written by its X prep and by the
 * delta-rule prefill's gated norm): x[m][k] of rows K wide as fp16 hi and
 * lo (x - hi), per 64-row tile and 64-column group g (G = K / 64) a 16 KB
 * block, hi then lo, each 64 rows of 128 bytes.  Word v = k / 8 of tile
 * row r sits at 16-byte slot (v % 8) ^ (r & 7) ^ ((r >> 3) & 1); half j of
 * the granule holds k % 8 = q35_xw_perm(j), the order 0,4,1,5,2,6,3,7 in
 * which a nibble word's values become fp16 pairs. */
constexpr int Q35_XW_ROWS = 64;
constexpr int Q35_XW_BLK = Q35_XW_ROWS * 128;
__device__ __forceinline__ int q35_xw_slot(int r, int j) { return j ^ (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int q35_xw_perm(int j) { return (j >> 1) + 4 * (j & 1); }
/* byte offset of the hi granule of word v of row m (lo: + Q35_XW_BLK) */
__device__ __forceinline__ size_t q35_xw_granule(int m, int v, int G) {
    const int r = m & (Q35_XW_ROWS - 1);
    return ((size_t)(m / Q35_XW_ROWS) * G + (v >> 3)) * (2 * Q35_XW_BLK) + r * 128 + q35_xw_slot(r, v & 7) * 16;
}

/* Direct-to-LDS loads (buffer_load ... lds): lane l's 16 (dma16) or 4
 * (dma4) bytes from buffer offset soff + voff, range-checked against the
 * resource, land at LDS byte lds + 16 l (4 l).  Issued as inline assembly
 * so the compiler's wait insertion does not see them: it cannot tell LDS
 * stages apart and would wait for every staging load in flight before the
 * next LDS read.  A kernel using them orders them itself (q35_wait_vm
 * before the barrier that publishes a stage); loads the compiler does not
 * count can only make its own load waits stricter. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   /* m0 is reserved; nothing else here uses it */
__device__ __forceinline__ void q35_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t lds, uint32_t voff,
                                          uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rs), "s"(soff)
                 : "memory", "m0");
}
__device__ __forceinline__ void q35_dma4(__amdgpu_buffer_rsrc_t rs, uint32_t lds, uint32_t voff,
                                         uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rs), "s"(soff)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

/* Cache policy (the aux operand of a raw buffer store) of the decode
 * kernels' outputs: sc1 sends the store through to the memory side instead
 * of leaving the line dirty in this XCD's L2, so the end-of-kernel
 * writeback has none of it left to flush, and the next kernel, on whichever
 * XCD, reads it from the MALL.  Delta-rule state stores: 4.92 -> 4.67 us a
 * decode call, 40-layer stack +1.7 %; GQA split partials: -0.2 us an op;
 * nt or sc0 alone change nothing, and sc0 | sc1 | nt (streaming) evicts the
 * state from the MALL (stack -2 %). */
constexpr int Q35_ST_SC1 = 0x10;

/* s_waitcnt vmcnt(N), expcnt and lgkmcnt left open: at most N of this
 * wave's vector memory loads (direct-to-LDS ones included) in flight */
template <int N>
__device__ __forceinline__ void q35_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

/* LDS byte address of a shared-memory pointer (for M0) */
template <typename T>
__device__ __forceinline__ uint32_t q35_lds_addr(T *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) T *)p;
}

/* Workgroup barrier that orders LDS only.  __syncthreads() carries a
 * workgroup-scope fence over all address spaces, which gfx950 implements as
 * s_waitcnt vmcnt(0) lgkmcnt(0) before s_barrier: every global load in
 * flight (a prefetch of the next tile) would be drained at each barrier.
 * Where waves exchange data through LDS alone, this barrier waits for LDS
 * operations only (s_waitcnt lgkmcnt(0); s_barrier) and global loads stay
 * in flight across it. */
__device__ __forceinline__ void q35_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* fp16 range guard.  A float of magnitude 65520 or more rounds to an fp16
 * infinity.  A kernel that stores values as fp16 operands passes each
 * value's check here; any lane whose value is out of range sets `bit` in
 * the status word (device memory the host reads after the launches), so the
 * host can recompute the affected work on a path without fp16 operands.
 * Out-of-range values never occur in normal activations; the check costs a
 * compare per value and the atomic only runs when one is out of range. */
__device__ __forceinline__ bool q35_f16_over(float x) { return fabsf(x) >= 65520.0f; }
__device__ __forceinline__ void q35_f16_guard(int *status, int bit, bool over) {
    if (over && status) atomicOr(status, bit);
}

/* exp on the hardware 2^x instruction (v_exp_f32), ~1e-7 relative error:
 * used for softmax weights, whose reference-order expf only matters to
 * float rounding. */
__device__ __forceinline__ float q35_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

/* sigmoid written as the reference writes it: 1 / (1 + expf(-x)). */
__device__ __forceinline__ float q35_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* The same on the hardware's approximate exp and reciprocal (v_exp_f32 of
 * -x log2(e), v_rcp_f32: about 1 ulp each; exp(-x) = inf for very negative
 * x gives rcp(inf) = 0), for the prefill epilogues, whose outputs carry
 * fp16-operand error orders of magnitude larger. */
__device__ __forceinline__ float q35_sigmoid_fast(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

/* splitmix64 finaliser (public algorithm; the same constants as the
 * reference's ds4f_mix64, src/router.c:11-16). */
__device__ __forceinline__ uint64_t q35_fmix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 27;
    z *= 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Draw i (0-based) of stream (seed, tid). */
__device__ __forceinline__ uint64_t q35_draw(uint64_t seed, uint64_t tid, uint64_t i) {
    uint64_t s0 = seed ^ (tid * 0xD1B54A32D192ED03ull);
    return q35_fmix64(s0 + (i + 1) * 0x9E3779B97F4A7C15ull);
}

__device__ __forceinline__ double q35_unit(uint64_t x) {
    return (double)(x >> 11) * (1.0 / 9007199254740992.0);
}

/* Element i of a normal stream, in double (Box-Muller, cosine branch). */
__device__ __forceinline__ double q35_normal(uint64_t seed, uint64_t tid, uint64_t i) {
    double u1 = q35_unit(q35_draw(seed, tid, 2 * i));
    double u2 = q35_unit(q35_draw(seed, tid, 2 * i + 1));
    return sqrt(-2.0 * log(1.0 - u1)) * cos(2.0 * 3.141592653589793 * u2);
}

/* GQA head prologue: RMSNorm (double sum of squares, eps on the mean, x / r * w) and
 * half-split RoPE of one head held as 4 dims per lane (dims 4l..4l+3).
 * w: the 4 bf16 weights of those dims; c, s: cos / sin of rotary index
 * (4l & 31) .. +3, used by lanes < 16 only. */
__device__ __forceinline__ float4 q35_norm_rope_head(float4 x, uint2 w, float4 c, float4 s,
                                                     int lane) {
#pragma clang fp contract(off)
    double ss = (double)x.x * x.x + (double)x.y * x.y + (double)x.z * x.z + (double)x.w * x.w;
    ss = q35_wave_sum(ss);
    const float r = sqrtf((float)(ss / (double)Q35_GQA_D) + 1e-6f);
    float v[4] = {x.x, x.y, x.z, x.w};
    const uint16_t wt[4] = {(uint16_t)(w.x & 0xffff), (uint16_t)(w.x >> 16),
                            (uint16_t)(w.y & 0xffff), (uint16_t)(w.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = v[e] / r * q35_bf2f(wt[e]);
    /* RoPE pairs (i, i+32), i < 32: lanes 0..7 hold i, lanes 8..15 hold i+32 */
    const float cc[4] = {c.x, c.y, c.z, c.w}, sn[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float pr = q35_xor8(v[e]);
        if (lane < Q35_ROPE_DIMS / 8)
            v[e] = v[e] * cc[e] - pr * sn[e];        /* x0*c - x1*s */
        else if (lane < Q35_ROPE_DIMS / 4)
            v[e] = pr * sn[e] + v[e] * cc[e];        /* x0*s + x1*c */
    }
    return make_float4(v[0], v[1], v[2], v[3]);
}

/* Causal conv tap sum + SiLU of one delta-rule channel
 * (src/attn_qwen.c:493-504): tap k reads position pos-3+k (k = 3 is the
 * incoming raw value); taps before position 0 are skipped.  w holds the
 * channel's 4 bf16 taps, oldest first. */
__device__ __forceinline__ float q35_conv_silu(const float (&x)[4], uint2 w, int pos) {
#pragma clang fp contract(off)
    const uint16_t wt[4] = {(uint16_t)(w.x & 0xffff), (uint16_t)(w.x >> 16),
                            (uint16_t)(w.y & 0xffff), (uint16_t)(w.y >> 16)};
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (pos - 3 + k >= 0) acc += x[k] * q35_bf2f(wt[k]);
    return acc * q35_sigmoid(acc);
}

/* The same with exp and the reciprocal on the hardware's approximate
 * instructions (v_exp_f32 of x log2(e), v_rcp_f32: about 1 ulp each for
 * the conv outputs' range); for the throughput-bound prefill. */
__device__ __forceinline__ float q35_conv_silu_fast(const float (&x)[4], uint2 w, int pos) {
#pragma clang fp contract(off)
    const uint16_t wt[4] = {(uint16_t)(w.x & 0xffff), (uint16_t)(w.x >> 16),
                            (uint16_t)(w.y & 0xffff), (uint16_t)(w.y >> 16)};
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (pos - 3 + k >= 0) acc += x[k] * q35_bf2f(wt[k]);
    return acc * __builtin_amdgcn_rcpf(1.0f + __expf(-acc));
}

/* Delta-rule gates of one value head (src/attn_qwen.c:545-551, :664-665):
 * log-decay g = -exp(A_log) * softplus(a + dt_bias) in the reference's
 * branch form, and beta = sigmoid(b). */
__device__ __forceinline__ void q35_lin_gates(float a, float b, float A_log, uint16_t dt_bias,
                                              float *g, float *beta) {
#pragma clang fp contract(off)
    const float x = a + q35_bf2f(dt_bias);
    const float sp = x > 0 ? x + log1pf(expf(-x)) : log1pf(expf(x));
    *g = -expf(A_log) * sp;
    *beta = q35_sigmoid(b);
}

/* Device K / V tile addressing (see q35_launch.h). */
__device__ __forceinline__ size_t q35_k_index(int kvh, int p, int d, int t_tiles) {
    return ((((size_t)kvh * t_tiles + (p >> 4)) * (Q35_GQA_D / 32) + (d >> 5)) * 16 + (p & 15)) * 32 +
           (d & 31);
}
__device__ __forceinline__ size_t q35_v_index(int kvh, int p, int d, int t_tiles) {
    return (((size_t)kvh * t_tiles + (p >> 4)) * Q35_GQA_D + d) * 16 + (p & 15);
}

#endif /* Q35_DEVICE_H */
