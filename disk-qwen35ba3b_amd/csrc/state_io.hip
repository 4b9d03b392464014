/*
 * state_io.hip -- moves attention state between the engine's host layouts
 * (include/ds4f/attn.h:26-34: fp32 cache rows [token][k | v], fp32 state
 * [vh][kd][vd]) and the device layouts of q35_launch.h, and fills device
 * state with the workload generator's streams.
 */
#include "q35_device.h"
#include "q35_launch.h"

namespace {

constexpr int D = Q35_GQA_D;

/* one thread per (row, kv head, dim) of k and of v */
__global__ void kv_import_kernel(const float *rows, int p0, int n, uint16_t *kt, uint16_t *vt,
                                 int t_tiles, int kvh_n) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per = (int64_t)kvh_n * D;
    if (e >= (int64_t)n * per) return;
    const int r = (int)(e / per), rem = (int)(e % per), kvh = rem / D, d = rem % D;
    const float *row = rows + (size_t)r * 2 * per;
    kt[q35_k_index(kvh, p0 + r, d, t_tiles)] = q35_f2bf(row[rem]);
    vt[q35_v_index(kvh, p0 + r, d, t_tiles)] = q35_f2bf(row[per + rem]);
}

__global__ void kv_export_kernel(float *rows, int p0, int n, const uint16_t *kt,
                                 const uint16_t *vt, int t_tiles, int kvh_n) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per = (int64_t)kvh_n * D;
    if (e >= (int64_t)n * per) return;
    const int r = (int)(e / per), rem = (int)(e % per), kvh = rem / D, d = rem % D;
    float *row = rows + (size_t)r * 2 * per;
    row[rem] = q35_bf2f(kt[q35_k_index(kvh, p0 + r, d, t_tiles)]);
    row[per + rem] = q35_bf2f(vt[q35_v_index(kvh, p0 + r, d, t_tiles)]);
}

/* dst[h][c][r] = src[h][r][c] through a 32x32 LDS tile */
__global__ void transpose_kernel(const float *src, float *dst, int rows, int cols) {
    __shared__ float tile[32][33];
    const int h = blockIdx.z;
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const float *s = src + (size_t)h * rows * cols;
    float *o = dst + (size_t)h * rows * cols;
    for (int i = threadIdx.y; i < 32; i += blockDim.y) {
        int r = r0 + i, c = c0 + threadIdx.x;
        if (r < rows && c < cols) tile[i][threadIdx.x] = s[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = threadIdx.y; i < 32; i += blockDim.y) {
        int c = c0 + i, r = r0 + threadIdx.x;
        if (r < rows && c < cols) o[(size_t)c * rows + r] = tile[threadIdx.x][i];
    }
}

__global__ void synth_kernel(void *dst, int64_t n, int dtype, int dist, double p0, double p1,
                             uint64_t seed, uint64_t tid) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    double v;
    if (dist == 0)
        v = p0 + p1 * q35_normal(seed, tid, (uint64_t)i);
    else
        v = p0 + (p1 - p0) * q35_unit(q35_draw(seed, tid, (uint64_t)i));
    const float f = (float)v;
    if (dtype == 0)
        static_cast<float *>(dst)[i] = f;
    else if (dtype == 1)
        static_cast<uint16_t *>(dst)[i] = q35_f2bf(f);
    else
        static_cast<float *>(dst)[i] = q35_bf2f(q35_f2bf(f));
}

/* element i of the logical [pos][kvh][dim] order -> tiles */
__global__ void synth_kv_kernel(uint16_t *kt, uint16_t *vt, int n_past, int t_tiles, int kvh_n,
                                uint64_t seed, uint64_t tid_k, uint64_t tid_v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per = (int64_t)kvh_n * D;
    if (i >= (int64_t)n_past * per) return;
    const int p = (int)(i / per), rem = (int)(i % per), kvh = rem / D, d = rem % D;
    kt[q35_k_index(kvh, p, d, t_tiles)] = q35_f2bf((float)q35_normal(seed, tid_k, (uint64_t)i));
    vt[q35_v_index(kvh, p, d, t_tiles)] = q35_f2bf((float)q35_normal(seed, tid_v, (uint64_t)i));
}

/* element i of the logical [h][kd][vd] order -> value-major [h][vd][kd] */
__global__ void synth_state_kernel(float *state, int heads, int kd, int vd, double sigma,
                                   uint64_t seed, uint64_t tid) {
    /* thread i writes element i of the value-major state (coalesced); the
     * value is element (h, r, c) of the row-major stream */
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)heads * kd * vd) return;
    const int h = (int)(i / ((int64_t)kd * vd)), rem = (int)(i % ((int64_t)kd * vd));
    const int c = rem / kd, r = rem % kd;
    const int64_t src = (int64_t)h * kd * vd + (int64_t)r * vd + c;
    state[i] = sigma == 0.0 ? 0.0f : (float)(sigma * q35_normal(seed, tid, (uint64_t)src));
}

/* element i of [3][rows] (positions token-3..token-1) -> ring slot pos%4 */
__global__ void synth_conv_kernel(float *ring, int rows, int token, uint64_t seed, uint64_t tid) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)3 * rows) return;
    const int r = (int)(i / rows), ch = (int)(i % rows);
    const int pos = token - 3 + r;
    if (pos < 0) return;
    ring[(size_t)(pos & 3) * rows + ch] = (float)q35_normal(seed, tid, (uint64_t)i);
}

inline dim3 grid_for(int64_t n, int bs) { return dim3((unsigned)((n + bs - 1) / bs)); }

}  // namespace

extern "C" hipError_t q35_kv_import(const float *rows, int p0, int n, uint16_t *kt, uint16_t *vt,
                                    int t_tiles, int kv_heads, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t total = (int64_t)n * kv_heads * D;
    hipLaunchKernelGGL(kv_import_kernel, grid_for(total, 256), dim3(256), 0, stream, rows, p0, n,
                       kt, vt, t_tiles, kv_heads);
    return hipGetLastError();
}

extern "C" hipError_t q35_kv_export(float *rows, int p0, int n, const uint16_t *kt,
                                    const uint16_t *vt, int t_tiles, int kv_heads,
                                    hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t total = (int64_t)n * kv_heads * D;
    hipLaunchKernelGGL(kv_export_kernel, grid_for(total, 256), dim3(256), 0, stream, rows, p0, n,
                       kt, vt, t_tiles, kv_heads);
    return hipGetLastError();
}

extern "C" hipError_t q35_state_transpose(const float *src, float *dst, int heads, int rows,
                                          int cols, hipStream_t stream) {
    dim3 grid((cols + 31) / 32, (rows + 31) / 32, heads);
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(32, 8), 0, stream, src, dst, rows, cols);
    return hipGetLastError();
}

extern "C" hipError_t q35_synth(void *dst, int64_t n, int dtype, int dist, double p0, double p1,
                                uint64_t seed, uint64_t tid, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(synth_kernel, grid_for(n, 256), dim3(256), 0, stream, dst, n, dtype, dist,
                       p0, p1, seed, tid);
    return hipGetLastError();
}

extern "C" hipError_t q35_synth_kv(uint16_t *kt, uint16_t *vt, int n_past, int t_tiles,
                                   int kv_heads, uint64_t seed, uint64_t tid_k, uint64_t tid_v,
                                   hipStream_t stream) {
    if (n_past <= 0) return hipSuccess;
    const int64_t total = (int64_t)n_past * kv_heads * D;
    hipLaunchKernelGGL(synth_kv_kernel, grid_for(total, 256), dim3(256), 0, stream, kt, vt,
                       n_past, t_tiles, kv_heads, seed, tid_k, tid_v);
    return hipGetLastError();
}

extern "C" hipError_t q35_synth_state(float *state, int heads, int kd, int vd, double sigma,
                                      uint64_t seed, uint64_t tid, hipStream_t stream) {
    const int64_t total = (int64_t)heads * kd * vd;
    hipLaunchKernelGGL(synth_state_kernel, grid_for(total, 256), dim3(256), 0, stream, state,
                       heads, kd, vd, sigma, seed, tid);
    return hipGetLastError();
}

extern "C" hipError_t q35_synth_conv(float *ring, int rows, int token, uint64_t seed,
                                     uint64_t tid, hipStream_t stream) {
    const int64_t total = (int64_t)3 * rows;
    hipLaunchKernelGGL(synth_conv_kernel, grid_for(total, 256), dim3(256), 0, stream, ring, rows,
                       token, seed, tid);
    return hipGetLastError();
}

/* ---- launch floor ---------------------------------------------------------
 * A kernel that does nothing: n launches of it in a row (in a HIP graph)
 * time the fixed cost of a kernel boundary on this GPU, the floor under
 * every latency-bound launch of the decode step. */
namespace {
__global__ void empty_kernel() {}
}  // namespace

extern "C" hipError_t q35_empty_kernels(int n, int grid, int block, hipStream_t stream) {
    if (n < 0 || grid < 1 || block < 1 || block > 1024) return hipErrorInvalidValue;
    for (int i = 0; i < n; i++) {
        hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(block), 0, stream);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
