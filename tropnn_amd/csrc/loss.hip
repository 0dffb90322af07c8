// Cross entropy of the classifier's training step (examples/emnist.py:221,
// F.cross_entropy(logits, y), mean over rows), forward and gradient in one
// launch. torch runs it as four kernels (log_softmax, nll forward, nll
// backward, log_softmax backward) plus a fill, ~25 us at batch 512; the
// answer needs one pass over the logits.
//
// One workgroup of 1024 threads; thread tid takes rows tid, tid + 1024, ...
// (of the whole input, or of each LDS tile of up to 1024 rows), in order, so
// every sum has a fixed order:
//   count  = number of rows whose target is not ignore_index
//   loss   = sum_i (log(sum_j exp(x_ij - max_i)) - (x_i,y_i - max_i)) / count
//   grad_ij = (exp(x_ij - max_i) / sum_i - [j == y_i]) / count  (0 on ignored rows)
// A target outside [0, classes) that is not ignore_index makes the loss NaN
// (torch stops on a device assert there).
#include <math.h>

#include "device.hpp"
#include "launch.hpp"

namespace tropnn {
namespace {

constexpr int kCeThreads = 1024;
constexpr int kCeTileFloats = 12288;  // 48 KB of LDS: a tile of rows

__device__ float block_sum(float v, float *red, int tid) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kCeThreads / kWave; ++w) s += red[w];  // the same order in every thread
    __syncthreads();
    return s;
}

// One row: the loss term (as log_softmax: no rounding at the logits'
// magnitude) added to `part`, the gradient row written through `g` (which may
// alias `x`: each x[j] is read before g[j] is written).
__device__ __forceinline__ void ce_row(const float *x, float *g, int64_t y, int classes, int64_t ignore_index,
                                       float inv, float &part) {
    if (y == ignore_index) {
        for (int j = 0; j < classes; ++j) g[j] = 0.f;
        return;
    }
    float mx = -INFINITY;
    for (int j = 0; j < classes; ++j) mx = fmaxf(mx, x[j]);
    float s = 0.f;
    for (int j = 0; j < classes; ++j) s += expf(x[j] - mx);
    if (y < 0 || y >= classes) {
        part += NAN;
        for (int j = 0; j < classes; ++j) g[j] = NAN;
        return;
    }
    part += logf(s) - (x[y] - mx);
    const float rs = 1.f / s;
    for (int j = 0; j < classes; ++j) g[j] = (expf(x[j] - mx) * rs - (j == y ? 1.f : 0.f)) * inv;
}

// tile_rows > 0: rows pass through LDS in tiles of tile_rows (coalesced loads
// and stores, one thread per row on the LDS copy); 0 (rows wider than the
// tile): each thread reads its rows from global memory.
// (count, loss) pairs summed over the workgroup in a fixed order.
__device__ float2 block_sum2(float2 v, float2 *red, int tid) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        v.x += __shfl_xor(v.x, d, kWave);
        v.y += __shfl_xor(v.y, d, kWave);
    }
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = v;
    __syncthreads();
    float2 s = make_float2(0.f, 0.f);
#pragma unroll
    for (int w = 0; w < kCeThreads / kWave; ++w) {
        s.x += red[w].x;
        s.y += red[w].y;
    }
    return s;
}

__global__ __launch_bounds__(kCeThreads) void cross_entropy_kernel(const float *__restrict__ logits,
                                                                  const int64_t *__restrict__ target, int64_t rows,
                                                                  int classes, int64_t ignore_index, int tile_rows,
                                                                  float *__restrict__ loss,
                                                                  float *__restrict__ grad) {
    __shared__ float red[kCeThreads / kWave];
    __shared__ float2 red2[kCeThreads / kWave];
    __shared__ __align__(16) float tile[kCeTileFloats];
    const int tid = threadIdx.x;
    // the first tile's logits and targets are loaded with the target count's
    // loads, all in flight together (the kernel is a chain of round trips)
    constexpr int kLoads = kCeTileFloats / kCeThreads;
    float v[kLoads];
    int64_t y = 0;
    auto load_tile = [&](int64_t r0, int nr) {
        const float *src = logits + r0 * classes;
        const int n = nr * classes;
#pragma unroll
        for (int u = 0; u < kLoads; ++u) v[u] = tid + u * kCeThreads < n ? src[tid + u * kCeThreads] : 0.f;
        y = tid < nr ? target[r0 + tid] : 0;
    };
    auto tile_rows_at = [&](int64_t r0) { return static_cast<int>(rows - r0 < tile_rows ? rows - r0 : tile_rows); };
    if (tile_rows > 0) load_tile(0, tile_rows_at(0));
    if (tile_rows >= rows) {
        // one tile: the rows' unscaled gradients go to LDS while the target
        // count and the loss sum share one reduction, then the scaled store
        const int nr = static_cast<int>(rows), n = nr * classes;
#pragma unroll
        for (int u = 0; u < kLoads; ++u)
            if (tid + u * kCeThreads < n) tile[tid + u * kCeThreads] = v[u];
        __syncthreads();
        float part = 0.f;
        if (tid < nr) ce_row(tile + tid * classes, tile + tid * classes, y, classes, ignore_index, 1.f, part);
        const float counted = tid < nr && y != ignore_index ? 1.f : 0.f;
        float2 cp = block_sum2(make_float2(counted, part), red2, tid);
        const float inv = cp.x > 0.f ? 1.f / cp.x : 0.f;  // every row ignored: zero gradients, NaN loss
#pragma unroll
        for (int u = 0; u < kLoads; ++u)
            if (tid + u * kCeThreads < n) grad[tid + u * kCeThreads] = tile[tid + u * kCeThreads] * inv;
        if (tid == 0) *loss = cp.y / cp.x;
        return;
    }
    float counted = 0.f;
    for (int64_t i = tid; i < rows; i += kCeThreads) counted += target[i] != ignore_index ? 1.f : 0.f;
    const float count = block_sum(counted, red, tid);
    const float inv = 1.f / count;
    float part = 0.f;
    if (tile_rows > 0) {
        for (int64_t r0 = 0; r0 < rows; r0 += tile_rows) {
            const int nr = tile_rows_at(r0), n = nr * classes;
#pragma unroll
            for (int u = 0; u < kLoads; ++u)
                if (tid + u * kCeThreads < n) tile[tid + u * kCeThreads] = v[u];
            __syncthreads();
            if (tid < nr) ce_row(tile + tid * classes, tile + tid * classes, y, classes, ignore_index, inv, part);
            __syncthreads();
            float *dst = grad + r0 * classes;
#pragma unroll
            for (int u = 0; u < kLoads; ++u)
                if (tid + u * kCeThreads < n) dst[tid + u * kCeThreads] = tile[tid + u * kCeThreads];
            if (r0 + tile_rows < rows) load_tile(r0 + tile_rows, tile_rows_at(r0 + tile_rows));
            __syncthreads();
        }
    } else {
        for (int64_t i = tid; i < rows; i += kCeThreads)
            ce_row(logits + i * classes, grad + i * classes, target[i], classes, ignore_index, inv, part);
    }
    const float total = block_sum(part, red, tid);
    if (tid == 0) *loss = total / count;
}

}  // namespace

hipError_t launch_cross_entropy(const float *logits, const int64_t *target, int64_t rows, int classes,
                                int64_t ignore_index, float *loss, float *grad_logits, hipStream_t stream) {
    int tile_rows = kCeTileFloats / classes;
    if (tile_rows > kCeThreads) tile_rows = kCeThreads;
    hipLaunchKernelGGL(cross_entropy_kernel, dim3(1), dim3(kCeThreads), 0, stream, logits, target, rows, classes,
                       ignore_index, tile_rows, loss, grad_logits);
    return hipGetLastError();
}

}  // namespace tropnn
