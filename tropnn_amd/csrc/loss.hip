// Cross entropy of the classifier's training step (examples/emnist.py:221,
// F.cross_entropy(logits, y), mean over rows), forward and gradient in one
// launch. torch runs it as four kernels (log_softmax, nll forward, nll
// backward, log_softmax backward) plus a fill, ~25 us at batch 512; the
// answer needs one pass over the logits.
//
// One workgroup of 1024 threads; thread tid takes rows tid, tid + 1024, ...
// in order, so every sum has a fixed order:
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

__global__ __launch_bounds__(kCeThreads) void cross_entropy_kernel(const float *__restrict__ logits,
                                                                  const int64_t *__restrict__ target, int64_t rows,
                                                                  int classes, int64_t ignore_index,
                                                                  float *__restrict__ loss,
                                                                  float *__restrict__ grad) {
    __shared__ float red[kCeThreads / kWave];
    const int tid = threadIdx.x;
    float counted = 0.f;
    for (int64_t i = tid; i < rows; i += kCeThreads) counted += target[i] != ignore_index ? 1.f : 0.f;
    const float count = block_sum(counted, red, tid);
    const float inv = 1.f / count;
    float part = 0.f;
    for (int64_t i = tid; i < rows; i += kCeThreads) {
        const float *x = logits + i * classes;
        float *g = grad + i * classes;
        const int64_t y = target[i];
        if (y == ignore_index) {
            for (int j = 0; j < classes; ++j) g[j] = 0.f;
            continue;
        }
        float mx = -INFINITY;
        for (int j = 0; j < classes; ++j) mx = fmaxf(mx, x[j]);
        float s = 0.f;
        for (int j = 0; j < classes; ++j) s += expf(x[j] - mx);
        if (y < 0 || y >= classes) {
            part += NAN;
            for (int j = 0; j < classes; ++j) g[j] = NAN;
            continue;
        }
        part += logf(s) - (x[y] - mx);  // as log_softmax: no rounding at the logits' magnitude
        const float rs = 1.f / s;
        for (int j = 0; j < classes; ++j) g[j] = (expf(x[j] - mx) * rs - (j == y ? 1.f : 0.f)) * inv;
    }
    const float total = block_sum(part, red, tid);
    if (tid == 0) *loss = total / count;
}

}  // namespace

hipError_t launch_cross_entropy(const float *logits, const int64_t *target, int64_t rows, int classes,
                                int64_t ignore_index, float *loss, float *grad_logits, hipStream_t stream) {
    hipLaunchKernelGGL(cross_entropy_kernel, dim3(1), dim3(kCeThreads), 0, stream, logits, target, rows, classes,
                       ignore_index, loss, grad_logits);
    return hipGetLastError();
}

}  // namespace tropnn
