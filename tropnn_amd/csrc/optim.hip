// Adam / AdamW step over many f32 tensors in one launch: the optimizer of the
// classifier's training step. The reference trains it with
// torch.optim.AdamW(weight_decay=0) (examples/emnist.py:310); torch's
// multi-tensor kernel gives each 65,536 parameters one workgroup, ~37
// workgroups for the classifier's 2.4 M parameters, so few CUs work. Here a
// grid-stride loop over the 4-element quads of all tensors fills the GPU.
//
// Per element, in the op order of torch's single-tensor Adam (non-amsgrad):
//   AdamW:  p = p * (1 - lr wd)          Adam: g = g + wd p          (wd != 0)
//   m = lerp(m, g, 1 - b1)               (torch's lerp: two fma forms around 0.5)
//   v = v b2 + (1 - b2) g g
//   p = p - (lr / (1 - b1^t)) * (m / (sqrt(v) / sqrt(1 - b2^t) + eps))
// with t = *steps[k] + 1 read from device memory (one counter per tensor, as
// torch keeps one per parameter), so a captured step replays with the current
// count; a second launch then stores *steps[k] = t.
#include "device.hpp"
#include "launch.hpp"

namespace tropnn {
namespace {

constexpr int kAdamThreads = 256;
// quads per thread and round (c5 step: 1 quad 78.5 us, 2 quads 78.7 us, 4
// quads 80.3 us; A/B on one box)
constexpr int kAdamQuads = 1;
constexpr int kAdamMaxBlocks = 65536;  // one round up to 16 M quads

struct AdamArgs {
    float *p[kAdamGroup];
    const float *g[kAdamGroup];
    float *m[kAdamGroup];
    float *v[kAdamGroup];
    float *steps[kAdamGroup];
    int64_t numel[kAdamGroup];
    int64_t qstart[kAdamGroup + 1];  // quad offsets of the tensors in the group's joint range
    unsigned vec_mask;               // bit k: tensor k's four pointers are 16-byte aligned
    double lr, b1, b2;               // for the bias corrections, computed in f64 as torch does on the host
    float b2f, w1, w2, eps, wd, decay;  // f32 per-element constants: beta2, 1 - beta1, 1 - beta2, eps, wd, 1 - lr wd
    int decoupled, n;
};

struct AdamScalars {
    float step_size, bc2_sqrt;
};

// One element in the op sequence of torch's single-tensor Adam, each op
// rounded to f32 (no contraction), except where torch's kernels form a fused
// multiply-add: lerp and add with alpha (the coupled weight decay).
__device__ __forceinline__ void adam_one(float &p, float g, float &m, float &v, const AdamArgs &a,
                                         const AdamScalars s) {
#pragma clang fp contract(off)
    if (a.wd != 0.f) {
        if (a.decoupled)
            p = p * a.decay;
        else
            g = __builtin_fmaf(p, a.wd, g);
    }
    m = a.w1 < 0.5f ? __builtin_fmaf(a.w1, g - m, m) : __builtin_fmaf(-(1.f - a.w1), g - m, g);
    v = v * a.b2f;
    v = v + a.w2 * g * g;
    const float denom = sqrtf(v) / s.bc2_sqrt + a.eps;
    p = p - s.step_size * (m / denom);
}

// Scalar bias corrections of tensor k from its step counter, in f64 as torch
// forms them on the host.
__device__ __forceinline__ AdamScalars adam_scalars(const AdamArgs &a, float step) {
    const double t = static_cast<double>(step + 1.f);
    AdamScalars s;
    s.step_size = static_cast<float>(a.lr / (1.0 - pow(a.b1, t)));
    s.bc2_sqrt = static_cast<float>(sqrt(1.0 - pow(a.b2, t)));
    return s;
}

// One quad (4 elements) of tensor k at element i, when its four pointers are
// 16-byte aligned and the quad is whole; else element by element.
__device__ __forceinline__ void adam_quad_general(const AdamArgs &a, const AdamScalars *sc, int64_t q) {
    int k = 0;
    while (k < a.n - 1 && q >= a.qstart[k + 1]) ++k;
    const int64_t i = (q - a.qstart[k]) * 4;
    const AdamScalars s = sc[k];
    if ((a.vec_mask >> k & 1u) && i + 4 <= a.numel[k]) {
        float4 p = *reinterpret_cast<const float4 *>(a.p[k] + i);
        const float4 g = *reinterpret_cast<const float4 *>(a.g[k] + i);
        float4 m = *reinterpret_cast<const float4 *>(a.m[k] + i);
        float4 v = *reinterpret_cast<const float4 *>(a.v[k] + i);
        adam_one(p.x, g.x, m.x, v.x, a, s);
        adam_one(p.y, g.y, m.y, v.y, a, s);
        adam_one(p.z, g.z, m.z, v.z, a, s);
        adam_one(p.w, g.w, m.w, v.w, a, s);
        *reinterpret_cast<float4 *>(a.p[k] + i) = p;
        *reinterpret_cast<float4 *>(a.m[k] + i) = m;
        *reinterpret_cast<float4 *>(a.v[k] + i) = v;
    } else {
        const int64_t end = i + 4 < a.numel[k] ? i + 4 : a.numel[k];
        for (int64_t e = i; e < end; ++e) {
            float p = a.p[k][e], m = a.m[k][e], v = a.v[k][e];
            adam_one(p, a.g[k][e], m, v, a, s);
            a.p[k][e] = p;
            a.m[k][e] = m;
            a.v[k][e] = v;
        }
    }
}

// A thread takes kAdamQuads quads per round, kAdamThreads apart (a wave's 64
// quads of a round are consecutive). Every load of a round is issued before
// the thread waits for any: in the first round also before the step counters
// and the bias corrections the update needs, which wave 0 forms while the
// data is in flight.
__global__ __launch_bounds__(kAdamThreads) void adam_kernel(AdamArgs a) {
    __shared__ AdamScalars sc[kAdamGroup];
    const int64_t total = a.qstart[a.n];
    const int lane = threadIdx.x % kWave;
    const bool counter = threadIdx.x < static_cast<unsigned>(a.n);
    const float step = counter ? *a.steps[threadIdx.x] : 0.f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * (kAdamThreads * kAdamQuads);
    bool have_scalars = false;  // uniform
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * (kAdamThreads * kAdamQuads);; base += stride) {
        // A wave whose 64 quads lie in one tensor with 16-byte aligned
        // pointers, none of them its partial last quad (the common case),
        // has a wave-uniform tensor index and pointers: scalar loads of the
        // arguments instead of per-lane ones.
        float4 p[kAdamQuads], g[kAdamQuads], m[kAdamQuads], v[kAdamQuads];
        int kw[kAdamQuads];
        bool fast[kAdamQuads];
#pragma unroll
        for (int u = 0; u < kAdamQuads; ++u) {
            const int64_t q = base + u * kAdamThreads + threadIdx.x;
            const int64_t qw = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(q - lane)) |
                               (static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>((q - lane) >> 32))) << 32);
            int k = 0;
            while (k < a.n - 1 && qw >= a.qstart[k + 1]) ++k;
            kw[u] = k;
            fast[u] = qw + kWave <= a.qstart[k + 1] && (a.vec_mask >> k & 1u) && (qw + kWave - a.qstart[k]) * 4 <= a.numel[k];
            if (fast[u]) {
                const int64_t i = (q - a.qstart[k]) * 4;
                p[u] = *reinterpret_cast<const float4 *>(a.p[k] + i);
                g[u] = *reinterpret_cast<const float4 *>(a.g[k] + i);
                m[u] = *reinterpret_cast<const float4 *>(a.m[k] + i);
                v[u] = *reinterpret_cast<const float4 *>(a.v[k] + i);
            }
        }
        if (!have_scalars) {
            if (counter) sc[threadIdx.x] = adam_scalars(a, step);
            __syncthreads();
            have_scalars = true;
        }
#pragma unroll
        for (int u = 0; u < kAdamQuads; ++u) {
            const int64_t q = base + u * kAdamThreads + threadIdx.x;
            if (fast[u]) {
                const int k = kw[u];
                const int64_t i = (q - a.qstart[k]) * 4;
                const AdamScalars s = sc[k];
                adam_one(p[u].x, g[u].x, m[u].x, v[u].x, a, s);
                adam_one(p[u].y, g[u].y, m[u].y, v[u].y, a, s);
                adam_one(p[u].z, g[u].z, m[u].z, v[u].z, a, s);
                adam_one(p[u].w, g[u].w, m[u].w, v[u].w, a, s);
                *reinterpret_cast<float4 *>(a.p[k] + i) = p[u];
                *reinterpret_cast<float4 *>(a.m[k] + i) = m[u];
                *reinterpret_cast<float4 *>(a.v[k] + i) = v[u];
            } else if (q < total) {
                adam_quad_general(a, sc, q);
            }
        }
        if (base + stride >= total) break;
    }
}

struct AdvanceArgs {
    float *steps[kAdamGroup];
    int n;
};

__global__ void adam_advance_kernel(AdvanceArgs a) {
    if (threadIdx.x < static_cast<unsigned>(a.n)) *a.steps[threadIdx.x] = *a.steps[threadIdx.x] + 1.f;
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

hipError_t launch_adam(int n, float *const *params, const float *const *grads, float *const *exp_avgs,
                       float *const *exp_avg_sqs, const int64_t *numels, float *const *steps, double lr,
                       double beta1, double beta2, double eps, double weight_decay, int decoupled,
                       hipStream_t stream) {
    // Every group reads its counters before any is advanced. Counters are
    // distinct per tensor (the advance kernel adds one to each).
    for (int g0 = 0; g0 < n; g0 += kAdamGroup) {
        AdamArgs a{};
        a.n = n - g0 < kAdamGroup ? n - g0 : kAdamGroup;
        a.qstart[0] = 0;
        for (int k = 0; k < a.n; ++k) {
            const int j = g0 + k;
            a.p[k] = params[j];
            a.g[k] = grads[j];
            a.m[k] = exp_avgs[j];
            a.v[k] = exp_avg_sqs[j];
            a.steps[k] = steps[j];
            a.numel[k] = numels[j];
            a.qstart[k + 1] = a.qstart[k] + (numels[j] + 3) / 4;
            if (aligned16(params[j]) && aligned16(grads[j]) && aligned16(exp_avgs[j]) && aligned16(exp_avg_sqs[j]))
                a.vec_mask |= 1u << k;
        }
        for (int k = a.n; k < kAdamGroup; ++k) a.qstart[k + 1] = a.qstart[a.n];
        a.lr = lr;
        a.b1 = beta1;
        a.b2 = beta2;
        a.b2f = static_cast<float>(beta2);
        a.w1 = static_cast<float>(1.0 - beta1);
        a.w2 = static_cast<float>(1.0 - beta2);
        a.eps = static_cast<float>(eps);
        a.wd = static_cast<float>(weight_decay);
        a.decay = static_cast<float>(1.0 - lr * weight_decay);
        a.decoupled = decoupled;
        const int64_t total = a.qstart[a.n];
        if (total == 0) continue;
        int64_t blocks = (total + kAdamThreads * kAdamQuads - 1) / (kAdamThreads * kAdamQuads);
        if (blocks > kAdamMaxBlocks) blocks = kAdamMaxBlocks;
        hipLaunchKernelGGL(adam_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kAdamThreads), 0, stream, a);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    for (int g0 = 0; g0 < n; g0 += kAdamGroup) {
        AdvanceArgs a{};
        a.n = n - g0 < kAdamGroup ? n - g0 : kAdamGroup;
        for (int k = 0; k < a.n; ++k) a.steps[k] = steps[g0 + k];
        hipLaunchKernelGGL(adam_advance_kernel, dim3(1), dim3(64), 0, stream, a);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace tropnn
