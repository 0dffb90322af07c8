// Device-side helpers shared by the PairwiseLinear kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tropnn_hip.h"

namespace tropnn {

constexpr int kWave = 64;

template <typename T, int V>
using vec_t = T __attribute__((ext_vector_type(V)));

// Load V consecutive LUT elements (16 bytes at most) and widen them to f32.
// `p` must be aligned to V * sizeof(T); the host picks V so that every row
// start and every lane offset is.
template <typename T, int V>
__device__ __forceinline__ void load_row(const T *__restrict__ p, float (&d)[V]) {
    if constexpr (V == 1) {
        d[0] = static_cast<float>(*p);
    } else {
        const vec_t<T, V> v = *reinterpret_cast<const vec_t<T, V> *>(p);
#pragma unroll
        for (int i = 0; i < V; ++i) d[i] = static_cast<float>(v[i]);
    }
}

template <int V>
__device__ __forceinline__ void load_f32(const float *__restrict__ p, float (&d)[V]) {
    load_row<float, V>(p, d);
}

template <int V>
__device__ __forceinline__ void store_f32(float *__restrict__ p, const float (&d)[V]) {
    if constexpr (V == 1) {
        *p = d[0];
    } else {
        vec_t<float, V> v;
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = d[i];
        *reinterpret_cast<vec_t<float, V> *>(p) = v;
    }
}

// Non-temporal (streaming) store of V floats: for outputs that the kernel does
// not read again, so that they do not sit dirty in this XCD's L2 until the
// kernel-end write-back.
template <int V>
__device__ __forceinline__ void store_f32_nt(float *__restrict__ p, const float (&d)[V]) {
    if constexpr (V == 1) {
        __builtin_nontemporal_store(d[0], p);
    } else if constexpr (V <= 4) {
        vec_t<float, V> v;
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = d[i];
        __builtin_nontemporal_store(v, reinterpret_cast<vec_t<float, V> *>(p));
    } else {
#pragma unroll
        for (int q = 0; q < V / 4; ++q) {
            vec_t<float, 4> v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = d[4 * q + i];
            __builtin_nontemporal_store(v, reinterpret_cast<vec_t<float, 4> *>(p + 4 * q));
        }
    }
}

// Butterfly sum over the lanes whose ids differ only in bits [lo, hi).
// Every lane of a group ends with the group's total.
__device__ __forceinline__ float xor_sum(float v, int lo, int hi) {
    for (int m = lo; m < hi; m <<= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Cross-lane move inside a 16-lane DPP row (no LDS traffic).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of n consecutive lanes (n a power of two <= 64);
// every lane ends with its group's total, bit-identical across the group
// (each step adds a partner's partial, and IEEE addition commutes).
// Steps: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// row_half_mirror (pairs the two quads of a half row), row_mirror (pairs the
// two half rows), then cross-row shuffles (ds_bpermute) for 32 and 64.
__device__ __forceinline__ float group_sum(float v, int n) {
    if (n >= 2) v += dpp_mov<0xB1>(v);
    if (n >= 4) v += dpp_mov<0x4E>(v);
    if (n >= 8) v += dpp_mov<0x141>(v);
    if (n >= 16) v += dpp_mov<0x140>(v);
    if (n >= 32) v += __shfl_xor(v, 16, kWave);
    if (n >= 64) v += __shfl_xor(v, 32, kWave);
    return v;
}

// Preference order of torch.argmin over |margin|: a NaN beats any number
// (argmin propagates NaN), a smaller value beats a larger one, and ties go to
// the lower comparison index.
__device__ __forceinline__ bool min_margin_before(float mag_a, int idx_a, float mag_b, int idx_b) {
    const bool nan_a = mag_a != mag_a, nan_b = mag_b != mag_b;
    if (nan_a != nan_b) return nan_a;
    if (!nan_a && mag_a != mag_b) return mag_a < mag_b;
    return idx_a < idx_b;
}

// torch.sign: +1, -1, or 0 for zeros and NaN.
__device__ __forceinline__ float torch_sign(float u) { return u > 0.f ? 1.f : (u < 0.f ? -1.f : 0.f); }

// fast_sigmoid_odd surrogate, -0.5 * sign(u) / (1 + |u|)^2, in the reference's
// op order (layers/surrogate.py:16-17) so that each rounding step matches:
// scale the sign, add one to |u|, square, then one IEEE division.
__device__ __forceinline__ float fast_sigmoid_odd(float u) {
    const float num = -0.5f * torch_sign(u);
    const float base = 1.0f + fabsf(u);
    const float den = base * base;
    return num / den;
}

// izhikevich surrogate, sign * 2 * sig * (1 - sig) with sig = sigmoid(|u|)
// and sign = -1 for u > 0, else +1 (so u = 0 gives 0.5), in the reference's op
// order (layers/surrogate.py:9-13). The logistic is 1 / (1 + exp(-|u|)) with
// the device expf; the reference's vectorised CPU sigmoid may differ in the
// last bit.
__device__ __forceinline__ float izhikevich(float u) {
    const float sig = 1.0f / (1.0f + expf(-fabsf(u)));
    const float sign = u > 0.f ? -1.0f : 1.0f;
    return sign * 2.0f * sig * (1.0f - sig);
}

// The surrogate derivative selected by TROPNN_SURROGATE_* (wave-uniform).
__device__ __forceinline__ float surrogate_grad(float u, int surrogate) {
    return surrogate == TROPNN_SURROGATE_IZHIKEVICH ? izhikevich(u) : fast_sigmoid_odd(u);
}

// Buffer-resource access (raw buffers, 32-bit offsets). An offset at or past
// the resource's byte range reads as zero, so masked lanes just pass
// kOutOfRange instead of branching.
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// N elements of T (f32 or f16) per lane at byte offset voff + soff (soff
// wave-uniform), widened to f32. The loaded words are reinterpreted as whole
// vectors, never element by element.
template <typename T, int N>
__device__ __forceinline__ void buffer_row(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, int soff, float (&v)[N]) {
    constexpr int kBytes = N * static_cast<int>(sizeof(T));
    if constexpr (kBytes == 2) {
        const uint16_t w = __builtin_amdgcn_raw_buffer_load_b16(rsrc, voff, soff, 0);
        v[0] = static_cast<float>(__builtin_bit_cast(_Float16, w));
    } else if constexpr (kBytes == 4) {
        const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(rsrc, voff, soff, 0);
        if constexpr (N == 1) {
            v[0] = __builtin_bit_cast(float, w);
        } else {
            const vec_t<_Float16, 2> h = __builtin_bit_cast(vec_t<_Float16, 2>, w);
            v[0] = static_cast<float>(h[0]);
            v[1] = static_cast<float>(h[1]);
        }
    } else if constexpr (kBytes == 8) {
        const auto w = __builtin_amdgcn_raw_buffer_load_b64(rsrc, voff, soff, 0);
        if constexpr (N == 2) {
            const vec_t<float, 2> f = __builtin_bit_cast(vec_t<float, 2>, w);
            v[0] = f[0];
            v[1] = f[1];
        } else {
            const vec_t<_Float16, 4> h = __builtin_bit_cast(vec_t<_Float16, 4>, w);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = static_cast<float>(h[e]);
        }
    } else {
        static_assert(kBytes % 16 == 0, "row loads are 2, 4, 8 or a multiple of 16 bytes per lane");
#pragma unroll
        for (int q = 0; q < kBytes / 16; ++q) {
            const auto w = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff + 16u * q, soff, 0);
            if constexpr (sizeof(T) == 4) {
                const vec_t<float, 4> f = __builtin_bit_cast(vec_t<float, 4>, w);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * q + e] = f[e];
            } else {
                const vec_t<_Float16, 8> h = __builtin_bit_cast(vec_t<_Float16, 8>, w);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[8 * q + e] = static_cast<float>(h[e]);
            }
        }
    }
}

// The dispatcher deals the workgroups of a grid to the 8 XCDs in turn
// (workgroup i runs on XCD i % 8). This maps workgroup i of n to unit
// x * (n / 8) + min(x, n % 8) + i / 8, x = i % 8: a bijection on [0, n) that
// gives each XCD one contiguous block of units, so per-unit entries of a
// [*, n] array that share a cache line go through one XCD's L2 (lines are
// not split between XCDs).
__device__ __forceinline__ int xcd_block_unit(int i, int n) {
    const int x = i & 7, k = i >> 3, per = n >> 3, extra = n & 7;
    return x * per + min(x, extra) + k;
}

// acc + the binary16 value in the low (HI = false) or high half of w, widened
// to f32: one v_fma_mix_f32 computing half * 1.0 + acc with a single
// rounding, the same value as a conversion (exact) followed by an add, which
// take two instructions. hipcc turns fmaf(float(half), 1.0f, acc) back into
// the two, hence the inline assembly.
template <bool HI>
__device__ __forceinline__ float add_f16_mix(float acc, uint32_t w) {
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(w));
    else
        asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(w));
    return acc;
}

// N elements of T per lane at byte offset voff + soff as raw 32-bit words
// (W = N * sizeof(T) / 4, at least one; a 2-byte load fills the low half).
template <typename T, int N>
__device__ __forceinline__ void buffer_words(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, int soff,
                                             uint32_t (&w)[(N * sizeof(T) + 3) / 4]) {
    constexpr int kBytes = N * static_cast<int>(sizeof(T));
    if constexpr (kBytes == 2) {
        w[0] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, voff, soff, 0);
    } else if constexpr (kBytes == 4) {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, voff, soff, 0);
    } else {
        static_assert(kBytes == 8, "2, 4 or 8 bytes per lane");
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rsrc, voff, soff, 0);
        const vec_t<uint32_t, 2> u = __builtin_bit_cast(vec_t<uint32_t, 2>, v);
        w[0] = u[0];
        w[1] = u[1];
    }
}

// acc[e] += element e of a row chunk held as raw words (T = f32 or f16).
template <typename T, int N>
__device__ __forceinline__ void add_words(float (&acc)[N], const uint32_t (&w)[(N * sizeof(T) + 3) / 4]) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int e = 0; e < N; ++e) acc[e] += __builtin_bit_cast(float, w[e]);
    } else {
#pragma unroll
        for (int e = 0; e < N; ++e) acc[e] = (e & 1) ? add_f16_mix<true>(acc[e], w[e >> 1]) : add_f16_mix<false>(acc[e], w[e >> 1]);
    }
}

// floor(x / d) for 0 <= x < 2^21 and d >= 1, given inv_d = 1.0f / d: the
// fractional part of (x + 0.5) / d is at least 0.5 / d away from an integer,
// and the float reciprocal and product err by less than (x + 0.5) * 2^-22 / d,
// which is smaller for such x. Four instructions instead of an integer
// division's fifteen or so.
__device__ __forceinline__ int small_div(int x, float inv_d) {
    return static_cast<int>((static_cast<float>(x) + 0.5f) * inv_d);
}

// Clamp an anchor into [0, n) so a corrupt anchor can never address memory
// outside the staged input row; the host validates anchors before launch.
__device__ __forceinline__ int clamp_index(int64_t a, int n) {
    return (a >= 0 && a < n) ? static_cast<int>(a) : 0;
}

}  // namespace tropnn
