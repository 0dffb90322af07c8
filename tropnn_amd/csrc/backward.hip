// PairwiseLinear backward for gfx950 (min-margin STE, fast_sigmoid_odd).
//
// Reference semantics: the autograd of the torch path,
//   LUT gradient     index_select backward of layers/pairwise.py:119
//   STE dot          mul/sum backward of layers/pairwise.py:164-165
//   surrogate        layers/surrogate.py:16-17, 36-38
//   input/threshold  gather + sub + advanced-index backward of
//                    layers/pairwise.py:131-133, 139
// with g = output_scale * grad_output (layers/base.py:76-77).
//
// Two launches:
//  (1) table kernel, one workgroup per (table, output chunk): the table's LUT
//      slab [R x chunk] is staged in LDS once; the items' route records and
//      grad rows stream through; each item adds g into its code's row of an
//      LDS gradient slab (LDS float atomics, no global atomics) and forms its
//      partial STE dot sum_o g * (L[nb] - L[code]) from LDS. The slab is
//      written to grad_lut once (no memset needed) and the partial dots go to
//      the workspace [chunks][T][B].
//  (2) input kernel, two roles in one grid: role A (one workgroup per
//      item_tile) sums the chunk partials into D, applies the surrogate and
//      accumulates +-gu at the two anchors of the selected comparison into an
//      LDS input-gradient row, then writes grad_latent once; role B (one
//      workgroup per table) reduces -gu per comparison over all items in a
//      fixed order and writes grad_thresholds directly.
#include "device.hpp"
#include "launch.hpp"

namespace tropnn {
namespace {

constexpr int kLutThreads = 256;
constexpr int kInThreads = 256;
constexpr int kItemUnroll = 4;

struct LutArgs {
    const float *grad_out;
    const void *lut;
    const tropnn_route_record *rec;
    float scale;
    float *grad_lut;
    float *dpart;
    int items, out_f, tables, rows, o_chunk, lpr_log2;
};

__device__ __forceinline__ void lds_add(float *p, float v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <typename T, int V>
__global__ __launch_bounds__(kLutThreads) void pairwise_bwd_table_kernel(LutArgs a) {
    extern __shared__ __align__(16) float lds_f[];
    const int oc = a.o_chunk;
    float *slab = lds_f;                  // [rows][oc] LUT values as f32
    float *grad = lds_f + a.rows * oc;    // [rows][oc] gradient accumulator

    const int t = blockIdx.x, chunk = blockIdx.y;
    const int o0 = chunk * oc;
    const int width = min(oc, a.out_f - o0);
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & (kWave - 1), wave = tid / kWave, nwaves = nthr / kWave;

    // 1. stage the LUT slab, clear the gradient slab
    {
        const T *src = static_cast<const T *>(a.lut) + static_cast<size_t>(t) * a.rows * a.out_f + o0;
        const int vpr = width / V;  // vectors per row (width is a multiple of V)
        for (int k = tid; k < a.rows * vpr; k += nthr) {
            const int r = k / vpr, j = k - r * vpr;
            float v[V];
            load_row<T, V>(src + static_cast<size_t>(r) * a.out_f + j * V, v);
#pragma unroll
            for (int e = 0; e < V; ++e) {
                slab[r * oc + j * V + e] = v[e];
                grad[r * oc + j * V + e] = 0.f;
            }
        }
    }
    __syncthreads();

    // 2. stream the items: sub-group = lanes_per_row lanes covering the chunk
    const int lpr = 1 << a.lpr_log2;
    const int sub = kWave >> a.lpr_log2;
    const int sg = lane >> a.lpr_log2, l = lane & (lpr - 1);
    const int nsg = nwaves * sub;
    const int col = l * V;
    const bool in_chunk = col < width;
    const tropnn_route_record *rec_t = a.rec + static_cast<size_t>(t) * a.items;
    float *dp_t = a.dpart ? a.dpart + (static_cast<size_t>(chunk) * a.tables + t) * a.items : nullptr;

    // wave-uniform trip count: every lane runs every iteration, invalid ones masked
    for (int base = wave * sub; base < a.items; base += nsg * kItemUnroll) {
        int b[kItemUnroll];
        bool ok[kItemUnroll];
        tropnn_route_record rr[kItemUnroll] = {};
        float g[kItemUnroll][V];
#pragma unroll
        for (int u = 0; u < kItemUnroll; ++u) {
            b[u] = base + u * nsg + sg;
            ok[u] = b[u] < a.items;
            if (ok[u]) rr[u] = rec_t[b[u]];
            if (ok[u] && in_chunk) {
                load_f32<V>(a.grad_out + static_cast<size_t>(b[u]) * a.out_f + o0 + col, g[u]);
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) g[u][e] = 0.f;
            }
        }
#pragma unroll
        for (int u = 0; u < kItemUnroll; ++u) {
            float d = 0.f;
            if (ok[u] && in_chunk) {
                // masks keep a corrupt record inside the slab
                const int code = rr[u].code & (a.rows - 1);
                const int nb = (code ^ (1 << (rr[u].r & 15))) & (a.rows - 1);
                const float *cur = slab + code * oc + col;
                const float *nbr = slab + nb * oc + col;
                float *acc = grad + code * oc + col;
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const float ge = g[u][e] * a.scale;
                    const float diff = nbr[e] - cur[e];
                    d += ge * diff;
                    lds_add(acc + e, ge);
                }
            }
            d = xor_sum(d, 1, lpr);
            if (dp_t != nullptr && ok[u] && l == 0) dp_t[b[u]] = d;
        }
    }
    __syncthreads();

    // 3. write the gradient slab once
    if (a.grad_lut != nullptr) {
        float *dst = a.grad_lut + static_cast<size_t>(t) * a.rows * a.out_f + o0;
        const int vpr = width / V;
        for (int k = tid; k < a.rows * vpr; k += nthr) {
            const int r = k / vpr, j = k - r * vpr;
            float v[V];
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] = grad[r * oc + j * V + e];
            store_f32<V>(dst + static_cast<size_t>(r) * a.out_f + j * V, v);
        }
    }
}

struct InArgs {
    const int64_t *anchors;
    const tropnn_route_record *rec;
    const float *dpart;
    float *grad_x;
    float *grad_thr;
    int items, in_f, tables, comps, chunks;
    int items_per_wg, role_a_blocks;
};

// gu[b,t] = (sum over chunks of the partial dots, in chunk order) * surrogate'(u)
__device__ __forceinline__ float input_grad_of(const InArgs &a, int t, int b, float u) {
    const size_t stride = static_cast<size_t>(a.tables) * a.items;
    const float *p = a.dpart + static_cast<size_t>(t) * a.items + b;
    float dsum = p[0];
    for (int k = 1; k < a.chunks; ++k) dsum += p[k * stride];
    return dsum * fast_sigmoid_odd(u);
}

__global__ __launch_bounds__(kInThreads) void pairwise_bwd_input_kernel(InArgs a) {
    extern __shared__ __align__(16) float lds_f[];
    const int tid = threadIdx.x, nthr = blockDim.x;
    if (static_cast<int>(blockIdx.x) < a.role_a_blocks) {
        // role A: input gradient rows of items_per_wg items
        const int item0 = blockIdx.x * a.items_per_wg;
        const int n_items = min(a.items_per_wg, a.items - item0);
        float *gx = lds_f;  // [n_items][in_f]
        for (int k = tid; k < n_items * a.in_f; k += nthr) gx[k] = 0.f;
        __syncthreads();
        // consecutive threads take consecutive items of one table: coalesced records
        for (int p = tid; p < n_items * a.tables; p += nthr) {
            const int t = p / n_items, i = p - t * n_items;
            const int b = item0 + i;
            const tropnn_route_record r = a.rec[static_cast<size_t>(t) * a.items + b];
            const float gu = input_grad_of(a, t, b, r.u);
            const int rsel = r.r < a.comps ? r.r : 0;  // keeps a corrupt record in bounds
            const int64_t *ap = a.anchors + (static_cast<size_t>(t) * a.comps + rsel) * 2;
            lds_add(gx + i * a.in_f + clamp_index(ap[0], a.in_f), gu);
            lds_add(gx + i * a.in_f + clamp_index(ap[1], a.in_f), -gu);
        }
        __syncthreads();
        float *dst = a.grad_x + static_cast<size_t>(item0) * a.in_f;
        for (int k = tid; k < n_items * a.in_f; k += nthr) dst[k] = gx[k];
        return;
    }
    // role B: threshold gradient of one table, fixed-order reduction
    const int t = blockIdx.x - a.role_a_blocks;
    float acc[TROPNN_MAX_COMPARISONS];
#pragma unroll
    for (int c = 0; c < TROPNN_MAX_COMPARISONS; ++c) acc[c] = 0.f;
    for (int b = tid; b < a.items; b += nthr) {
        const tropnn_route_record r = a.rec[static_cast<size_t>(t) * a.items + b];
        const float gu = input_grad_of(a, t, b, r.u);
#pragma unroll
        for (int c = 0; c < TROPNN_MAX_COMPARISONS; ++c)
            if (c == r.r) acc[c] -= gu;
    }
    float *part = lds_f;  // [waves][MAX_COMPARISONS]
    const int lane = tid & (kWave - 1), wave = tid / kWave, nwaves = nthr / kWave;
#pragma unroll
    for (int c = 0; c < TROPNN_MAX_COMPARISONS; ++c) {
        const float v = xor_sum(acc[c], 1, kWave);
        if (lane == 0) part[wave * TROPNN_MAX_COMPARISONS + c] = v;
    }
    __syncthreads();
    if (tid < a.comps) {
        float s = part[tid];
        for (int w = 1; w < nwaves; ++w) s += part[w * TROPNN_MAX_COMPARISONS + tid];
        a.grad_thr[t * a.comps + tid] = s;
    }
}

template <typename T, int V>
hipError_t launch_table(const LutArgs &args, const BackwardPlan &p, hipStream_t stream) {
    hipLaunchKernelGGL((pairwise_bwd_table_kernel<T, V>), dim3(args.tables, p.o_chunks), dim3(p.lut_threads),
                       p.lut_lds_bytes, stream, args);
    return hipGetLastError();
}

int ilog2(int v) {
    int r = 0;
    while ((1 << r) < v) ++r;
    return r;
}

__global__ void fill_zero_kernel(float *p, size_t n) {
    for (size_t k = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; k < n;
         k += static_cast<size_t>(gridDim.x) * blockDim.x)
        p[k] = 0.f;
}

}  // namespace

hipError_t launch_fill_zero(float *p, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p, n);
    return hipGetLastError();
}

BackwardPlan plan_backward(const Dims &d) {
    BackwardPlan p{};
    const int esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    // one vector width for both the f32 grad rows and the LUT rows
    p.vec = 4;
    while (p.vec > 1 && (d.out_f % p.vec != 0 || (p.vec * esize) > 16)) p.vec >>= 1;
    // slab + gradient slab (both f32) within 64 KB of LDS
    const int max_cols = (64 * 1024) / (8 * d.rows);
    int oc = 1;
    while (oc * 2 <= max_cols && oc * 2 <= kWave * p.vec) oc *= 2;
    if (oc > d.out_f) oc = d.out_f;
    if (oc % p.vec != 0) oc = (oc / p.vec) * p.vec;
    if (oc < p.vec) oc = p.vec;
    // split further while the grid has fewer than 256 workgroups
    while (static_cast<long long>(d.tables) * ((d.out_f + oc - 1) / oc) < 256 && oc >= 8 * p.vec &&
           (oc / 2) % p.vec == 0)
        oc /= 2;
    p.o_chunk = oc;
    p.o_chunks = (d.out_f + oc - 1) / oc;
    p.lpr_log2 = ilog2((oc + p.vec - 1) / p.vec);
    p.lut_threads = kLutThreads;
    p.lut_lds_bytes = 8 * d.rows * oc;
    int ipw = 8;
    while (ipw > 1 && static_cast<long long>(ipw) * d.in_f * 4 > 32 * 1024) ipw >>= 1;
    p.in_items_per_wg = ipw;
    p.in_threads = kInThreads;
    const int role_a_lds = ipw * d.in_f * 4;
    const int role_b_lds = (kInThreads / kWave) * TROPNN_MAX_COMPARISONS * 4;
    p.in_lds_bytes = role_a_lds > role_b_lds ? role_a_lds : role_b_lds;
    p.workspace_bytes = static_cast<size_t>(p.o_chunks) * d.tables * d.items * sizeof(float);
    return p;
}

hipError_t launch_backward(const Dims &d, const BackwardPlan &p, const float *grad_out, const int64_t *anchors,
                           const void *lut, const tropnn_route_record *rec, float scale, float *grad_x,
                           float *grad_thr, float *grad_lut, float *workspace, hipStream_t stream) {
    const bool need_dots = grad_x != nullptr || grad_thr != nullptr;
    if (grad_lut != nullptr || need_dots) {
        LutArgs a{};
        a.grad_out = grad_out;
        a.lut = lut;
        a.rec = rec;
        a.scale = scale;
        a.grad_lut = grad_lut;
        a.dpart = need_dots ? workspace : nullptr;
        a.items = d.items;
        a.out_f = d.out_f;
        a.tables = d.tables;
        a.rows = d.rows;
        a.o_chunk = p.o_chunk;
        a.lpr_log2 = p.lpr_log2;
        hipError_t e;
        if (d.lut_dtype == TROPNN_LUT_F16) {
            switch (p.vec) {
                case 4: e = launch_table<_Float16, 4>(a, p, stream); break;
                case 2: e = launch_table<_Float16, 2>(a, p, stream); break;
                default: e = launch_table<_Float16, 1>(a, p, stream); break;
            }
        } else {
            switch (p.vec) {
                case 4: e = launch_table<float, 4>(a, p, stream); break;
                case 2: e = launch_table<float, 2>(a, p, stream); break;
                default: e = launch_table<float, 1>(a, p, stream); break;
            }
        }
        if (e != hipSuccess) return e;
    }
    if (!need_dots) return hipSuccess;
    InArgs b{};
    b.anchors = anchors;
    b.rec = rec;
    b.dpart = workspace;
    b.grad_x = grad_x;
    b.grad_thr = grad_thr;
    b.items = d.items;
    b.in_f = d.in_f;
    b.tables = d.tables;
    b.comps = d.comps;
    b.chunks = p.o_chunks;
    b.items_per_wg = p.in_items_per_wg;
    b.role_a_blocks = grad_x != nullptr ? (d.items + p.in_items_per_wg - 1) / p.in_items_per_wg : 0;
    const int blocks = b.role_a_blocks + (grad_thr != nullptr ? d.tables : 0);
    hipLaunchKernelGGL(pairwise_bwd_input_kernel, dim3(blocks), dim3(p.in_threads), p.in_lds_bytes, stream, b);
    return hipGetLastError();
}

}  // namespace tropnn
