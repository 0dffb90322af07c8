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
// No float atomics anywhere (LDS float atomics serialise badly on gfx950, and
// fixed summation orders make every gradient deterministic). Two launches:
//  (1) table kernel, one workgroup per (table, output chunk). Items are taken
//      in tiles of blockDim items; each tile is counting-sorted by LUT row
//      code in LDS (per-wave ballot ranking, per-wave histograms, one scan),
//      which keeps item order inside a bucket. Each thread owns fixed
//      (row, column-slice) units of the table's gradient and accumulates its
//      bucket's grad rows in registers, so grad_lut is written exactly once.
//      The same pass forms the STE partial dot
//      sum_{o in chunk} g[o] * (L[nb,o] - L[code,o]) from the LDS LUT slab,
//      reduced over the row's lanes with DPP, into the workspace
//      [chunks][T][B].
//  (2) input kernel, two roles in one grid. Role A (item tiles): gu[b,t] =
//      D[b,t] * surrogate'(u) for the tile's items go to LDS; then one thread
//      per (item, input feature) walks that feature's entries of the inverse
//      anchor index (the (table, comparison, side) triples that read the
//      feature, in increasing order) and writes grad_latent directly. Role B
//      (one workgroup per table) reduces -gu per comparison over all items in
//      a fixed order and writes grad_thresholds.
//  A third, tiny kernel builds the inverse anchor index; callers rebuild it
//  only when the anchors change.
#include "device.hpp"
#include "launch.hpp"

namespace tropnn {
namespace {

constexpr int kLutThreads = 1024;
constexpr int kInThreads = 256;
constexpr int kBatch = 8;     // bucket items whose grad rows are loaded together
constexpr int kUnits = 4;     // max (row, slice) units per thread in the table kernel
constexpr int kPairs = 4;     // records per thread per batch in the input kernel

struct LutArgs {
    const float *grad_out;
    const void *lut;
    const uint64_t *rec;
    float scale;
    float *grad_lut;
    float *dpart;
    int items, out_f, tables, comps, rows, o_chunk, pitch, slices_log2;
    int hist_off, start_off, sorted_off;  // LDS byte offsets
};

__device__ __forceinline__ int rec_code(uint64_t r) { return static_cast<int>((r >> 32) & 0xffffu); }
__device__ __forceinline__ int rec_r(uint64_t r) { return static_cast<int>((r >> 48) & 0xffu); }
__device__ __forceinline__ float rec_u(uint64_t r) { return __builtin_bit_cast(float, static_cast<uint32_t>(r)); }

// Exclusive prefix sum over n <= 1024 ints in LDS, in place, by the first
// wave (serial across 64-wide chunks, shuffle scan inside a chunk).
__device__ void wave_exclusive_scan(int *v, int n, int lane) {
    int carry = 0;
    for (int base = 0; base < n; base += kWave) {
        const int k = base + lane;
        const int x = k < n ? v[k] : 0;
        int incl = x;
        for (int d = 1; d < kWave; d <<= 1) {
            const int y = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += y;
        }
        if (k < n) v[k] = carry + incl - x;
        carry += __shfl(incl, kWave - 1, kWave);
    }
    if (lane == 0) v[n] = carry;
}

template <typename T, int V>
__global__ __launch_bounds__(kLutThreads) void pairwise_bwd_table_kernel(LutArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    float *slab = reinterpret_cast<float *>(lds);                // [rows][pitch] LUT chunk as f32
    int *hist = reinterpret_cast<int *>(lds + a.hist_off);       // [waves][rows] counts, then bases
    int *start = reinterpret_cast<int *>(lds + a.start_off);     // [rows + 1] bucket starts
    uint32_t *sorted = reinterpret_cast<uint32_t *>(lds + a.sorted_off);  // [tile] item | nb << 16

    const int t = blockIdx.x, chunk = blockIdx.y;
    const int oc = a.o_chunk, pitch = a.pitch;
    const int o0 = chunk * oc;
    const int width = min(oc, a.out_f - o0);
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & (kWave - 1), wave = tid / kWave, nwaves = nthr / kWave;
    const int S = 1 << a.slices_log2;  // lanes per gradient row (one V-wide slice each)
    const int R = a.rows;
    const uint64_t *rec_t = a.rec + static_cast<size_t>(t) * a.items;
    float *dp_t = a.dpart ? a.dpart + (static_cast<size_t>(chunk) * a.tables + t) * a.items : nullptr;

    // stage the LUT slab [R x width] as f32
    {
        const T *src = static_cast<const T *>(a.lut) + static_cast<size_t>(t) * R * a.out_f + o0;
        const int vpr = width / V;  // width is a multiple of V
        for (int k = tid; k < R * vpr; k += nthr) {
            const int r = k / vpr, j = k - r * vpr;
            float v[V];
            load_row<T, V>(src + static_cast<size_t>(r) * a.out_f + j * V, v);
            store_f32<V>(slab + r * pitch + j * V, v);
        }
    }

    // this thread's (row, slice) units: unit = row * S + slice
    const int nunits = R * S;
    float acc[kUnits][V];
#pragma unroll
    for (int p = 0; p < kUnits; ++p)
#pragma unroll
        for (int e = 0; e < V; ++e) acc[p][e] = 0.f;

    for (int tile0 = 0; tile0 < a.items; tile0 += nthr) {
        // 1. this thread's item of the tile
        const int b = tile0 + tid;
        const bool valid = b < a.items;
        const uint64_t r0 = valid ? rec_t[b] : 0ull;
        const int code = rec_code(r0) & (R - 1);  // masks keep a corrupt record in range
        const int nb = (code ^ (1 << (rec_r(r0) & 15))) & (R - 1);
        for (int k = tid; k < nwaves * R; k += nthr) hist[k] = 0;
        // 2. rank among equal codes of the wave: intersect per-bit ballots
        uint64_t same = __ballot(valid);
        for (int c = 0; c < a.comps; ++c) {
            const uint64_t bits = __ballot(valid && ((code >> c) & 1));
            same &= ((code >> c) & 1) ? bits : ~bits;
        }
        const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
        const int rank = __popcll(same & below);
        __syncthreads();
        if (valid && rank == 0) hist[wave * R + code] = __popcll(same);
        __syncthreads();
        // 3. bucket starts, then per-wave bases inside each bucket
        for (int r = tid; r < R; r += nthr) {
            int run = 0;
            for (int w = 0; w < nwaves; ++w) {
                const int h = hist[w * R + r];
                hist[w * R + r] = run;
                run += h;
            }
            start[r] = run;  // bucket size for now
        }
        __syncthreads();
        if (wave == 0) wave_exclusive_scan(start, R, lane);
        __syncthreads();
        // 4. stable placement
        if (valid) sorted[start[code] + hist[wave * R + code] + rank] = static_cast<uint32_t>(tid) | (nb << 16);
        __syncthreads();
        // 5. owned units walk their buckets
#pragma unroll
        for (int p = 0; p < kUnits; ++p) {
            const int unit = tid + p * nthr;
            if (p * nthr >= nunits) break;  // block-uniform
            const bool own = unit < nunits;
            const int row = own ? unit >> a.slices_log2 : 0;
            const int slice = unit & (S - 1);
            const int col = slice * V;
            const bool live = own && col < width;
            const int kb = own ? start[row] : 0, ke = own ? start[row + 1] : 0;
            float lrow[V];
            load_f32<V>(slab + row * pitch + (live ? col : 0), lrow);
            const float *gcol = a.grad_out + o0 + (live ? col : 0);
            for (int k0 = kb; __ballot(k0 < ke) != 0; k0 += kBatch) {  // wave-uniform trip count
                uint32_t ent[kBatch];
                float g[kBatch][V];
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const int k = k0 + u;
                    ent[u] = (k < ke) ? sorted[k] : 0u;
                    const int item = tile0 + static_cast<int>(ent[u] & 0xffffu);
                    load_f32<V>(gcol + static_cast<size_t>(item < a.items ? item : 0) * a.out_f, g[u]);
                }
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const bool ok = (k0 + u < ke) && live;
                    const int nbr = static_cast<int>(ent[u] >> 16);
                    float d = 0.f;
                    if (ok) {
                        float ln[V];
                        load_f32<V>(slab + nbr * pitch + col, ln);
#pragma unroll
                        for (int e = 0; e < V; ++e) {
                            const float ge = g[u][e] * a.scale;
                            acc[p][e] += ge;
                            d += ge * (ln[e] - lrow[e]);
                        }
                    }
                    d = group_sum(d, S);
                    if (dp_t != nullptr && (k0 + u < ke) && own && slice == 0)
                        dp_t[tile0 + static_cast<int>(ent[u] & 0xffffu)] = d;
                }
            }
        }
        __syncthreads();  // LDS is reused by the next tile
    }

    // 6. each unit's gradient slice is written once
    if (a.grad_lut != nullptr) {
        float *dst = a.grad_lut + static_cast<size_t>(t) * R * a.out_f + o0;
#pragma unroll
        for (int p = 0; p < kUnits; ++p) {
            const int unit = tid + p * nthr;
            if (unit >= nunits) break;
            const int row = unit >> a.slices_log2, col = (unit & (S - 1)) * V;
            if (col < width) store_f32<V>(dst + static_cast<size_t>(row) * a.out_f + col, acc[p]);
        }
    }
}

struct InArgs {
    const uint64_t *rec;
    const float *dpart;
    const int32_t *index_offsets;  // [in_f + 1]
    const int32_t *index_entries;  // (t << 4) | (c << 1) | side
    float *grad_x;
    float *grad_thr;
    int items, in_f, tables, comps, chunks;
    int items_per_wg, role_a_blocks;
};

// D[b,t]: the chunk partial dots summed in chunk order
__device__ __forceinline__ float dot_of(const InArgs &a, int t, int b) {
    const size_t stride = static_cast<size_t>(a.tables) * a.items;
    const float *p = a.dpart + static_cast<size_t>(t) * a.items + b;
    float dsum = p[0];
    for (int k = 1; k < a.chunks; ++k) dsum += p[k * stride];
    return dsum;
}

__global__ __launch_bounds__(kInThreads) void pairwise_bwd_input_kernel(InArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x, nthr = blockDim.x;
    if (static_cast<int>(blockIdx.x) < a.role_a_blocks) {
        // role A: input gradient rows of items_per_wg items
        const int item0 = blockIdx.x * a.items_per_wg;
        const int n_items = min(a.items_per_wg, a.items - item0);
        const int npairs = n_items * a.tables;
        const int nent = 2 * a.tables * a.comps;
        int32_t *off_s = reinterpret_cast<int32_t *>(lds);            // [in_f + 1]
        int32_t *ent_s = off_s + (a.in_f + 1);                        // [2 T C]
        float *gu_s = reinterpret_cast<float *>(ent_s + nent);        // [n_items][T]
        uint8_t *r_s = reinterpret_cast<uint8_t *>(gu_s + a.items_per_wg * a.tables);  // [n_items][T]
        for (int k = tid; k <= a.in_f; k += nthr) off_s[k] = a.index_offsets[k];
        for (int k = tid; k < nent; k += nthr) ent_s[k] = a.index_entries[k];
        for (int p0 = tid; p0 < npairs; p0 += kPairs * nthr) {
            uint64_t rr[kPairs];
            float dsum[kPairs];
#pragma unroll
            for (int q = 0; q < kPairs; ++q) {
                int p = p0 + q * nthr;
                p = p < npairs ? p : npairs - 1;
                const int t = p / n_items, b = item0 + (p - t * n_items);
                rr[q] = a.rec[static_cast<size_t>(t) * a.items + b];
                dsum[q] = dot_of(a, t, b);
            }
#pragma unroll
            for (int q = 0; q < kPairs; ++q) {
                const int p = p0 + q * nthr;
                if (p < npairs) {
                    const int t = p / n_items, i = p - t * n_items;
                    gu_s[i * a.tables + t] = dsum[q] * fast_sigmoid_odd(rec_u(rr[q]));
                    r_s[i * a.tables + t] = static_cast<uint8_t>(rec_r(rr[q]));
                }
            }
        }
        __syncthreads();
        // one thread per (item, feature): walk the feature's anchor entries in order
        for (int k = tid; k < n_items * a.in_f; k += nthr) {
            const int i = k / a.in_f, f = k - i * a.in_f;
            const int e0 = off_s[f], e1 = off_s[f + 1];
            float g = 0.f;
            for (int e = e0; e < e1; ++e) {
                const int ent = ent_s[e];
                const int t = ent >> 4, c = (ent >> 1) & 7;
                if (r_s[i * a.tables + t] == c) {
                    const float gu = gu_s[i * a.tables + t];
                    g = (ent & 1) ? g - gu : g + gu;
                }
            }
            a.grad_x[static_cast<size_t>(item0 + i) * a.in_f + f] = g;
        }
        return;
    }
    // role B: threshold gradient of one table, fixed-order reduction
    const int t = blockIdx.x - a.role_a_blocks;
    float acc[TROPNN_MAX_COMPARISONS];
#pragma unroll
    for (int c = 0; c < TROPNN_MAX_COMPARISONS; ++c) acc[c] = 0.f;
    const uint64_t *rec_t = a.rec + static_cast<size_t>(t) * a.items;
    for (int b0 = tid; b0 < a.items; b0 += kPairs * nthr) {
        uint64_t rr[kPairs];
        float dsum[kPairs];
#pragma unroll
        for (int q = 0; q < kPairs; ++q) {
            int b = b0 + q * nthr;
            b = b < a.items ? b : a.items - 1;
            rr[q] = rec_t[b];
            dsum[q] = dot_of(a, t, b);
        }
#pragma unroll
        for (int q = 0; q < kPairs; ++q) {
            if (b0 + q * nthr < a.items) {
                const float gu = dsum[q] * fast_sigmoid_odd(rec_u(rr[q]));
                const int r = rec_r(rr[q]);
#pragma unroll
                for (int c = 0; c < TROPNN_MAX_COMPARISONS; ++c)
                    if (c == r) acc[c] -= gu;
            }
        }
    }
    float *part = reinterpret_cast<float *>(lds);  // [waves][MAX_COMPARISONS]
    const int lane = tid & (kWave - 1), wave = tid / kWave, nwaves = nthr / kWave;
#pragma unroll
    for (int c = 0; c < TROPNN_MAX_COMPARISONS; ++c) {
        const float v = group_sum(acc[c], kWave);
        if (lane == 0) part[wave * TROPNN_MAX_COMPARISONS + c] = v;
    }
    __syncthreads();
    if (tid < a.comps) {
        float sum = part[tid];
        for (int w = 1; w < nwaves; ++w) sum += part[w * TROPNN_MAX_COMPARISONS + tid];
        a.grad_thr[t * a.comps + tid] = sum;
    }
}

// Inverse anchor index: for every input feature f, the entries
// (t << 4) | (c << 1) | side of the anchors[t][c][side] equal to f, in
// increasing (t, c, side) order. One thread per feature scans the anchors,
// so the order is fixed.
__global__ __launch_bounds__(256) void anchor_index_kernel(const int64_t *anchors, int in_f, int tables, int comps,
                                                          int32_t *offsets, int32_t *entries) {
    extern __shared__ __align__(16) unsigned char lds[];
    int *count = reinterpret_cast<int *>(lds);  // [in_f + 1]
    const int n = tables * comps * 2;
    for (int f = threadIdx.x; f < in_f; f += blockDim.x) {
        int cnt = 0;
        for (int k = 0; k < n; ++k) cnt += anchors[k] == f;
        count[f] = cnt;
    }
    __syncthreads();
    if (threadIdx.x < kWave) wave_exclusive_scan(count, in_f, threadIdx.x);
    __syncthreads();
    for (int f = threadIdx.x; f <= in_f; f += blockDim.x) offsets[f] = count[f];
    for (int f = threadIdx.x; f < in_f; f += blockDim.x) {
        int pos = count[f];
        for (int k = 0; k < n; ++k)
            if (anchors[k] == f) entries[pos++] = (k >> 1) / comps << 4 | ((k >> 1) % comps) << 1 | (k & 1);
    }
}

template <typename T, int V>
hipError_t launch_table(const LutArgs &args, const BackwardPlan &p, hipStream_t stream) {
    const ArmedEvents ev = take_armed_events(TROPNN_KERNEL_BACKWARD_TABLE);
    record_event(ev.start, stream);
    hipLaunchKernelGGL((pairwise_bwd_table_kernel<T, V>), dim3(args.tables, p.o_chunks), dim3(p.lut_threads),
                       p.lut_lds_bytes, stream, args);
    const hipError_t e = hipGetLastError();
    record_event(ev.stop, stream);
    return e;
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

int table_lds_bytes(int rows, int pitch, int threads) {
    const int waves = threads / kWave;
    return rows * pitch * 4 + waves * rows * 4 + (rows + 1) * 4 + threads * 4 + 64;
}

}  // namespace

hipError_t launch_fill_zero(float *p, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p, n);
    return hipGetLastError();
}

hipError_t launch_anchor_index(const int64_t *anchors, int in_f, int tables, int comps, int32_t *offsets,
                               int32_t *entries, hipStream_t stream) {
    hipLaunchKernelGGL(anchor_index_kernel, dim3(1), dim3(256), (in_f + 1) * 4 + 64, stream, anchors, in_f, tables,
                       comps, offsets, entries);
    return hipGetLastError();
}

BackwardPlan plan_backward(const Dims &d) {
    BackwardPlan p{};
    const int esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    // one vector width for both the f32 grad rows and the LUT rows
    p.vec = 4;
    while (p.vec > 1 && (d.out_f % p.vec != 0 || (p.vec * esize) > 16)) p.vec >>= 1;
    p.lut_threads = kLutThreads;
    // widest chunk (<= 64 lanes x vec columns) whose slab + sort buffers fit
    // 64 KB of LDS and whose (row, slice) units fit kUnits per thread
    int oc = p.vec;
    while (oc * 2 <= kWave * p.vec && oc * 2 <= ((d.out_f + p.vec - 1) / p.vec) * p.vec * 2 &&
           table_lds_bytes(d.rows, oc * 2 + 4, p.lut_threads) <= 64 * 1024 &&
           d.rows * ((oc * 2) / p.vec) <= kUnits * p.lut_threads)
        oc *= 2;
    if (oc > d.out_f) oc = ((d.out_f + p.vec - 1) / p.vec) * p.vec;
    p.o_chunk = oc;
    p.o_chunks = (d.out_f + oc - 1) / oc;
    p.pitch = ((oc + 3) & ~3) + 4;  // +4 floats: rows start in different LDS banks
    p.slices_log2 = ilog2((oc + p.vec - 1) / p.vec);
    p.lut_lds_bytes = table_lds_bytes(d.rows, p.pitch, p.lut_threads);
    const int index_lds = (d.in_f + 1) * 4 + 2 * d.tables * d.comps * 4;
    int ipw = 4;
    while (ipw > 1 && index_lds + static_cast<long long>(ipw) * d.tables * 5 > 64 * 1024) ipw >>= 1;
    p.in_items_per_wg = ipw;
    p.in_threads = kInThreads;
    const int role_a_lds = index_lds + ipw * d.tables * 5 + 16;
    const int role_b_lds = (kInThreads / kWave) * TROPNN_MAX_COMPARISONS * 4;
    p.in_lds_bytes = role_a_lds > role_b_lds ? role_a_lds : role_b_lds;
    p.workspace_bytes = static_cast<size_t>(p.o_chunks) * d.tables * d.items * sizeof(float);
    return p;
}

hipError_t launch_backward(const Dims &d, const BackwardPlan &p, const float *grad_out, const void *lut,
                           const tropnn_route_record *rec, const int32_t *index_offsets,
                           const int32_t *index_entries, float scale, float *grad_x, float *grad_thr,
                           float *grad_lut, float *workspace, hipStream_t stream) {
    const bool need_dots = grad_x != nullptr || grad_thr != nullptr;
    const uint64_t *rec64 = reinterpret_cast<const uint64_t *>(rec);
    if (grad_lut != nullptr || need_dots) {
        LutArgs a{};
        a.grad_out = grad_out;
        a.lut = lut;
        a.rec = rec64;
        a.scale = scale;
        a.grad_lut = grad_lut;
        a.dpart = need_dots ? workspace : nullptr;
        a.items = d.items;
        a.out_f = d.out_f;
        a.tables = d.tables;
        a.comps = d.comps;
        a.rows = d.rows;
        a.o_chunk = p.o_chunk;
        a.pitch = p.pitch;
        a.slices_log2 = p.slices_log2;
        const int waves = p.lut_threads / kWave;
        a.hist_off = d.rows * p.pitch * 4;
        a.start_off = a.hist_off + waves * d.rows * 4;
        a.sorted_off = (a.start_off + (d.rows + 1) * 4 + 15) & ~15;
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
    b.rec = rec64;
    b.dpart = workspace;
    b.index_offsets = index_offsets;
    b.index_entries = index_entries;
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
    const ArmedEvents ev = take_armed_events(TROPNN_KERNEL_BACKWARD_INPUT);
    record_event(ev.start, stream);
    hipLaunchKernelGGL(pairwise_bwd_input_kernel, dim3(blocks), dim3(p.in_threads), p.in_lds_bytes, stream, b);
    const hipError_t e = hipGetLastError();
    record_event(ev.stop, stream);
    return e;
}

}  // namespace tropnn
