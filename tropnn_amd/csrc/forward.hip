// Fused PairwiseLinear forward for gfx950: comparator route -> LUT row gather
// summed over tables -> output scale, in one launch.
//
// Reference semantics (what each phase restates):
//   route   layers/pairwise.py:127-135, kernels/src/lut.zig:24-43
//   gather  layers/pairwise.py:99-125 (sum over tables of lut[t, code, :])
//   scale   layers/base.py:76-77
//   min-margin selection saved for the backward: layers/pairwise.py:138-140
//
// Workgroup = items_per_wg items x one output tile. The kernel is latency
// bound at small batch, so every phase issues all of its independent global
// loads before it waits:
//   1. each wave loads the anchors and thresholds of its first route ballots
//      while the workgroup stages the items' input rows in LDS (one round trip);
//   2. route: one wave ballot evaluates 64 / P tables (P lanes per table, one
//      comparison per lane, P = next power of two >= C); P-bit fields of the
//      ballot mask are the LUT row codes, written to LDS. Training also
//      reduces argmin |margin| inside each P-lane group and writes the route
//      record; the debug path writes int64 codes and f32 margins;
//   3. gather: lanes cover the output tile with 16-byte row loads (float4 or
//      8 x f16); the 64 / lanes_per_row sub-groups of a wave and the
//      waves_per_item waves of an item take disjoint strided sets of tables,
//      issuing up to 16 row loads per lane before the first add; partial sums
//      are combined by a lane butterfly and, across waves, through LDS in a
//      fixed order, then scaled and stored.
#include "device.hpp"
#include "launch.hpp"

namespace tropnn {
namespace {

struct FwdArgs {
    const float *x;
    const int64_t *anchors;
    const float *thr;
    const void *lut;
    float scale;
    float *out;
    tropnn_route_record *rec;
    int64_t *indices;
    float *margins;
    int items, in_f, out_f, tables, comps, rows;
    int lpt_log2, lpr_log2, o_tile, items_per_wg, waves_per_item;
    int codes_off, red_off;
};

constexpr int kGather = 16;   // row loads in flight per lane
constexpr int kBallots = 4;   // ballots whose parameters a wave prefetches

// One lane's comparator: anchors (clamped) and threshold of (table, comparison).
struct Comparator {
    int a, b;
    float thr;
    bool valid;
};

__device__ __forceinline__ Comparator load_comparator(const FwdArgs &p, int t, int c) {
    Comparator q{0, 0, 0.f, false};
    if (t < p.tables && c < p.comps) {
        const int64_t *ap = p.anchors + (static_cast<size_t>(t) * p.comps + c) * 2;
        q.a = clamp_index(ap[0], p.in_f);
        q.b = clamp_index(ap[1], p.in_f);
        q.thr = p.thr[t * p.comps + c];
        q.valid = true;
    }
    return q;
}

template <bool TRAIN, bool DEBUG>
__device__ __forceinline__ void route_ballot(const FwdArgs &p, const float *xs, uint16_t *codes, const Comparator &q,
                                             int t, int c, int slot, int lpt, int n_items, int item0) {
    const uint64_t field = (1ull << lpt) - 1ull;
    for (int i = 0; i < n_items; ++i) {  // wave-uniform
        float m = 0.f;
        if (q.valid) m = (xs[i * p.in_f + q.a] - xs[i * p.in_f + q.b]) - q.thr;
        const uint64_t mask = __ballot(q.valid && m > 0.f);
        const int code = static_cast<int>((mask >> (slot * lpt)) & field);
        const bool head = (c == 0) && (t < p.tables);
        const size_t b = static_cast<size_t>(item0 + i);
        if (head) codes[i * p.tables + t] = static_cast<uint16_t>(code);
        if constexpr (DEBUG) {
            if (p.margins != nullptr && q.valid) p.margins[(b * p.tables + t) * p.comps + c] = m;
            if (p.indices != nullptr && head) p.indices[b * p.tables + t] = code;
        }
        if constexpr (TRAIN) {
            // argmin |m| over the P lanes of this table; padding lanes
            // (c >= C) carry +inf and index 64 so they never win.
            float mag = q.valid ? fabsf(m) : __builtin_inff();
            int idx = q.valid ? c : kWave;
            float val = m;
            for (int s = 1; s < lpt; s <<= 1) {
                const float omag = __shfl_xor(mag, s, kWave);
                const int oidx = __shfl_xor(idx, s, kWave);
                const float oval = __shfl_xor(val, s, kWave);
                if (min_margin_before(omag, oidx, mag, idx)) {
                    mag = omag;
                    idx = oidx;
                    val = oval;
                }
            }
            if (head) {
                tropnn_route_record r;
                r.u = val;
                r.code = static_cast<uint16_t>(code);
                r.r = static_cast<uint8_t>(idx);
                r.reserved = 0;
                p.rec[static_cast<size_t>(t) * p.items + b] = r;
            }
        }
    }
}

template <typename T, int V, bool TRAIN, bool DEBUG>
__global__ __launch_bounds__(512) void pairwise_forward_kernel(FwdArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    float *xs = reinterpret_cast<float *>(lds);
    uint16_t *codes = reinterpret_cast<uint16_t *>(lds + a.codes_off);
    float *red = reinterpret_cast<float *>(lds + a.red_off);

    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & (kWave - 1), wave = tid / kWave, nwaves = nthr / kWave;
    const int item0 = blockIdx.x * a.items_per_wg;
    const int n_items = min(a.items_per_wg, a.items - item0);

    const int lpt = 1 << a.lpt_log2;
    const int tpb = kWave >> a.lpt_log2;
    const int nballot = (a.tables + tpb - 1) / tpb;
    const int slot = lane >> a.lpt_log2;
    const int c = lane & (lpt - 1);

    // 1. prefetch this wave's first ballots, stage the input rows
    Comparator pre[kBallots];
#pragma unroll
    for (int j = 0; j < kBallots; ++j) pre[j] = load_comparator(a, (wave + j * nwaves) * tpb + slot, c);
    {
        const float *src = a.x + static_cast<size_t>(item0) * a.in_f;
        const int n = n_items * a.in_f;
        if ((a.in_f & 3) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
            const int n4 = n >> 2;
            for (int k = tid; k < n4; k += nthr)
                reinterpret_cast<vec_t<float, 4> *>(xs)[k] = reinterpret_cast<const vec_t<float, 4> *>(src)[k];
        } else {
            for (int k = tid; k < n; k += nthr) xs[k] = src[k];
        }
    }
    __syncthreads();

    // 2. route
#pragma unroll
    for (int j = 0; j < kBallots; ++j) {
        const int kb = wave + j * nwaves;
        if (kb < nballot) route_ballot<TRAIN, DEBUG>(a, xs, codes, pre[j], kb * tpb + slot, c, slot, lpt, n_items, item0);
    }
    for (int kb = wave + kBallots * nwaves; kb < nballot; kb += nwaves) {  // many tables: rest of the ballots
        const Comparator q = load_comparator(a, kb * tpb + slot, c);
        route_ballot<TRAIN, DEBUG>(a, xs, codes, q, kb * tpb + slot, c, slot, lpt, n_items, item0);
    }
    __syncthreads();

    // 3. gather + sum over tables
    const int lpr = 1 << a.lpr_log2;
    const int sub = kWave >> a.lpr_log2;
    const int i = wave / a.waves_per_item;
    const int wi = wave - i * a.waves_per_item;
    const int sg = lane >> a.lpr_log2;
    const int l = lane & (lpr - 1);
    const int gid = wi * sub + sg;
    const int gpi = a.waves_per_item * sub;
    const int col = blockIdx.y * a.o_tile + l * V;
    const bool in_tile = (l * V < a.o_tile) && (col < a.out_f);
    const bool active = (i < n_items) && in_tile;

    float acc[V];
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = 0.f;

    if (active) {
        const T *lut = static_cast<const T *>(a.lut) + col;
        const uint16_t *my = codes + i * a.tables;
        const size_t row_stride = static_cast<size_t>(a.out_f);
        const size_t table_stride = static_cast<size_t>(a.rows) * a.out_f;
        for (int t0 = gid; t0 < a.tables; t0 += kGather * gpi) {
            float v[kGather][V];
#pragma unroll
            for (int u = 0; u < kGather; ++u) {
                const int tt = t0 + u * gpi;
                const bool ok = tt < a.tables;
                const int ts = ok ? tt : 0;  // masked lanes read row 0 of table 0
                load_row<T, V>(lut + ts * table_stride + (ok ? my[ts] : 0) * row_stride, v[u]);
                if (!ok) {
#pragma unroll
                    for (int e = 0; e < V; ++e) v[u][e] = 0.f;
                }
            }
#pragma unroll
            for (int u = 0; u < kGather; ++u)
#pragma unroll
                for (int e = 0; e < V; ++e) acc[e] += v[u][e];
        }
    }

    // combine the sub-groups of the wave (lanes that differ in bits >= lpr)
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = xor_sum(acc[e], lpr, kWave);

    if (a.waves_per_item > 1) {
        if (sg == 0 && in_tile && wi > 0) {
            float *dst = red + ((i * a.waves_per_item + wi) * a.o_tile) + l * V;
#pragma unroll
            for (int e = 0; e < V; ++e) dst[e] = acc[e];
        }
        __syncthreads();
        if (wi == 0 && sg == 0 && active) {
            for (int w = 1; w < a.waves_per_item; ++w) {
                const float *src = red + ((i * a.waves_per_item + w) * a.o_tile) + l * V;
#pragma unroll
                for (int e = 0; e < V; ++e) acc[e] += src[e];
            }
        }
    }

    if (wi == 0 && sg == 0 && active) {
        float y[V];
#pragma unroll
        for (int e = 0; e < V; ++e) y[e] = acc[e] * a.scale;
        store_f32<V>(a.out + static_cast<size_t>(item0 + i) * a.out_f + col, y);
    }
}

template <typename T, int V>
hipError_t launch_typed(const FwdArgs &args, const ForwardPlan &p, bool train, bool debug, hipStream_t stream) {
    const dim3 grid(p.blocks, p.o_tiles), block(p.threads);
    const ArmedEvents ev = take_armed_events(TROPNN_KERNEL_FORWARD);
    record_event(ev.start, stream);
    if (train && debug)
        hipLaunchKernelGGL((pairwise_forward_kernel<T, V, true, true>), grid, block, p.lds_bytes, stream, args);
    else if (train)
        hipLaunchKernelGGL((pairwise_forward_kernel<T, V, true, false>), grid, block, p.lds_bytes, stream, args);
    else if (debug)
        hipLaunchKernelGGL((pairwise_forward_kernel<T, V, false, true>), grid, block, p.lds_bytes, stream, args);
    else
        hipLaunchKernelGGL((pairwise_forward_kernel<T, V, false, false>), grid, block, p.lds_bytes, stream, args);
    const hipError_t e = hipGetLastError();
    record_event(ev.stop, stream);
    return e;
}

int ilog2(int v) {
    int r = 0;
    while ((1 << r) < v) ++r;
    return r;
}

}  // namespace

ForwardPlan plan_forward(const Dims &d) {
    ForwardPlan p{};
    const int esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    // widest load (<= 16 bytes) that divides a row, so every row start and
    // every lane offset stays aligned
    p.vec = 16 / esize;
    while (p.vec > 1 && d.out_f % p.vec != 0) p.vec >>= 1;
    p.lpt_log2 = ilog2(d.comps);
    const int lanes_needed = (d.out_f + p.vec - 1) / p.vec;
    const int lanes = lanes_needed < kWave ? lanes_needed : kWave;
    p.lpr_log2 = ilog2(lanes);
    p.o_tile = (1 << p.lpr_log2) * p.vec;
    if (p.o_tile > d.out_f) p.o_tile = d.out_f;
    p.o_tiles = (d.out_f + p.o_tile - 1) / p.o_tile;
    const int sub = kWave >> p.lpr_log2;

    // Aim for ~4096 waves (256 CUs x 16): split an item's tables over several
    // waves only when items x tiles alone cannot fill the chip.
    const long long units = static_cast<long long>(d.items) * p.o_tiles;
    int wpi = 1;
    while (wpi < 8 && units * wpi < 4096 && static_cast<long long>(wpi) * 2 * sub <= d.tables) wpi <<= 1;
    int ipw = 8 / wpi;
    // keep the staged input rows within 32 KB of LDS
    while (ipw > 1 && static_cast<long long>(ipw) * d.in_f * 4 > 32 * 1024) ipw >>= 1;
    if (ipw > d.items) ipw = d.items < 1 ? 1 : d.items;
    p.waves_per_item = wpi;
    p.items_per_wg = ipw;
    p.threads = ipw * wpi * kWave;
    p.blocks = (d.items + ipw - 1) / ipw;

    int off = ipw * d.in_f * 4;
    off = (off + 15) & ~15;
    p.codes_off = off;
    off += ipw * d.tables * 2;
    off = (off + 15) & ~15;
    p.red_off = off;
    if (wpi > 1) off += ipw * wpi * p.o_tile * 4;
    p.lds_bytes = off;
    return p;
}

hipError_t launch_forward(const Dims &d, const ForwardPlan &p, const float *x, const int64_t *anchors,
                          const float *thr, const void *lut, float scale, float *out, tropnn_route_record *rec,
                          int64_t *indices, float *margins, hipStream_t stream) {
    FwdArgs a{};
    a.x = x;
    a.anchors = anchors;
    a.thr = thr;
    a.lut = lut;
    a.scale = scale;
    a.out = out;
    a.rec = rec;
    a.indices = indices;
    a.margins = margins;
    a.items = d.items;
    a.in_f = d.in_f;
    a.out_f = d.out_f;
    a.tables = d.tables;
    a.comps = d.comps;
    a.rows = d.rows;
    a.lpt_log2 = p.lpt_log2;
    a.lpr_log2 = p.lpr_log2;
    a.o_tile = p.o_tile;
    a.items_per_wg = p.items_per_wg;
    a.waves_per_item = p.waves_per_item;
    a.codes_off = p.codes_off;
    a.red_off = p.red_off;
    const bool train = rec != nullptr;
    const bool debug = indices != nullptr || margins != nullptr;
    if (d.lut_dtype == TROPNN_LUT_F16) {
        switch (p.vec) {
            case 8: return launch_typed<_Float16, 8>(a, p, train, debug, stream);
            case 4: return launch_typed<_Float16, 4>(a, p, train, debug, stream);
            case 2: return launch_typed<_Float16, 2>(a, p, train, debug, stream);
            default: return launch_typed<_Float16, 1>(a, p, train, debug, stream);
        }
    }
    switch (p.vec) {
        case 4: return launch_typed<float, 4>(a, p, train, debug, stream);
        case 2: return launch_typed<float, 2>(a, p, train, debug, stream);
        default: return launch_typed<float, 1>(a, p, train, debug, stream);
    }
}

}  // namespace tropnn
