// Fused PairwiseLinear forward for gfx950: comparator route -> LUT row gather
// summed over tables -> output scale, in one launch.
//
// Reference semantics (what each phase restates):
//   route   layers/pairwise.py:127-135, kernels/src/lut.zig:24-43
//   gather  layers/pairwise.py:99-125 (sum over tables of lut[t, code, :])
//   scale   layers/base.py:76-77
//   min-margin selection saved for the backward: layers/pairwise.py:138-140
//
// Workgroup = one item x one output tile of 64 * N columns; its W waves take
// disjoint contiguous blocks of tables. The kernel is latency bound at the
// batch sizes of interest, so each wave keeps its instruction count small and
// issues every independent load before it waits:
//   1. each wave loads the comparators of its first ballots while the
//      workgroup stages the item's input row in LDS (one round trip; a row
//      too wide for LDS is read from global memory by the route instead);
//   2. route: one wave ballot evaluates 64 / P of the wave's tables (P lanes
//      per table, one comparison per lane, P = next power of two >= C); the
//      P-bit fields of the ballot mask are the LUT row codes, which the table's
//      first lane writes to the wave's own LDS code list. Training also picks
//      argmin |margin| inside each P-lane group with DPP moves on a 64-bit key
//      and the winning lane writes the route record; the debug path writes
//      uint8 codes (one coalesced store per wave from the code list), int64
//      codes and f32 margins, from the first column tile only;
//   3. gather: the wave reads its codes back 16 at a time (one broadcast LDS
//      read), moves them to scalar registers, and loads each table's row with
//      one buffer load whose row offset is a scalar: lane l reads columns
//      [l N, l N + N) of the tile. Lanes past the last column get an offset
//      beyond the buffer range, which the buffer unit answers with zeros, so
//      the loop carries no masks. All of a chunk's row loads are in flight
//      before the first add;
//   4. the waves' partial rows are summed through LDS in wave order, scaled
//      and stored by wave 0.
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
    uint64_t *rec;
    int64_t *indices;
    float *margins;
    uint8_t *codes;
    uint32_t lut_bytes;  // buffer range of the LUT (<= 2^31)
    int items, in_f, out_f, tables, comps;
    int row_bytes, table_bytes;
    int lpt_log2, per_wave, codes_pitch;
    int codes_off, red_off;
    int wave_lpr_log2, wave_tile_bytes, wave_x_off;  // wave-item kernel
};

// Ballots whose comparators a wave prefetches: two cover 16 tables of up to
// 8 comparisons, every wave of the configurations of interest; further
// ballots load their comparators in turn. (Four prefetch slots made the c2
// forward ~0.4 us slower for the registers and code they take.)
constexpr int kBallots = 2;

// One lane's comparator: anchors (clamped) and threshold of (table, comparison).
// Padding lanes load table 0 / comparison 0 so that the loads are issued
// unconditionally; `valid` masks them out.
struct Comparator {
    int a, b;
    float thr;
    bool valid;
};

__device__ __forceinline__ Comparator load_comparator(const FwdArgs &p, int t, int t_end, int c) {
    Comparator q;
    q.valid = t < t_end && c < p.comps;
    const size_t k = q.valid ? static_cast<size_t>(t) * p.comps + c : 0;
    q.a = clamp_index(p.anchors[2 * k], p.in_f);
    q.b = clamp_index(p.anchors[2 * k + 1], p.in_f);
    q.thr = p.thr[k];
    return q;
}

// One DPP step of the min-margin argmin: the smaller key of this lane and
// its CTRL partner.
template <int CTRL>
__device__ __forceinline__ uint32_t key_min_step(uint32_t key) {
    const uint32_t other = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(key), CTRL, 0xF, 0xF, false));
    return other < key ? other : key;
}

// Route record of a table, held by the lane that wins its min-margin pick.
struct RouteOut {
    uint64_t rec;
    bool win;
};

template <bool TRAIN, bool DEBUG>
__device__ __forceinline__ RouteOut route_ballot(const FwdArgs &p, const float *xs, uint8_t *my_codes,
                                                 const Comparator &q, int t, int j, int c, int slot, int item) {
    const float m = (xs[q.a] - xs[q.b]) - q.thr;
    const uint64_t mask = __ballot(q.valid && m > 0.f);
    const int code = static_cast<int>((mask >> (slot << p.lpt_log2)) & ((1ull << p.comps) - 1ull));
    const bool head = q.valid && c == 0;
    if (head) my_codes[j] = static_cast<uint8_t>(code);
    if constexpr (DEBUG) {
        const size_t bt = static_cast<size_t>(item) * p.tables + t;
        if (blockIdx.y == 0) {
            if (p.margins != nullptr && q.valid) p.margins[bt * p.comps + c] = m;
            if (p.indices != nullptr && head) p.indices[bt] = code;
        }
    }
    RouteOut r{0ull, false};
    if constexpr (TRAIN) {
        // torch.argmin over |m|: NaN first, then the smaller magnitude, then
        // the lower comparison index. Key = 0 for NaN else bits(|m|) + 1
        // (below 2^31 + 2); padding lanes carry the largest key. The group's
        // smallest key by a DPP butterfly, then the lowest lane holding it
        // (the lowest comparison index) wins.
        const float mag = fabsf(m);
        const uint32_t key = q.valid ? (mag != mag ? 0u : __builtin_bit_cast(uint32_t, mag) + 1u) : 0xFFFFFFFFu;
        uint32_t mn = key;
        const int lpt = 1 << p.lpt_log2;   // wave-uniform
        if (lpt >= 2) mn = key_min_step<0xB1>(mn);   // quad_perm [1,0,3,2]
        if (lpt >= 4) mn = key_min_step<0x4E>(mn);   // quad_perm [2,3,0,1]
        if (lpt >= 8) mn = key_min_step<0x141>(mn);  // row_half_mirror
        const uint64_t holders = __ballot(key == mn);  // lanes holding their group's smallest key
        const uint32_t before = static_cast<uint32_t>(holders >> (slot << p.lpt_log2)) & ((1u << c) - 1u);
        r.win = q.valid && key == mn && before == 0u;
        r.rec = static_cast<uint64_t>(__builtin_bit_cast(uint32_t, m)) | (static_cast<uint64_t>(code) << 32) |
                (static_cast<uint64_t>(c) << 48);
    }
    return r;
}

// XG (inputs too wide for LDS): the route reads the item's input row from
// global memory instead of the LDS copy, and the LDS holds the code lists and
// partial rows only. Same arithmetic, same outputs.
template <typename T, int N, bool TRAIN, bool DEBUG, bool XG>
__global__ __launch_bounds__(1024) void pairwise_forward_kernel(FwdArgs a) {
    constexpr int kG = gather_chunk(static_cast<int>(sizeof(T)), N);
    extern __shared__ __align__(16) unsigned char lds[];
    float *red = reinterpret_cast<float *>(lds + a.red_off);

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nwaves = blockDim.x >> 6;
    const int item = xcd_block_unit(blockIdx.x, gridDim.x);  // route records of adjacent items share lines
    uint8_t *my_codes = lds + a.codes_off + wave * a.codes_pitch;
    const float *xrow = a.x + static_cast<size_t>(item) * a.in_f;
    float *xl = reinterpret_cast<float *>(lds);
    const float *xs = XG ? xrow : xl;

    const int tpb = kWave >> a.lpt_log2;
    const int slot = lane >> a.lpt_log2;
    const int c = lane & ((1 << a.lpt_log2) - 1);
    const int t_begin = wave * a.per_wave;
    const int t_end = min(a.tables, t_begin + a.per_wave);
    const int n_t = max(0, t_end - t_begin);
    const int nballot = (n_t + tpb - 1) / tpb;

    // 1. prefetch this wave's first ballots, stage the input row
    Comparator pre[kBallots];
#pragma unroll
    for (int j = 0; j < kBallots; ++j) pre[j] = load_comparator(a, t_begin + j * tpb + slot, t_end, c);
    if constexpr (!XG) {
        if ((a.in_f & 3) == 0 && (reinterpret_cast<uintptr_t>(xrow) & 15) == 0) {
            for (int k = tid; k < (a.in_f >> 2); k += blockDim.x)
                reinterpret_cast<vec_t<float, 4> *>(xl)[k] = reinterpret_cast<const vec_t<float, 4> *>(xrow)[k];
        } else {
            for (int k = tid; k < a.in_f; k += blockDim.x) xl[k] = xrow[k];
        }
        __syncthreads();
    }

    // 2. route this wave's tables; codes go to the wave's LDS list, route
    //    records are stored after the last ballot (off the ballots' path)
    RouteOut ro[kBallots];
#pragma unroll
    for (int j = 0; j < kBallots; ++j) {
        ro[j] = RouteOut{0ull, false};
        if (j < nballot)
            ro[j] = route_ballot<TRAIN, DEBUG>(a, xs, my_codes, pre[j], t_begin + j * tpb + slot, j * tpb + slot, c,
                                               slot, item);
    }
    for (int k = kBallots; k < nballot; ++k) {
        const Comparator q = load_comparator(a, t_begin + k * tpb + slot, t_end, c);
        const RouteOut r =
            route_ballot<TRAIN, DEBUG>(a, xs, my_codes, q, t_begin + k * tpb + slot, k * tpb + slot, c, slot, item);
        if (TRAIN && r.win) a.rec[static_cast<size_t>(t_begin + k * tpb + slot) * a.items + item] = r.rec;
    }
    if constexpr (TRAIN) {
#pragma unroll
        for (int j = 0; j < kBallots; ++j)
            if (ro[j].win) a.rec[static_cast<size_t>(t_begin + j * tpb + slot) * a.items + item] = ro[j].rec;
    }
    // LDS operations of one wave complete in order: the code list is ready
    if constexpr (DEBUG) {
        if (a.codes != nullptr && blockIdx.y == 0)
            for (int k = lane; k < n_t; k += kWave) a.codes[static_cast<size_t>(item) * a.tables + t_begin + k] = my_codes[k];
    }

    // 3. gather + sum over the wave's tables
    const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(a.lut, a.lut_bytes);
    const int col = blockIdx.y * (kWave * N) + lane * N;
    const uint32_t voff = col < a.out_f ? static_cast<uint32_t>(col) * static_cast<uint32_t>(sizeof(T)) : kOutOfRange;
    float acc[N];
#pragma unroll
    for (int e = 0; e < N; ++e) acc[e] = 0.f;
    for (int t0 = 0; t0 < n_t; t0 += kG) {
        const int cnt = min(kG, n_t - t0);
        static_assert(kG % 8 == 0, "codes are read 8 or 16 at a time");
        constexpr int kRead = kG >= 16 ? 16 : 8;  // bytes per broadcast LDS read
        uint32_t words[kG / 4];
#pragma unroll
        for (int q = 0; q < kG / kRead; ++q) {
            const vec_t<uint32_t, kRead / 4> w =
                *reinterpret_cast<const vec_t<uint32_t, kRead / 4> *>(my_codes + t0 + kRead * q);
#pragma unroll
            for (int e = 0; e < kRead / 4; ++e) words[(kRead / 4) * q + e] = __builtin_amdgcn_readfirstlane(w[e]);
        }
        const int tbase = (t_begin + t0) * a.table_bytes;
        // every slot issues its load; slots past the wave's last table read
        // out of range (zeros), so the loads need no branches
        float v[kG][N];
#pragma unroll
        for (int u = 0; u < kG; ++u) {
            const bool live = u < cnt;
            const int code = static_cast<int>((words[u >> 2] >> (8 * (u & 3))) & 0xffu);
            const int soff = live ? tbase + u * a.table_bytes + code * a.row_bytes : 0;
            buffer_row<T, N>(rsrc, live ? voff : kOutOfRange, soff, v[u]);
        }
#pragma unroll
        for (int u = 0; u < kG; ++u)
#pragma unroll
            for (int e = 0; e < N; ++e) acc[e] += v[u][e];
    }

    // 4. sum the waves' partial rows in wave order, scale, store
    if (nwaves > 1) {
        if (wave > 0) {
#pragma unroll
            for (int e = 0; e < N; ++e) red[((wave - 1) * kWave + lane) * N + e] = acc[e];
        }
        __syncthreads();
        if (wave == 0) {
            for (int w = 1; w < nwaves; ++w) {
#pragma unroll
                for (int e = 0; e < N; ++e) acc[e] += red[((w - 1) * kWave + lane) * N + e];
            }
        }
    }
    if (wave == 0 && col < a.out_f) {
        float y[N];
#pragma unroll
        for (int e = 0; e < N; ++e) y[e] = acc[e] * a.scale;
        store_f32_nt<N>(a.out + static_cast<size_t>(item) * a.out_f + col, y);
    }
}


// Large batches: one workgroup takes kMultiItems consecutive items (and one
// output tile of 64 * N columns). Its waves load their comparators once for
// all the items, the items' input rows are staged as one contiguous block,
// every item is routed from LDS (its codes to the wave's per-item list), and
// the gathers go two items at a time (2 x 16 row loads in flight per wave,
// rows summed in table order as the one-item kernel sums them). The waves'
// partial rows of all the items meet in LDS once and are summed in wave
// order, so this kernel's outputs equal the one-item kernel's bit for bit.
// Planner conditions: at most 16 tables per wave in at most kBallots
// ballots, and at most 8 bytes of a row per lane.
constexpr int kMultiItems = 8;
constexpr int kMultiMinItems = 2048;  // batches from which a workgroup takes kMultiItems items

template <typename T, int N, bool TRAIN, bool DEBUG>
__global__ __launch_bounds__(1024) void pairwise_forward_multi_kernel(FwdArgs a) {
    constexpr int M = kMultiItems;
    constexpr int kG = 16;
    static_assert(N * sizeof(T) <= 8, "two items' row chunks must fit the registers");
    extern __shared__ __align__(16) unsigned char lds[];
    float *xs = reinterpret_cast<float *>(lds);                // [M][in_f]
    float *red = reinterpret_cast<float *>(lds + a.red_off);   // [waves][M][64 N]

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nwaves = blockDim.x >> 6;
    const int b0 = xcd_block_unit(blockIdx.x, gridDim.x) * M;
    const int nitems = min(M, a.items - b0);
    uint8_t *codes_w = lds + a.codes_off + wave * M * a.codes_pitch;  // [M][pitch]

    const int tpb = kWave >> a.lpt_log2;
    const int slot = lane >> a.lpt_log2;
    const int c = lane & ((1 << a.lpt_log2) - 1);
    const int t_begin = wave * a.per_wave;
    const int t_end = min(a.tables, t_begin + a.per_wave);
    const int n_t = max(0, t_end - t_begin);
    const int nballot = (n_t + tpb - 1) / tpb;

    // 1. comparators, once for all the items; the items' input rows
    Comparator pre[kBallots];
#pragma unroll
    for (int j = 0; j < kBallots; ++j) pre[j] = load_comparator(a, t_begin + j * tpb + slot, t_end, c);
    {
        const float *src = a.x + static_cast<size_t>(b0) * a.in_f;
        const int n = nitems * a.in_f;
        if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
            for (int k = tid; k < (n >> 2); k += blockDim.x)
                reinterpret_cast<vec_t<float, 4> *>(xs)[k] = reinterpret_cast<const vec_t<float, 4> *>(src)[k];
        } else {
            for (int k = tid; k < n; k += blockDim.x) xs[k] = src[k];
        }
    }
    __syncthreads();

    // 2. route every item (LDS and ballots only); route records after each
    for (int m = 0; m < M; ++m) {
        if (m >= nitems) break;
        const float *xm = xs + m * a.in_f;
        uint8_t *cm = codes_w + m * a.codes_pitch;
        RouteOut ro[kBallots];
#pragma unroll
        for (int j = 0; j < kBallots; ++j) {
            ro[j] = RouteOut{0ull, false};
            if (j < nballot)
                ro[j] = route_ballot<TRAIN, DEBUG>(a, xm, cm, pre[j], t_begin + j * tpb + slot, j * tpb + slot, c, slot,
                                                   b0 + m);
        }
        if constexpr (TRAIN) {
#pragma unroll
            for (int j = 0; j < kBallots; ++j)
                if (ro[j].win) a.rec[static_cast<size_t>(t_begin + j * tpb + slot) * a.items + b0 + m] = ro[j].rec;
        }
        if constexpr (DEBUG) {
            if (a.codes != nullptr && blockIdx.y == 0)
                for (int k = lane; k < n_t; k += kWave) a.codes[static_cast<size_t>(b0 + m) * a.tables + t_begin + k] = cm[k];
        }
    }
    // LDS operations of one wave complete in order: the code lists are ready

    // 3. gather two items at a time
    const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(a.lut, a.lut_bytes);
    const int col = blockIdx.y * (kWave * N) + lane * N;
    const uint32_t voff = col < a.out_f ? static_cast<uint32_t>(col) * static_cast<uint32_t>(sizeof(T)) : kOutOfRange;
    const int tbase = t_begin * a.table_bytes;
#pragma unroll
    for (int m0 = 0; m0 < M; m0 += 2) {
        if (m0 >= nitems) break;
        uint32_t words[2][kG / 4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const vec_t<uint32_t, 4> w = *reinterpret_cast<const vec_t<uint32_t, 4> *>(codes_w + (m0 + h) * a.codes_pitch);
#pragma unroll
            for (int e = 0; e < 4; ++e) words[h][e] = __builtin_amdgcn_readfirstlane(w[e]);
        }
        constexpr int W = (N * sizeof(T) + 3) / 4;
        uint32_t v[2][kG][W];
        if (n_t == kG && m0 + 1 < nitems) {  // every row live (wave-uniform): no selects
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int u = 0; u < kG; ++u) {
                    const int code = static_cast<int>((words[h][u >> 2] >> (8 * (u & 3))) & 0xffu);
                    buffer_words<T, N>(rsrc, voff, tbase + u * a.table_bytes + code * a.row_bytes, v[h][u]);
                }
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int u = 0; u < kG; ++u) {
                    const bool live = u < n_t && m0 + h < nitems;
                    const int code = static_cast<int>((words[h][u >> 2] >> (8 * (u & 3))) & 0xffu);
                    const int soff = live ? tbase + u * a.table_bytes + code * a.row_bytes : 0;
                    buffer_words<T, N>(rsrc, live ? voff : kOutOfRange, soff, v[h][u]);
                }
        }
        // the pair's partial rows (tables in order) go to LDS at once
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float acc[N];
#pragma unroll
            for (int e = 0; e < N; ++e) acc[e] = 0.f;
#pragma unroll
            for (int u = 0; u < kG; ++u) add_words<T, N>(acc, v[h][u]);
            if (m0 + h < nitems) {
#pragma unroll
                for (int e = 0; e < N; ++e) red[((wave * M + m0 + h) * kWave + lane) * N + e] = acc[e];
            }
        }
    }

    // 4. every item's partial rows, summed in wave order, scaled, stored
    __syncthreads();
    for (int u = tid; u < nitems * kWave; u += blockDim.x) {
        const int m = u / kWave, l = u % kWave;
        const int cl = blockIdx.y * (kWave * N) + l * N;
        if (cl < a.out_f) {
            float y[N];
#pragma unroll
            for (int e = 0; e < N; ++e) y[e] = red[((0 * M + m) * kWave + l) * N + e];
            for (int w = 1; w < nwaves; ++w)
#pragma unroll
                for (int e = 0; e < N; ++e) y[e] += red[((w * M + m) * kWave + l) * N + e];
#pragma unroll
            for (int e = 0; e < N; ++e) y[e] *= a.scale;
            store_f32_nt<N>(a.out + static_cast<size_t>(b0 + m) * a.out_f + cl, y);
        }
    }
}

// Large batches whose LUT row (or column tile of it) is 128, 256, 512 or 1024
// bytes: every wave owns whole items, so no wave waits for another after the
// comparators are staged. Lane (g, j) of a wave holds 16 bytes at byte 16 j of
// item g's row tile (P = 64 / (tile bytes / 16) items per wave).
//   1. The comparators of every table go to LDS once per workgroup, 8 bytes
//      each (both anchors as 16-bit indices, the threshold's bits), and each
//      wave stages its items' input rows: the workgroup's only barrier.
//   2. Route with one lane per table (64 tables a round): the comparisons in
//      order, each margin the same two f32 subtractions as the other
//      kernels', the min-margin pick by the same key order (NaN first, then
//      the smaller |m|, then the lower comparison); codes to LDS.
//   3. Gather: per block of per_wave tables, 16-byte row loads of every table
//      of the block (the next block's loads issued before this one's are
//      summed), the rows summed in table order and the blocks in block order,
//      as the other forward kernels sum them: the outputs are bit-identical.
constexpr int kWaveThreads = 256;
constexpr int kWaveWaves = kWaveThreads / kWave;
constexpr int kWaveBlock = 16;    // tables per block, at most (the plan's per_wave)
constexpr int kWaveMinItems = 2048;
constexpr int kWaveMinWaves = 1024;  // below, the one-item and multi-item kernels spread the work wider
constexpr int kWaveRing = 2;         // blocks of row loads in flight (3 and 4 measured slower)

struct WaveComparator {
    uint32_t ab;  // anchors a | b << 16
    float thr;
};

template <typename T, int P, int K, bool TRAIN, bool DEBUG>
__global__ __launch_bounds__(kWaveThreads) void pairwise_forward_wave_kernel(FwdArgs a) {
    constexpr int E = 16 / static_cast<int>(sizeof(T));  // elements of a 16-byte load
    constexpr int kC = TROPNN_MAX_COMPARISONS;
    constexpr int lpr_log2 = P == 1 ? 6 : P == 2 ? 5 : P == 4 ? 4 : 3;  // lanes per row tile: 64 / P
    static_assert(P == 1 || P == 2 || P == 4 || P == 8, "1, 2, 4 or 8 items per wave");
    using u32x4 = vec_t<uint32_t, 4>;
    extern __shared__ __align__(16) unsigned char lds[];
    WaveComparator *cmp = reinterpret_cast<WaveComparator *>(lds);  // [kC][T]
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float *xs = reinterpret_cast<float *>(lds + a.wave_x_off) + wave * P * a.in_f;  // [in_f][P]: items interleaved
    uint8_t *cw = lds + a.codes_off + wave * P * a.codes_pitch;  // [P][blocks][16]
    const int item0 = (blockIdx.x * kWaveWaves + wave) * P;
    const int nitems = max(0, min(P, a.items - item0));
    const int C = a.comps;

    // 1. comparators (kC slots per table; the unused ones compare x[0] with
    // itself), slot-major so that the route's lanes (consecutive tables) read
    // consecutive 8-byte words; this wave's input rows
#pragma unroll 4
    for (int k = tid; k < a.tables * kC; k += kWaveThreads) {
        const int t = k / kC, c = k - t * kC;
        const size_t tc = static_cast<size_t>(t) * C + min(c, C - 1);  // loads issued unconditionally
        const uint32_t ia = static_cast<uint32_t>(clamp_index(a.anchors[2 * tc], a.in_f));
        const uint32_t ib = static_cast<uint32_t>(clamp_index(a.anchors[2 * tc + 1], a.in_f));
        const float th = a.thr[tc];
        cmp[c * a.tables + t] = c < C ? WaveComparator{ia | (ib << 16), th} : WaveComparator{0u, 0.f};
    }
    {
        // element f of item i at xs[f * P + i], so that one vector read gets
        // feature f of all P items; absent items read zeros
        const float *src = a.x + static_cast<size_t>(item0) * a.in_f;
        const int n = nitems * a.in_f;
        if ((a.in_f & 3) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
            for (int k = 4 * lane; k < P * a.in_f; k += 4 * kWave) {
                const int i = k / a.in_f, f = k - i * a.in_f;
                vec_t<float, 4> v = {0.f, 0.f, 0.f, 0.f};
                if (k < n) v = *reinterpret_cast<const vec_t<float, 4> *>(src + k);
#pragma unroll
                for (int e = 0; e < 4; ++e) xs[(f + e) * P + i] = v[e];
            }
        } else {
            for (int k = lane; k < P * a.in_f; k += kWave) {
                const int i = k / a.in_f, f = k - i * a.in_f;
                xs[f * P + i] = k < n ? src[k] : 0.f;
            }
        }
    }
    __syncthreads();

    // 2. route: lane = table (lanes past the last table idle), its C
    // comparisons in order, each read of an input giving all P items' values
    const bool tile0 = blockIdx.y == 0;
    auto route = [&](int t0) {
        const int t = t0 + lane;
        if (t < a.tables) {
            const int tblk = t / a.per_wave;
            const int cpos = tblk * kWaveBlock + (t - tblk * a.per_wave);  // the code's byte in the list
            uint32_t code[P], key[P];  // min-margin pick: key 0 for NaN, else bits(|m|) + 1
            int pick[P];
            float pm[P];
#pragma unroll
            for (int i = 0; i < P; ++i) {
                code[i] = 0u;
                key[i] = 0xFFFFFFFFu;
                pick[i] = 0;
                pm[i] = 0.f;
            }
            for (int c = 0; c < C; ++c) {
                const WaveComparator q = cmp[c * a.tables + t];
                const vec_t<float, P> xa = *reinterpret_cast<const vec_t<float, P> *>(xs + (q.ab & 0xFFFFu) * P);
                const vec_t<float, P> xb = *reinterpret_cast<const vec_t<float, P> *>(xs + (q.ab >> 16) * P);
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    const float m = (xa[i] - xb[i]) - q.thr;
                    code[i] |= (m > 0.f ? 1u : 0u) << c;
                    if constexpr (TRAIN) {
                        const float mag = fabsf(m);
                        const uint32_t k = mag != mag ? 0u : __builtin_bit_cast(uint32_t, mag) + 1u;
                        if (k < key[i]) {
                            key[i] = k;
                            pick[i] = c;
                            pm[i] = m;
                        }
                    }
                    if constexpr (DEBUG) {
                        if (tile0 && i < nitems && a.margins != nullptr)
                            a.margins[(static_cast<size_t>(item0 + i) * a.tables + t) * C + c] = m;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < P; ++i) {
                if (i < nitems) {
                    cw[i * a.codes_pitch + cpos] = static_cast<uint8_t>(code[i]);
                    const size_t bt = static_cast<size_t>(item0 + i) * a.tables + t;
                    if constexpr (TRAIN) {
                        if (tile0)
                            a.rec[static_cast<size_t>(t) * a.items + item0 + i] =
                                static_cast<uint64_t>(__builtin_bit_cast(uint32_t, pm[i])) |
                                (static_cast<uint64_t>(code[i]) << 32) | (static_cast<uint64_t>(pick[i]) << 48);
                    }
                    if constexpr (DEBUG) {
                        if (tile0) {
                            if (a.indices != nullptr) a.indices[bt] = code[i];
                            if (a.codes != nullptr) a.codes[bt] = static_cast<uint8_t>(code[i]);
                        }
                    }
                }
            }
        }
    };
    // The first 64 tables are routed, then the gather's first blocks (every
    // table of a block below 64: blocks hold at most kWaveBlock tables) are
    // issued, and their rows are in flight while the other tables are
    // routed. LDS operations of one wave complete in order: a block's codes
    // are in the list before the block reads them.
    route(0);

    // 3. gather
    const int g = lane >> lpr_log2, j = lane & ((1 << lpr_log2) - 1);
    const int item = item0 + g;
    const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(a.lut, a.lut_bytes);
    const uint32_t lane_off =
        (static_cast<uint32_t>(blockIdx.y) * static_cast<uint32_t>(a.wave_tile_bytes) + 16u * static_cast<uint32_t>(j)) |
        (g < nitems ? 0u : kOutOfRange);
    const uint8_t *cg = cw + (g < nitems ? g : 0) * a.codes_pitch;
    const int nblk = (a.tables + a.per_wave - 1) / a.per_wave;

    // block b's rows: codes of its tables (16 at a time from LDS), one load
    // per table; a block past the last loads zeros (every offset out of range)
    auto issue = [&](int b, u32x4 (&w)[kWaveBlock]) {
        const int tb = b * a.per_wave, n = max(0, min(a.per_wave, a.tables - tb));
        const u32x4 cv = *reinterpret_cast<const u32x4 *>(cg + min(b, nblk - 1) * kWaveBlock);
#pragma unroll
        for (int u = 0; u < kWaveBlock; ++u) {
            const uint32_t code = (cv[u >> 2] >> (8 * (u & 3))) & 0xFFu;
            const uint32_t voff = u < n ? lane_off + code * static_cast<uint32_t>(a.row_bytes) : kOutOfRange;
            const int soff = u < n ? (tb + u) * a.table_bytes : 0;
            w[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, soff, 0));
        }
        // the block's loads stay together, ahead of the sums that follow
        // (the scheduler would otherwise sink each load to its add)
        __builtin_amdgcn_sched_barrier(0);
    };
    // Every slot of a block is summed: a slot past the block's tables loaded
    // zeros (out of range), and adding +0 changes no partial sum, none being
    // -0 (the sum starts at +0; an exact cancellation rounds to +0 and a sum
    // of floats cannot underflow), so the bits equal the other kernels'
    // sums over the live rows alone.
    float tot[E];
    auto consume = [&](int b, const u32x4 (&w)[kWaveBlock]) {
        float acc[E];
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] = 0.f;
#pragma unroll
        for (int u = 0; u < kWaveBlock; ++u) {
            {
                if constexpr (sizeof(T) == 4) {
                    // the whole vector, then its elements: hipcc (ROCm 7.2)
                    // bit-casts an element of an ext_vector_type value from
                    // the vector's first element
                    const vec_t<float, 4> f = __builtin_bit_cast(vec_t<float, 4>, w[u]);
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[e] += f[e];
                } else {
#pragma unroll
                    for (int e = 0; e < E; ++e)
                        acc[e] = (e & 1) ? add_f16_mix<true>(acc[e], w[u][e >> 1]) : add_f16_mix<false>(acc[e], w[u][e >> 1]);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < E; ++e) tot[e] = b == 0 ? acc[e] : tot[e] + acc[e];  // + 0 past the last block
    };
    // a ring of K blocks in flight: block b + K - 1 is issued before block b
    // is summed. Straight-line code: the blocks past the last are issued and
    // summed too (zeros), so that every wait counts exactly the loads issued
    // since (a conditional issue would merge two counts into the smaller).
    u32x4 w[K][kWaveBlock];
    static_assert((K - 1) * kWaveBlock <= kWave, "the prefetched blocks lie in the first 64 tables");
#pragma unroll
    for (int q = 0; q < K - 1; ++q) issue(q, w[q]);
    for (int t0 = kWave; t0 < a.tables; t0 += kWave) route(t0);
    for (int b0 = 0; b0 < nblk; b0 += K) {
#pragma unroll
        for (int q = 0; q < K; ++q) {
            const int b = b0 + q;
            issue(b + K - 1, w[(q + K - 1) % K]);
            consume(b, w[q]);
        }
    }
    if (g < nitems) {
        float y[E];
#pragma unroll
        for (int e = 0; e < E; ++e) y[e] = tot[e] * a.scale;
        const int col = blockIdx.y * (a.wave_tile_bytes / static_cast<int>(sizeof(T))) + j * E;
        store_f32_nt<E>(a.out + static_cast<size_t>(item) * a.out_f + col, y);
    }
}

// Route only (no gather): one thread per (item, table) evaluates the table's
// comparisons in order and writes any of uint8 codes, int64 codes and f32
// margins, laid out [items][tables] and [items][tables][comparisons]. The
// margin is the same two f32 subtractions as the forward's, so both write
// identical bits. Restates layers/pairwise.py:127-135.
struct RouteArgs {
    const float *x;
    const int64_t *anchors;
    const float *thr;
    uint8_t *codes;
    int64_t *indices;
    float *margins;
    int items, in_f, tables, comps;
};

// ------------------------------------------------------------------ streamed forward (large training shapes)

// Route of a block of items for every table: one thread per table, the
// block's input rows staged in LDS. Writes the route records [T][B] (the
// streamed gather reads the codes from them) and any debug output, with the
// fused forward's arithmetic and its argmin rules (NaN first, then the
// smaller |m|, then the lower comparison index), so records, codes and
// margins are bit-identical to the fused forward's.
struct RouteRecArgs {
    const float *x;
    const int64_t *anchors;
    const float *thr;
    uint64_t *rec;
    int64_t *indices;
    float *margins;
    uint8_t *codes;
    int items, in_f, tables, comps, block_items;
    int rec_stage;  // the block's records gathered in LDS after its input rows, then stored as whole runs
};

constexpr int kRouteRecThreads = 512;
constexpr int kRouteStageBytes = 64 * 1024;  // rows plus staged records, two workgroups per CU

__global__ __launch_bounds__(kRouteRecThreads) void pairwise_route_records_kernel(RouteRecArgs a) {
    extern __shared__ __align__(16) float xs[];  // [block_items][in_f], then (rec_stage) records [T][block_items]
    const int b0 = blockIdx.x * a.block_items, n = min(a.block_items, a.items - b0);
    uint64_t *rs = reinterpret_cast<uint64_t *>(xs + ((a.block_items * a.in_f + 3) & ~3));
    const float *src = a.x + static_cast<size_t>(b0) * a.in_f;
    const int total = n * a.in_f, tid = threadIdx.x;
    // the rows in 16-byte pieces, eight loads per thread in flight before
    // their LDS stores (one or two round trips, not one per piece)
    constexpr int kU = 8;
    if ((a.in_f & 3) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
        const vec_t<float, 4> *s4 = reinterpret_cast<const vec_t<float, 4> *>(src);
        vec_t<float, 4> *d4 = reinterpret_cast<vec_t<float, 4> *>(xs);
        const int n4 = total >> 2;
        for (int k0 = tid; k0 < n4; k0 += kU * kRouteRecThreads) {
            vec_t<float, 4> v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u)
                if (k0 + u * kRouteRecThreads < n4) v[u] = s4[k0 + u * kRouteRecThreads];
#pragma unroll
            for (int u = 0; u < kU; ++u)
                if (k0 + u * kRouteRecThreads < n4) d4[k0 + u * kRouteRecThreads] = v[u];
        }
    } else {
        for (int k0 = tid; k0 < total; k0 += kU * kRouteRecThreads) {
            float v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u)
                if (k0 + u * kRouteRecThreads < total) v[u] = src[k0 + u * kRouteRecThreads];
#pragma unroll
            for (int u = 0; u < kU; ++u)
                if (k0 + u * kRouteRecThreads < total) xs[k0 + u * kRouteRecThreads] = v[u];
        }
    }
    __syncthreads();
    for (int t = tid; t < a.tables; t += kRouteRecThreads) {
        int ia[TROPNN_MAX_COMPARISONS], ib[TROPNN_MAX_COMPARISONS];
        float th[TROPNN_MAX_COMPARISONS];
#pragma unroll
        for (int c = 0; c < TROPNN_MAX_COMPARISONS; ++c) {
            const size_t q = static_cast<size_t>(t) * a.comps + (c < a.comps ? c : 0);
            ia[c] = clamp_index(a.anchors[2 * q], a.in_f);
            ib[c] = clamp_index(a.anchors[2 * q + 1], a.in_f);
            th[c] = a.thr[q];
        }
        for (int m = 0; m < n; ++m) {
            const float *xr = xs + m * a.in_f;
            const size_t bt = static_cast<size_t>(b0 + m) * a.tables + t;
            int code = 0, best = 0;
            uint32_t best_key = 0xFFFFFFFFu;
            float best_m = 0.f;
            for (int c = 0; c < a.comps; ++c) {
                const float mg = (xr[ia[c]] - xr[ib[c]]) - th[c];
                code |= (mg > 0.f ? 1 : 0) << c;
                const float mag = fabsf(mg);
                const uint32_t key = mag != mag ? 0u : __builtin_bit_cast(uint32_t, mag) + 1u;
                if (key < best_key) {  // strict: the first index wins a tie
                    best_key = key;
                    best = c;
                    best_m = mg;
                }
                if (a.margins != nullptr) a.margins[bt * a.comps + c] = mg;
            }
            const uint64_t rec = static_cast<uint64_t>(__builtin_bit_cast(uint32_t, best_m)) |
                                 (static_cast<uint64_t>(code) << 32) | (static_cast<uint64_t>(best) << 48);
            if (a.rec_stage)
                rs[t * a.block_items + m] = rec;
            else
                a.rec[static_cast<size_t>(t) * a.items + b0 + m] = rec;
            if (a.indices != nullptr) a.indices[bt] = code;
            if (a.codes != nullptr) a.codes[bt] = static_cast<uint8_t>(code);
        }
    }
    if (a.rec_stage) {
        // a table's n records are one contiguous run of rec: consecutive
        // lanes store consecutive records of a run
        __syncthreads();
        for (int k = tid; k < a.tables * n; k += kRouteRecThreads) {
            const int t = k / n, m = k - t * n;
            a.rec[static_cast<size_t>(t) * a.items + b0 + m] = rs[t * a.block_items + m];
        }
    }
}

// Streamed gather: one workgroup per (block of 2048 items, chunk of 64 bytes
// of every LUT row: 32 f16 or 16 f32 columns), the workgroups of a chunk
// adjacent on one XCD. The workgroup walks the tables in order with the
// tables' LUT chunks (R rows x 64 bytes) and the items' codes in four LDS
// buffers, filled by LDS-direct loads (global_load_lds: no registers, no LDS
// write instructions) three tables ahead. Thread (slot, piece) owns items
// 8 slot .. 8 slot + 7 and one 16-byte piece of the chunk: per table eight
// LDS row reads and the adds. The workgroups of one chunk stream the same LUT
// chunks at about the same time, so the LUT crosses HBM about once instead of
// once per (item, table) row gather. Each item's row is summed over the tables
// in table order: deterministic, but not the one-item kernel's association
// (its waves' blocks), whose second set of accumulators would not fit the
// registers beside eight items' rows.
//   The buffers are four distinct LDS arrays and the table loop is unrolled
// by four, so that the compiler tells them apart: a read of one buffer does
// not wait for the LDS-direct loads still filling the others.
struct StreamArgs {
    const void *lut;
    const uint64_t *rec;
    float *out;
    float scale;
    int items, out_f, tables, rows, nblk;
};

constexpr int kStreamThreads = 1024;
constexpr int kStreamChunkBytes = 64;                        // bytes of a LUT row in a chunk
constexpr int kStreamPieces = kStreamChunkBytes / 16;        // 16-byte pieces of a row chunk
constexpr int kStreamIpt = 8;                                // items per thread
constexpr int kStreamItems = kStreamThreads / kStreamPieces * kStreamIpt;  // items per workgroup
constexpr int kStreamChunkLds = 256 * kStreamChunkBytes;     // one table's chunk, room for R = 256 rows
constexpr int kStreamRecLoads = kStreamItems / kStreamThreads;  // record words per thread per table
// a buffer: the chunk, then one word per item: the upper word of its route
// record (code | r << 16)
constexpr int kStreamBufBytes = kStreamChunkLds + kStreamItems * 4;
constexpr int kStreamAhead = 3;                              // tables in flight beside the one summed
constexpr int kStreamLoads = kStreamChunkLds / 16 / kStreamThreads + kStreamRecLoads;  // LDS-direct loads per thread per table
constexpr int kStreamMinItems = 4096;
constexpr long long kStreamMinLutBytes = 32ll << 20;

template <typename T>
__global__ __launch_bounds__(kStreamThreads) void pairwise_forward_stream_kernel(StreamArgs a) {
    constexpr int PE = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte piece
    constexpr int COLS = kStreamChunkBytes / static_cast<int>(sizeof(T));
    constexpr int M = kStreamItems;
    constexpr int STAGE = kStreamChunkLds / 16 / kStreamThreads;  // chunk loads per thread per table
    static_assert(kStreamLoads == 3 && kStreamAhead == 3, "the wait below counts 2 tables of loads");
    __shared__ __align__(16) unsigned char sb0[kStreamBufBytes];
    __shared__ __align__(16) unsigned char sb1[kStreamBufBytes];
    __shared__ __align__(16) unsigned char sb2[kStreamBufBytes];
    __shared__ __align__(16) unsigned char sb3[kStreamBufBytes];
    const int R = a.rows;

    const int unit = xcd_block_unit(blockIdx.x, gridDim.x);
    const int chunk = unit / a.nblk, blk = unit - chunk * a.nblk;
    const int b0 = blk * M;
    const int tid = threadIdx.x, slot = tid / kStreamPieces, piece = tid % kStreamPieces;
    const int wave = tid >> 6;
    const size_t row_bytes = static_cast<size_t>(a.out_f) * sizeof(T);
    const unsigned char *lut = static_cast<const unsigned char *>(a.lut) + static_cast<size_t>(chunk) * kStreamChunkBytes;
    const uint32_t *rec_hi[kStreamRecLoads];
#pragma unroll
    for (int j = 0; j < kStreamRecLoads; ++j)
        rec_hi[j] = reinterpret_cast<const uint32_t *>(a.rec) +
                    2 * static_cast<size_t>(min(b0 + j * kStreamThreads + tid, a.items - 1)) + 1;

    auto issue_table = [&](int t, unsigned char *buf) {
        const unsigned char *base = lut + static_cast<size_t>(t) * R * row_bytes;
#pragma unroll
        for (int i = 0; i < STAGE; ++i) {
            const int q = tid + i * kStreamThreads, row = min(q / kStreamPieces, R - 1), pc = q % kStreamPieces;
            __builtin_amdgcn_global_load_lds(base + row * row_bytes + pc * 16,
                                             (__attribute__((address_space(3))) void *)(buf + (i * kStreamThreads + wave * kWave) * 16),
                                             16, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < kStreamRecLoads; ++j)
            __builtin_amdgcn_global_load_lds(rec_hi[j] + 2 * static_cast<size_t>(t) * a.items,
                                             (__attribute__((address_space(3))) void *)(buf + kStreamChunkLds + (j * kStreamThreads + wave * kWave) * 4),
                                             4, 0, 0);
    };

    float acc[kStreamIpt][PE];
#pragma unroll
    for (int k = 0; k < kStreamIpt; ++k)
#pragma unroll
        for (int e = 0; e < PE; ++e) acc[k][e] = 0.f;

    auto step = [&](int t, const unsigned char *cur, unsigned char *nxt) {
        asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        const bool live = t < a.tables;  // workgroup-uniform
        vec_t<uint32_t, 4> w[kStreamIpt];
        if (live) {
#pragma unroll
            for (int h = 0; h < kStreamIpt / 4; ++h) {
                const vec_t<uint32_t, 4> cv =
                    *reinterpret_cast<const vec_t<uint32_t, 4> *>(cur + kStreamChunkLds + slot * kStreamIpt * 4 + h * 16);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    w[4 * h + k] = *reinterpret_cast<const vec_t<uint32_t, 4> *>(
                        cur + (cv[k] & static_cast<uint32_t>(R - 1)) * kStreamChunkBytes + piece * 16);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        issue_table(min(t + kStreamAhead, a.tables - 1), nxt);
        if (live) {
#pragma unroll
            for (int k = 0; k < kStreamIpt; ++k) {
                if constexpr (sizeof(T) == 2) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc[k][2 * e] = add_f16_mix<false>(acc[k][2 * e], w[k][e]);
                        acc[k][2 * e + 1] = add_f16_mix<true>(acc[k][2 * e + 1], w[k][e]);
                    }
                } else {
                    const vec_t<float, 4> f = __builtin_bit_cast(vec_t<float, 4>, w[k]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[k][e] += f[e];
                }
            }
        }
    };

    issue_table(0, sb0);
    issue_table(min(1, a.tables - 1), sb1);
    issue_table(min(2, a.tables - 1), sb2);
    for (int t0 = 0; t0 < a.tables; t0 += 4) {
        step(t0, sb0, sb3);
        step(t0 + 1, sb1, sb0);
        step(t0 + 2, sb2, sb1);
        step(t0 + 3, sb3, sb2);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int col = chunk * COLS + piece * PE;
#pragma unroll
    for (int k = 0; k < kStreamIpt; ++k) {
        const int b = b0 + slot * kStreamIpt + k;
        if (b < a.items) {
            float y[PE];
#pragma unroll
            for (int e = 0; e < PE; ++e) y[e] = acc[k][e] * a.scale;
            store_f32_nt<PE>(a.out + static_cast<size_t>(b) * a.out_f + col, y);
        }
    }
}

constexpr int kRouteThreads = 256;

__global__ __launch_bounds__(kRouteThreads) void pairwise_route_kernel(RouteArgs a) {
    const int k = blockIdx.x * kRouteThreads + threadIdx.x;  // item * tables + table
    if (k >= a.items * a.tables) return;
    const int item = k / a.tables;
    const int t = k - item * a.tables;
    const float *xr = a.x + static_cast<size_t>(item) * a.in_f;
    int code = 0;
    for (int c = 0; c < a.comps; ++c) {
        const size_t q = static_cast<size_t>(t) * a.comps + c;
        const float m = (xr[clamp_index(a.anchors[2 * q], a.in_f)] - xr[clamp_index(a.anchors[2 * q + 1], a.in_f)]) -
                        a.thr[q];
        code |= (m > 0.f ? 1 : 0) << c;
        if (a.margins != nullptr) a.margins[static_cast<size_t>(k) * a.comps + c] = m;
    }
    if (a.codes != nullptr) a.codes[k] = static_cast<uint8_t>(code);
    if (a.indices != nullptr) a.indices[k] = code;
}

template <typename T, int P>
hipError_t launch_wave_items(const FwdArgs &args, const ForwardPlan &p, bool train, bool debug, hipStream_t stream) {
    constexpr int K = kWaveRing;
    auto kernel = train ? (debug ? pairwise_forward_wave_kernel<T, P, K, true, true> : pairwise_forward_wave_kernel<T, P, K, true, false>)
                        : (debug ? pairwise_forward_wave_kernel<T, P, K, false, true> : pairwise_forward_wave_kernel<T, P, K, false, false>);
    return launch_kernel(TROPNN_KERNEL_FORWARD, kernel, dim3(p.wave_blocks, p.wave_tiles), dim3(kWaveThreads),
                         p.wave_lds_bytes, stream, args);
}

template <typename T>
hipError_t launch_wave(const FwdArgs &args, const ForwardPlan &p, bool train, bool debug, hipStream_t stream) {
    switch (kWave >> p.wave_lpr_log2) {
        case 8: return launch_wave_items<T, 8>(args, p, train, debug, stream);
        case 4: return launch_wave_items<T, 4>(args, p, train, debug, stream);
        case 2: return launch_wave_items<T, 2>(args, p, train, debug, stream);
        default: return launch_wave_items<T, 1>(args, p, train, debug, stream);
    }
}

template <typename T, int N>
hipError_t launch_typed(const FwdArgs &args, const ForwardPlan &p, bool train, bool debug, hipStream_t stream) {
    const dim3 grid(p.blocks, p.o_tiles), block(p.threads);
    if constexpr (N * sizeof(T) <= 8) {
        if (p.multi) {
            auto kernel = train ? (debug ? pairwise_forward_multi_kernel<T, N, true, true>
                                         : pairwise_forward_multi_kernel<T, N, true, false>)
                                : (debug ? pairwise_forward_multi_kernel<T, N, false, true>
                                         : pairwise_forward_multi_kernel<T, N, false, false>);
            return launch_kernel(TROPNN_KERNEL_FORWARD, kernel, grid, block, p.lds_bytes, stream, args);
        }
    }
    if (p.wide_x) {
        auto kernel = train ? (debug ? pairwise_forward_kernel<T, N, true, true, true>
                                     : pairwise_forward_kernel<T, N, true, false, true>)
                            : (debug ? pairwise_forward_kernel<T, N, false, true, true>
                                     : pairwise_forward_kernel<T, N, false, false, true>);
        if (hipError_t e = allow_dynamic_lds(reinterpret_cast<const void *>(kernel), p.lds_bytes); e != hipSuccess)
            return e;
        return launch_kernel(TROPNN_KERNEL_FORWARD, kernel, grid, block, p.lds_bytes, stream, args);
    }
    auto kernel = train ? (debug ? pairwise_forward_kernel<T, N, true, true, false>
                                 : pairwise_forward_kernel<T, N, true, false, false>)
                        : (debug ? pairwise_forward_kernel<T, N, false, true, false>
                                 : pairwise_forward_kernel<T, N, false, false, false>);
    return launch_kernel(TROPNN_KERNEL_FORWARD, kernel, grid, block, p.lds_bytes, stream, args);
}

template <typename T>
hipError_t launch_stream(const StreamArgs &args, const ForwardPlan &p, hipStream_t stream) {
    // the LDS buffers are static (4 x 24 KB)
    return launch_kernel(TROPNN_KERNEL_FORWARD, pairwise_forward_stream_kernel<T>, dim3(p.stream_blocks),
                         dim3(kStreamThreads), 0, stream, args);
}

int ilog2(int v) {
    int r = 0;
    while ((1 << r) < v) ++r;
    return r;
}

}  // namespace

ForwardPlan plan_forward(const Dims &d, bool rows16) {
    ForwardPlan p{};
    const int esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    // N elements per lane: the smallest power of two whose 64-lane tile spans
    // the row (16 bytes at most), reduced until it divides the row so that
    // every lane's slice is aligned and either wholly inside or outside it
    p.vec = 1;
    while (p.vec * esize < 16 && p.vec * kWave < d.out_f) p.vec <<= 1;
    while (p.vec > 1 && d.out_f % p.vec != 0) p.vec >>= 1;
    p.o_tile = kWave * p.vec;
    p.o_tiles = (d.out_f + p.o_tile - 1) / p.o_tile;
    p.lpt_log2 = ilog2(d.comps);
    const int chunk = gather_chunk(esize, p.vec);

    // waves per item: enough that one gather chunk covers a wave's tables,
    // more while items x tiles alone cannot give ~4096 waves, at most 16,
    // and at least two tables per wave where there are two: at 16 tables
    // and 8 items, workgroups of 16 one-table waves took 4.8 us per launch
    // against 4.0 us for 8 two-table waves (or 1, 2, 4 waves)
    const long long units = static_cast<long long>(d.items) * p.o_tiles;
    int w = (d.tables + chunk - 1) / chunk;
    const long long want = units > 0 ? (4096 + units - 1) / units : 16;
    if (want > w) w = static_cast<int>(want < 16 ? want : 16);
    if (w > 16) w = 16;
    if (w > (d.tables + 1) / 2) w = (d.tables + 1) / 2;
    p.per_wave = (d.tables + w - 1) / w;
    p.waves_per_item = (d.tables + p.per_wave - 1) / p.per_wave;
    p.threads = p.waves_per_item * kWave;
    p.blocks = d.items;
    p.codes_pitch = ((p.per_wave + chunk - 1) / chunk) * chunk;

    // LDS: the item's input row (unless it would take the workgroup past the
    // default 64 KB: then the route reads it from global memory), the waves'
    // code lists, the waves' partial rows
    auto one_item_lds = [&](long long x_bytes, int &codes_off, int &red_off) {
        long long o = (x_bytes + 15) & ~15ll;
        codes_off = static_cast<int>(o);
        o += static_cast<long long>(p.waves_per_item) * p.codes_pitch;
        o = (o + 15) & ~15ll;
        red_off = static_cast<int>(o);
        return o + static_cast<long long>(p.waves_per_item - 1) * kWave * p.vec * 4;
    };
    long long lds = one_item_lds(static_cast<long long>(d.in_f) * 4, p.codes_off, p.red_off);
    p.wide_x = lds > 64 * 1024;
    if (p.wide_x) lds = one_item_lds(0, p.codes_off, p.red_off);
    p.lds_bytes = static_cast<int>(lds <= kMaxLdsBytes ? lds : kMaxLdsBytes + 1);  // above the maximum: refused

    // large batches: kMultiItems items per workgroup when every wave's
    // tables fit one gather chunk of 16 in at most kBallots ballots and a
    // lane's row chunk is at most 8 bytes
    p.multi = false;
    if (d.items >= kMultiMinItems && p.vec * esize <= 8 && d.in_f <= 16384) {
        const int w16 = (d.tables + 15) / 16;
        const int per16 = (d.tables + w16 - 1) / w16;
        const int tpb = kWave >> p.lpt_log2;
        if (w16 <= 16 && (per16 + tpb - 1) / tpb <= kBallots) {
            int moff = ((kMultiItems * d.in_f * 4) + 15) & ~15;
            const int mcodes = moff;
            moff += w16 * kMultiItems * 16;
            moff = (moff + 15) & ~15;
            const int mred = moff;
            moff += w16 * kMultiItems * kWave * p.vec * 4;
            if (moff <= 64 * 1024) {
                p.multi = true;
                p.per_wave = per16;
                p.waves_per_item = (d.tables + per16 - 1) / per16;
                p.threads = p.waves_per_item * kWave;
                p.blocks = (d.items + kMultiItems - 1) / kMultiItems;
                p.codes_pitch = 16;
                p.codes_off = mcodes;
                p.red_off = mred;
                p.lds_bytes = moff;
            }
        }
    }

    // wave-item kernel: large batches (>= kWaveMinItems items and >=
    // kWaveMinWaves waves) whose row, or 1024-byte column tile of it, is 128
    // to 1024 bytes (a power of two), tables summed in the multi-item
    // kernel's blocks of at most 16; comparators, input rows and code lists
    // within 64 KB of LDS; the LUT and the output 16-byte aligned
    p.wave = false;
    {
        const int row_bytes = d.out_f * esize;
        const int tile = row_bytes <= 1024 ? row_bytes : 1024;
        const bool pow2 = (tile & (tile - 1)) == 0;
        const int ipw = tile >= 128 ? kWave / (tile / 16) : 1;
        if (rows16 && d.items >= kWaveMinItems && (d.items + ipw - 1) / ipw >= kWaveMinWaves && tile >= 128 &&
            pow2 && row_bytes % tile == 0 && d.in_f <= 16384) {
            const int w16 = (d.tables + kWaveBlock - 1) / kWaveBlock;
            const int per16 = (d.tables + w16 - 1) / w16;
            const int lpr = tile / 16;
            const int pitch = w16 * kWaveBlock;  // block b's codes at byte 16 b
            int off = d.tables * TROPNN_MAX_COMPARISONS * 8;
            const int x_off = off;
            off += kWaveWaves * ipw * d.in_f * 4;
            off = (off + 15) & ~15;
            const int c_off = off;
            off += kWaveWaves * ipw * pitch;
            if (off <= 64 * 1024) {
                p.wave = true;
                p.per_wave = per16;
                p.codes_pitch = pitch;
                p.codes_off = c_off;
                p.wave_x_off = x_off;
                p.wave_lpr_log2 = ilog2(lpr);
                p.wave_tile_bytes = tile;
                p.wave_tiles = row_bytes / tile;
                p.wave_blocks = (d.items + kWaveWaves * ipw - 1) / (kWaveWaves * ipw);
                p.wave_lds_bytes = off;
                p.lds_bytes = off;
            }
        }
    }

    // streamed gather (training only: it reads the codes from the route
    // records): large batches over a LUT far beyond the L2, rows of whole
    // 64-byte chunks, at most 256 rows per table, the LUT and the output
    // 16-byte aligned (LDS-direct 16-byte pieces)
    const long long lut_bytes = static_cast<long long>(d.tables) * d.rows * d.out_f * esize;
    p.stream_ok = rows16 && d.items >= kStreamMinItems && (d.out_f * esize) % kStreamChunkBytes == 0 &&
                  d.rows <= 256 && lut_bytes >= kStreamMinLutBytes && d.in_f <= 16384;
    if (p.stream_ok) {
        p.stream_nblk = (d.items + kStreamItems - 1) / kStreamItems;
        p.stream_blocks = p.stream_nblk * (d.out_f * esize / kStreamChunkBytes);
        p.stream_lds = 4 * kStreamBufBytes;  // static
        p.route_block_items = 8;
        while (p.route_block_items > 1 && p.route_block_items * d.in_f * 4 > 64 * 1024) p.route_block_items >>= 1;
        p.route_lds = p.route_block_items * d.in_f * 4;
        const long long rec_lds = static_cast<long long>(d.tables) * p.route_block_items * 8;
        const int x_lds = ((p.route_block_items * d.in_f + 3) & ~3) * 4;
        p.route_rec_stage = x_lds + rec_lds <= kRouteStageBytes;
        if (p.route_rec_stage) p.route_lds = x_lds + static_cast<int>(rec_lds);
    }
    return p;
}

hipError_t launch_forward(const Dims &d, const ForwardPlan &p, const float *x, const int64_t *anchors,
                          const float *thr, const void *lut, float scale, float *out, tropnn_route_record *rec,
                          int64_t *indices, float *margins, uint8_t *codes, hipStream_t stream) {
    const int esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    FwdArgs a{};
    a.x = x;
    a.anchors = anchors;
    a.thr = thr;
    a.lut = lut;
    a.scale = scale;
    a.out = out;
    a.rec = reinterpret_cast<uint64_t *>(rec);
    a.indices = indices;
    a.margins = margins;
    a.codes = codes;
    a.lut_bytes = static_cast<uint32_t>(static_cast<size_t>(d.tables) * d.rows * d.out_f * esize);
    a.items = d.items;
    a.in_f = d.in_f;
    a.out_f = d.out_f;
    a.tables = d.tables;
    a.comps = d.comps;
    a.row_bytes = d.out_f * esize;
    a.table_bytes = d.rows * d.out_f * esize;
    a.lpt_log2 = p.lpt_log2;
    a.per_wave = p.per_wave;
    a.codes_pitch = p.codes_pitch;
    a.codes_off = p.codes_off;
    a.red_off = p.red_off;
    a.wave_lpr_log2 = p.wave_lpr_log2;
    a.wave_tile_bytes = p.wave_tile_bytes;
    a.wave_x_off = p.wave_x_off;
    const bool train = rec != nullptr;
    const bool debug = indices != nullptr || margins != nullptr || codes != nullptr;
    if (train && p.stream_ok) {
        RouteRecArgs r{x, anchors, thr, a.rec, indices, margins, codes, d.items, d.in_f, d.tables, d.comps,
                       p.route_block_items, p.route_rec_stage ? 1 : 0};
        if (hipError_t e = launch_kernel(TROPNN_KERNEL_FORWARD_ROUTE, pairwise_route_records_kernel,
                                         dim3((d.items + p.route_block_items - 1) / p.route_block_items),
                                         dim3(kRouteRecThreads), p.route_lds, stream, r);
            e != hipSuccess)
            return e;
        StreamArgs g{lut, a.rec, out, scale, d.items, d.out_f, d.tables, d.rows, p.stream_nblk};
        return d.lut_dtype == TROPNN_LUT_F16 ? launch_stream<_Float16>(g, p, stream) : launch_stream<float>(g, p, stream);
    }
    if (p.wave)
        return d.lut_dtype == TROPNN_LUT_F16 ? launch_wave<_Float16>(a, p, train, debug, stream)
                                             : launch_wave<float>(a, p, train, debug, stream);
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

hipError_t launch_route(const Dims &d, const float *x, const int64_t *anchors, const float *thr, uint8_t *codes,
                        int64_t *indices, float *margins, hipStream_t stream) {
    RouteArgs a{x, anchors, thr, codes, indices, margins, d.items, d.in_f, d.tables, d.comps};
    const int units = d.items * d.tables;
    const dim3 grid((units + kRouteThreads - 1) / kRouteThreads), block(kRouteThreads);
    hipLaunchKernelGGL(pairwise_route_kernel, grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace tropnn
