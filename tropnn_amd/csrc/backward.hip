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
// fixed summation orders make every gradient deterministic).
//
// Narrow rows (O a multiple of 4 up to 64, or of 8 up to 256, one table's LUT
// rows within 64 KB as f32; c2 is one) with the min-margin STE take the fused
// path, two launches:
//  (F) fused kernel, one workgroup per table. The table's LUT rows are staged
//      in LDS as f32; each tile of 1024 items is counting-sorted by code (one
//      ballot per code bit, per-wave counts written by each code's first item,
//      a DPP scan), every row padded to whole batches of 32 / V slots whose
//      entries carry the item's grad-row offset and the LDS offset of its
//      neighbour row nb. The batches are dealt to row groups (S lanes x V
//      columns spanning the row) as contiguous balanced ranges. One grad-row
//      load per item serves the row's LUT-gradient sum (registers; rows that
//      cross a range boundary are combined in range order afterwards) and the
//      item's STE dot against L[nb] - L[code], completed by one
//      reduce-scatter per batch and left in the slot's LDS word; after the
//      walk one thread per slot forms gu = dot * surrogate'(u), stores it as
//      a {gu, r} record per (table, item) and sums it per comparison into the
//      threshold gradient.
//  (S) scatter kernel, one workgroup per item: expands the item's records into
//      (table, comparison) slots and walks the inverse anchor index into
//      grad_latent, as the item kernel's last phase does.
//
// Other shapes take the general path. With the min-margin STE, four launches:
//  (1) sort kernel, one workgroup per table: the stable counting sort of the
//      table's items by LUT row code (C wave ballots per tile of 1024 items
//      give each item its rank among equal codes of its wave; per-wave counts
//      and a DPP scan give row starts), written once to the workspace as the
//      items' grad-row offsets (with the item's min-margin comparison in the
//      low bits) with every row padded to whole batches of 8 slots, plus each
//      batch's row; and the table's share of a chunk-major copy of G
//      (64-column chunks, each one contiguous block).
//  (2) row kernel, one workgroup per (table, 64-column chunk): row groups of
//      S lanes (V columns each) walk balanced contiguous ranges of the sorted
//      batches, eight grad-row loads in flight per batch (padding slots read
//      out of range: zeros), summing each row in registers; a row inside one
//      range is scaled and written there, a row crossing ranges is combined
//      from the ranges' LDS slots in range order, and empty rows are written
//      as zeros. The same grad-row pieces give each item's partial STE dot
//      over the chunk against L[nb] - L[code] from the table's LUT chunk in
//      LDS; one reduce-scatter per batch completes the batch's partial dots,
//      stored per (table, chunk, item). So the STE reads every LUT row once
//      per (table, chunk), not twice per (item, table).
//  (3) reduce kernel, one workgroup per table: each item's partial dots summed
//      in chunk order, gu = dot * scale * surrogate'(u), the {gu, r} record
//      and the threshold gradient.
//  (4) the scatter kernel above: the input gradient.
// With the full STE (every comparison carries a dot), three launches: the
// full-STE item kernel (one workgroup per item, shaped like the forward: each
// wave takes a block of tables, their current and C neighbour rows in flight,
// one reduce-scatter completing the block's dots; gu per comparison, then the
// feature walk into grad_latent), the sort kernel (which then also sums the
// threshold gradient from gu) and the row kernel without dots.
//  A third, tiny kernel builds the inverse anchor index; callers rebuild it
//  only when the anchors change.
#include <atomic>
#include <limits>
#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "device.hpp"
#include "launch.hpp"

namespace tropnn {
namespace {

constexpr int kSortThreads = 1024;  // items per tile of the sort kernel
constexpr int kRowsThreads = 1024;  // threads of a row-kernel workgroup (but see rows_threads)
constexpr int kRowsBatch = 8;       // sorted slots per row-kernel batch; rows are padded to whole batches

// A row-kernel batch: 32 grad-row floats per lane in flight, so 4 slots for
// 8-column pieces, else kRowsBatch slots. The sort kernel pads rows to whole
// batches of this size.
constexpr int rows_batch(int vec) { return vec == 8 ? 4 : kRowsBatch; }

// Threads of a row-kernel workgroup. With partial dots over an f16 LUT the
// LUT chunk stays f16 in LDS (32 KB at 64 columns), so that a 512-thread
// workgroup needs under 80 KB and two share a CU: one's staging and combine
// overlap the other's walk. Otherwise 1024.
constexpr int rows_threads(bool dots, int lut_esize) { return dots && lut_esize == 2 ? 512 : kRowsThreads; }
// Whether the row kernel with nb packed in its slot offsets forms the
// neighbour row's LDS address with one byte permute: the LUT chunk held in
// LDS (f32 in 1024-thread workgroups, else f16) has rows of 256 bytes. The
// permute yields the address relative to the chunk, so the chunk must sit at
// LDS address 0; launch_rows_vs checks that on the host.
constexpr bool rows_nb_perm(bool dots, int lut_esize, int s, int v) {
    return dots && s * v * (rows_threads(dots, lut_esize) == kRowsThreads ? 4 : 2) == 256;
}
constexpr int kRowsChunk = 64;     // columns of a row-kernel workgroup (at most): 2 MB of G at c4, within an L2
constexpr uint32_t kSlotPad = 0x80000000u;  // grad-row offset of a padding slot: past any grad buffer (<= 2 GiB)
constexpr int kEntries = 16;       // index entries a walker reads per batch

struct ItemArgs {
    const float *grad_out;
    const void *lut;
    const uint64_t *rec;
    const float *margins;          // [B][T][C] (full STE)
    const int32_t *index_offsets;  // [in_f + 1]
    const int32_t *index_entries;  // ((t * C + c) << 1) | side
    float scale;
    int surrogate;  // TROPNN_SURROGATE_*
    float *grad_x;
    float *gu;  // min-margin: [T][B]; full STE: [T][C][B]
    uint32_t lut_bytes, g_bytes;
    int items, in_f, out_f, tables, comps, rows, row_bytes, table_bytes, per_wave, o_tiles;
};

// Sort kernel (general path), one workgroup per table.
struct SortArgs {
    const uint64_t *rec;  // [T][B] route records
    const float *gu;      // [T][B] (min-margin) or [T][C][B] (full STE); null: no threshold gradient
    uint32_t *slot_off;   // [T][slots] sorted grad-row byte offsets, kSlotPad in padding; null: no sort
    int32_t *row_start;   // [T][R + 1] first slot of each LUT row; [R] = the padded length
    int32_t *batch_row;   // [T][slots / batch] the LUT row of each batch of slots
    float *grad_thr;      // or null
    const float *grad_out;  // G [B][O]
    float *g_chunked;     // G copied chunk-major: [chunks][B][P] (P = the row kernel's chunk width)
    int full;             // full STE: gu of every comparison
    int nb_pack;          // slot offsets' low bits: 1: the neighbour row nb = code ^ (1 << r); 0: r
    int items, out_f, comps, rows, slots;
    int chunk_cols, chunk_vec, chunks;  // P, the row kernel's V, ceil(O / P)
    int batch;                          // rows_batch(V): rows are padded to whole batches
};

// Row kernel (general path), one workgroup per (table, column chunk).
struct RowsArgs {
    const float *g_chunked;  // [chunks][B][P]
    const uint32_t *slot_off;
    const int32_t *row_start;
    const int32_t *batch_row;
    float *grad_lut;         // or null (dots only)
    float scale;
    uint32_t gc_bytes;     // bytes of the chunk-major copy
    uint32_t chunk_bytes;  // B * P * 4: one chunk of the copy
    int out_f, rows, tables, slots, part_off;
    // partial STE dots (min-margin): the table's LUT chunk staged in LDS
    const void *lut;       // [T][R][O] f32 or f16
    uint32_t lut_bytes;
    float *pdot;           // [T][chunks][slots] per sorted slot: sum over the chunk's columns of G (L[nb] - L[code]), unscaled
    int items, chunks, lut_off, rs_off;  // LDS byte offsets: LUT chunk (0 with dots), row starts
    int ring_off;                        // LDS byte offset of the row groups' slot-offset rings
};

// Reduce kernel (general path, min-margin), one workgroup per table.
struct ReduceArgs {
    const float *pdot;     // [T][chunks][slots]
    const uint32_t *slot_off;  // [T][slots] the sort kernel's slots: item offset | r, or kSlotPad
    const int32_t *row_start;  // [T][R + 1]: [R] is the table's slot count
    const uint64_t *rec;   // [T][B] route records
    uint64_t *gurec;       // [T][B] {gu bits, r} for the scatter kernel, or null
    float *grad_thr;       // or null
    float scale;
    int surrogate;
    int items, chunks, comps, rows, slots;
    int item_shift;        // slot offset >> item_shift = item (offsets are item * P * 4)
    int stage;             // gurec's records of a table gathered in LDS first (items * 8 bytes of dynamic LDS)
};

__device__ __forceinline__ int rec_code(uint64_t r) { return static_cast<int>((r >> 32) & 0xffffu); }
__device__ __forceinline__ int rec_r(uint64_t r) { return static_cast<int>((r >> 48) & 0xffu); }
__device__ __forceinline__ float rec_u(uint64_t r) { return __builtin_bit_cast(float, static_cast<uint32_t>(r)); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// DPP controls: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1]
// (lane ^ 2), row_half_mirror (lane ^ 7 inside 8), row_ror:8 (lane ^ 8 inside
// 16).
constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kMirror8 = 0x141, kRor8 = 0x128;

// The value of the lane whose id differs in bit BIT (inside a row of 16 via
// DPP; bit 2 uses the half-row mirror, lane ^ 7, which also flips the lower
// bits, and every step below only relies on the flipped high bit; bits 4 and 5
// via cross-row shuffles).
template <int BIT>
__device__ __forceinline__ float flip(float v) {
    if constexpr (BIT == 5) return __shfl_xor(v, 32, kWave);
    else if constexpr (BIT == 4) return __shfl_xor(v, 16, kWave);
    else if constexpr (BIT == 3) return dpp<kRor8>(v);
    else if constexpr (BIT == 2) return dpp<kMirror8>(v);
    else if constexpr (BIT == 1) return dpp<kXor2>(v);
    else return dpp<kXor1>(v);
}

// Reduce-scatter of N values per lane over the S lanes of an aligned lane
// group (N <= S <= 64, powers of two): lane j returns the group total of value
// u = (j / (S / N)) & (N - 1). The first log2(N) steps pair lanes across one
// high bit, keep half of the values and add the partner's copy of that half;
// the remaining steps are plain butterflies. The sum tree is fixed, so every
// total is deterministic.
template <int BIT, int N>
__device__ __forceinline__ void rs_select(float (&v)[N], int j) {
    if constexpr (N > 1) {
        constexpr int H = N / 2;
        const bool up = ((j >> BIT) & 1) != 0;
        float w[H];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const float keep = up ? v[H + i] : v[i];
            const float send = up ? v[i] : v[H + i];
            w[i] = keep + flip<BIT>(send);
        }
        rs_select<BIT - 1, H>(w, j);
        v[0] = w[0];
    } else if constexpr (BIT >= 0) {
        v[0] += flip<BIT>(v[0]);
        rs_select<BIT - 1, 1>(v, j);
    }
}

template <int S, int N>
__device__ __forceinline__ float reduce_scatter(const float (&d)[N], int j) {
    static_assert(S == 4 || S == 8 || S == 16 || S == 32 || S == 64, "lane groups of 4 to 64 lanes");
    static_assert(N <= S && (N & (N - 1)) == 0, "N is a power of two <= S");
    float v[N];
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = d[i];
    constexpr int kTop = S == 64 ? 5 : (S == 32 ? 4 : (S == 16 ? 3 : (S == 8 ? 2 : 1)));
    rs_select<kTop, N>(v, j);
    return v[0];
}

// Word k of the inverse anchor index as the feature walk stages it in LDS:
// offsets [in_f + 1], entries [n_ent = 2 T C], then kEntries zeros, so that
// the walk may read a whole batch of entries past a feature's last one.
__device__ __forceinline__ int index_word(const int32_t *offs, const int32_t *ents, int in_f, int n_ent, int k) {
    return k <= in_f ? offs[k] : (k - in_f - 1 < n_ent ? ents[k - in_f - 1] : 0);
}

// Words [k_begin, nidx) of the index into idx_s, kStageWords per thread in
// flight (all loaded, then all stored): a few round trips instead of one per
// word of a large index.
constexpr int kStageWords = 8;
__device__ __forceinline__ void stage_index(int *idx_s, const int32_t *offs, const int32_t *ents, int in_f, int n_ent,
                                            int k_begin, int nidx, int tid, int nthr) {
    for (int k0 = k_begin + tid; k0 < nidx; k0 += kStageWords * nthr) {
        int iv[kStageWords];
#pragma unroll
        for (int q = 0; q < kStageWords; ++q) {
            const int k = k0 + q * nthr;
            iv[q] = k < nidx ? index_word(offs, ents, in_f, n_ent, k) : 0;
        }
#pragma unroll
        for (int q = 0; q < kStageWords; ++q)
            if (k0 + q * nthr < nidx) idx_s[k0 + q * nthr] = iv[q];
    }
}

// grad_x row of one item: the item's signed gu slots gud[(t * C + c)] named
// by feature f's entries of the inverse anchor index (staged in LDS as
// index_word lays it out), summed in entry order; side 1 subtracts. A batch
// reads its kEntries entries and slots unconditionally (entries past the
// feature's last belong to later features or are the zero padding, so every
// slot index is in range) and drops the extra ones with a select: straight-
// line code instead of a branch around every load.
// When all the features fit half the threads, two adjacent lanes walk a
// feature: lane h of the pair takes the entry batches h, h + 2, ... and the
// feature's value is (lane 0's sum) + (lane 1's sum), so a feature of up to
// 2 kEntries entries takes one batch per lane (c2: 128 features of ~13
// entries, one in six above kEntries, on 256 threads). Otherwise one lane
// walks a feature's batches in order. nthr is even.
__device__ __forceinline__ void feature_walk(const float *gud, const int *idx_s, int in_f, float *grad_x_row, int tid,
                                             int nthr) {
    const int *off_s = idx_s, *ent_s = idx_s + in_f + 1;
    const bool pair = in_f * 2 <= nthr;  // uniform
    const int h = pair ? tid & 1 : 0;
    const int fstep = pair ? nthr >> 1 : nthr, estep = pair ? 2 * kEntries : kEntries;
    // both lanes of a pair see the same f, so they leave the loop together
    for (int f = pair ? tid >> 1 : tid; f < in_f; f += fstep) {
        const int f0 = off_s[f], f1 = off_s[f + 1];
        float gx = 0.f;
        for (int eb = f0 + h * kEntries; eb < f1; eb += estep) {
            int en[kEntries];
#pragma unroll
            for (int q = 0; q < kEntries; ++q) en[q] = ent_s[eb + q];
            float v[kEntries];
#pragma unroll
            for (int q = 0; q < kEntries; ++q) v[q] = gud[en[q] >> 1];
#pragma unroll
            for (int q = 0; q < kEntries; ++q) {
                const float sv = (en[q] & 1) ? -v[q] : v[q];  // gx + (-v) rounds as gx - v
                gx = eb + q < f1 ? gx + sv : gx;
            }
        }
        if (pair) {
            const float other = dpp<kXor1>(gx);  // the partner lane's sum
            if (h == 0) __builtin_nontemporal_store(gx + other, grad_x_row + f);
        } else {
            __builtin_nontemporal_store(gx, grad_x_row + f);
        }
    }
}

// ------------------------------------------------------------------ full-STE item kernel

// Full STE (layers/pairwise.py:168-200): every comparison c of (item, table)
// carries gu_c = s * sum_o G[b,o] (L[code ^ 2^c, o] - L[code, o]) * sg'(m_c),
// m_c being that comparison's own margin. One workgroup per item; each wave
// takes its block of tables F at a time (F = 4, 2 or 1 as the lane's row
// piece widens, so that the F (C + 1) rows in flight fit the registers): lane
// l holds the record of table l % F of the block, the block's current and
// neighbour rows are loaded with scalar row offsets (64 lanes spanning the
// row), and one reduce-scatter over the wave completes its 8 F dots (8
// comparison slots per table). Then the item kernel's feature walk.
template <typename T, int N>
__global__ __launch_bounds__(1024) void pairwise_bwd_full_kernel(ItemArgs a) {
    constexpr int kFullTables = N <= 2 ? 4 : (N == 4 ? 2 : 1);
    extern __shared__ __align__(16) unsigned char lds[];
    float *gud = reinterpret_cast<float *>(lds);  // [T * C] this item's gu slots
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = xcd_block_unit(blockIdx.x, gridDim.x);  // [T][B] records of adjacent items share lines
    const int C = a.comps, R = a.rows;
    const int t0 = wave * a.per_wave;
    const int nt = max(0, min(a.tables, t0 + a.per_wave) - t0);
    const int n_ent = 2 * a.tables * C;
    const int nidx = a.grad_x != nullptr ? a.in_f + 1 + n_ent + kEntries : 0;
    int *idx_s = reinterpret_cast<int *>(gud + a.tables * C);  // [in_f + 1 + 2 T C + kEntries]
    stage_index(idx_s, a.index_offsets, a.index_entries, a.in_f, n_ent, 0, nidx, tid, nthr);

    const __amdgpu_buffer_rsrc_t lut_rsrc = buffer_rsrc(a.lut, a.lut_bytes);
    const __amdgpu_buffer_rsrc_t g_rsrc = buffer_rsrc(a.grad_out, a.g_bytes);
    constexpr int kSlots = kFullTables * TROPNN_MAX_COMPARISONS;  // dots per block
    for (int tb = t0; tb < t0 + nt; tb += kFullTables) {
        const int ntb = min(kFullTables, t0 + nt - tb);
        const int tq = lane & (kFullTables - 1);
        const uint64_t rr = tq < ntb ? a.rec[static_cast<size_t>(tb + tq) * a.items + b] : 0ull;
        const int code_v = rec_code(rr) & (R - 1);
        float d[kSlots];
#pragma unroll
        for (int i = 0; i < kSlots; ++i) d[i] = 0.f;
        for (int ct = 0; ct < a.o_tiles; ++ct) {
            const int col = ct * (kWave * N) + lane * N;
            const bool col_ok = col < a.out_f;
            float g[N];
            buffer_row<float, N>(g_rsrc, col_ok ? static_cast<uint32_t>(b * a.out_f + col) * 4u : kOutOfRange, 0, g);
            const uint32_t voff = col_ok ? static_cast<uint32_t>(col) * static_cast<uint32_t>(sizeof(T)) : kOutOfRange;
#pragma unroll
            for (int q = 0; q < kFullTables; ++q) {
                const bool live = q < ntb;
                const int code = __builtin_amdgcn_readlane(code_v, q);
                const int trow = live ? (tb + q) * a.table_bytes : 0;
                float lk[N];
                buffer_row<T, N>(lut_rsrc, live ? voff : kOutOfRange, trow + code * a.row_bytes, lk);
#pragma unroll
                for (int c = 0; c < TROPNN_MAX_COMPARISONS; ++c) {
                    const bool on = live && c < C;
                    float ln[N];
                    buffer_row<T, N>(lut_rsrc, on ? voff : kOutOfRange,
                                     on ? trow + ((code ^ (1 << c)) & (R - 1)) * a.row_bytes : 0, ln);
#pragma unroll
                    for (int e = 0; e < N; ++e) d[q * TROPNN_MAX_COMPARISONS + c] += g[e] * (ln[e] - lk[e]);
                }
            }
        }
        // lane l completes dot (l / (64 / slots)) % slots: table q = dot / 8,
        // comparison c = dot % 8
        const float dot = reduce_scatter<kWave, kSlots>(d, lane) * a.scale;
        constexpr int kSpread = kWave / kSlots;
        const int slot = (lane / kSpread) & (kSlots - 1);
        const int q = slot / TROPNN_MAX_COMPARISONS, c = slot % TROPNN_MAX_COMPARISONS;
        if (lane % kSpread == 0 && q < ntb && c < C) {
            const int t = tb + q;
            const float gu =
                dot * surrogate_grad(a.margins[(static_cast<size_t>(b) * a.tables + t) * C + c], a.surrogate);
            if (a.grad_x != nullptr) gud[t * C + c] = gu;  // (no LDS with the wide scatter kernel)
            if (a.gu != nullptr) a.gu[(static_cast<size_t>(t) * C + c) * a.items + b] = gu;
        }
    }
    if (a.grad_x == nullptr) return;
    __syncthreads();
    feature_walk(gud, idx_s, a.in_f, a.grad_x + static_cast<size_t>(b) * a.in_f, tid, nthr);
}

// ------------------------------------------------------------------ sort and row kernels (general path)

// Inclusive prefix sum over the 64 lanes of a wave: DPP shifts inside rows of
// 16, then the row broadcasts of lanes 15 and 31. All lanes must be active.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return v;
}

// Exclusive prefix sum over n <= 1024 ints in LDS, in place, by the first
// wave (serial across 64-wide chunks, shuffle scan inside a chunk); v[n]
// receives the total.
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

// Counting-sort step of one wave over its 64 items: zeroes the wave's code
// counts, gives each valid item its rank among the equal codes of the wave
// (one ballot per code bit) and has each code's first item write the code's
// count. One wave's LDS operations complete in order, so the zeroing lands
// before the counts.
__device__ __forceinline__ int wave_code_rank(int code, bool valid, int R, int C, int *cnt_w, int lane) {
    for (int k = lane; k < R; k += kWave) cnt_w[k] = 0;
    uint64_t same = __ballot(valid);
    for (int c = 0; c < C; ++c) {
        const uint64_t bc = __ballot(valid && ((code >> c) & 1));
        same &= ((code >> c) & 1) ? bc : ~bc;
    }
    const int rank = __popcll(same & ((1ull << lane) - 1ull));
    if (valid && rank == 0) cnt_w[code] = __popcll(same);
    return rank;
}

// Sort kernel: the stable counting sort of table t's items by LUT row code,
// written once for every column chunk of the row kernel, and table t's share
// of a chunk-major copy of G for the row kernel (G's rows are O * 4 bytes
// apart, a power of two at c4, so one column chunk of every row maps onto
// few L2 sets; the copy makes a chunk one contiguous block). Pass 1 counts each
// code over tiles of 1024 items (and sums the threshold gradient's partials:
// -gu at each item's min-margin comparison, or at every comparison with the
// full STE, a fixed tree per wave, waves in order, tiles in order); the row
// starts are the counts rounded up to whole batches of rows_batch(V) slots,
// exclusively scanned. Pass 2 places every item at its row's next free slot
// (tiles, waves and lanes in order, so item order is kept inside a row) as
// its byte offset b * P * 4 inside a chunk of the copy, with the item's
// min-margin comparison r in the offset's low 3 bits (P * 4 >= 16); padding
// slots get kSlotPad.
__global__ __launch_bounds__(kSortThreads) void pairwise_bwd_sort_kernel(SortArgs a) {
    constexpr int kWaves = kSortThreads / kWave;
    const int K = a.batch;
    extern __shared__ __align__(16) unsigned char lds[];
    const int R = a.rows, C = a.comps;
    int *cnt = reinterpret_cast<int *>(lds);                 // [waves][R] counts -> slots
    int *base = cnt + kWaves * R;                            // [R] next free slot of each row
    int *wtot = base + R;                                    // [waves] scan carries
    float *tp = reinterpret_cast<float *>(wtot + kWaves);    // [waves][8] threshold partials
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint64_t *rec_t = a.rec + static_cast<size_t>(t) * a.items;
    const bool thr = a.grad_thr != nullptr;
    const float *gu_t = thr ? a.gu + static_cast<size_t>(t) * (a.full ? C : 1) * a.items : nullptr;
    if (lane < 8) tp[wave * 8 + lane] = 0.f;  // each wave its own slots

    // 1. per-code totals, threshold partials
    int tot = 0;  // thread k < R: items of code k
    for (int tile0 = 0; tile0 < a.items; tile0 += kSortThreads) {
        const int b = tile0 + tid;
        const bool valid = b < a.items;
        const uint64_t r = valid ? rec_t[b] : 0ull;
        wave_code_rank(rec_code(r) & (R - 1), valid, R, C, cnt + wave * R, lane);
        if (thr) {
            float tv[8];
            if (a.full) {
#pragma unroll
                for (int c = 0; c < 8; ++c) tv[c] = valid && c < C ? -gu_t[static_cast<size_t>(c) * a.items + b] : 0.f;
            } else {
                const float gu = valid ? gu_t[b] : 0.f;
                const int rr = rec_r(r) & 7;
#pragma unroll
                for (int c = 0; c < 8; ++c) tv[c] = rr == c ? -gu : 0.f;
            }
            const float s = reduce_scatter<kWave, 8>(tv, lane);  // lane 8c: the wave's sum for comparison c
            if ((lane & 7) == 0) tp[wave * 8 + (lane >> 3)] += s;
        }
        __syncthreads();
        if (tid < R)
            for (int w = 0; w < kWaves; ++w) tot += cnt[w * R + tid];
        __syncthreads();
    }

    if (a.slot_off != nullptr) {
        // 2. row starts: totals rounded up to whole batches, exclusive scan;
        //    padding slots and the row of every batch
        const int nscan = ((R + kWave - 1) / kWave) * kWave;  // whole waves
        int padded = 0, incl = 0;
        if (tid < nscan) {
            padded = tid < R ? (tot + K - 1) / K * K : 0;
            incl = wave_inclusive_scan(padded);
        }
        if (R > kWave) {
            if (tid < nscan && lane == kWave - 1) wtot[wave] = incl;
            __syncthreads();
            if (tid < nscan)
                for (int w = 0; w < wave; ++w) incl += wtot[w];
        }
        uint32_t *so = a.slot_off + static_cast<size_t>(t) * a.slots;
        if (tid < R) {
            const int excl = incl - padded;
            a.row_start[static_cast<size_t>(t) * (R + 1) + tid] = excl;
            if (tid == R - 1) a.row_start[static_cast<size_t>(t) * (R + 1) + R] = incl;
            base[tid] = excl;
            for (int q = excl + tot; q < excl + padded; ++q) so[q] = kSlotPad;
            int32_t *br = a.batch_row + static_cast<size_t>(t) * (a.slots / K);
            for (int bb = excl / K; bb < incl / K; ++bb) br[bb] = tid;
        }
        __syncthreads();

        // 3. stable placement
        for (int tile0 = 0; tile0 < a.items; tile0 += kSortThreads) {
            const int b = tile0 + tid;
            const bool valid = b < a.items;
            const uint64_t rr = valid ? rec_t[b] : 0ull;
            const int code = rec_code(rr) & (R - 1);
            const int rank = wave_code_rank(code, valid, R, C, cnt + wave * R, lane);
            __syncthreads();
            if (tid < R) {
                int run = base[tid];
                for (int w = 0; w < kWaves; ++w) {
                    const int x = cnt[w * R + tid];
                    cnt[w * R + tid] = run;
                    run += x;
                }
                base[tid] = run;
            }
            __syncthreads();
            if (valid) {
                const int r = rec_r(rr) & 7;
                const uint32_t low = a.nb_pack ? static_cast<uint32_t>((code ^ (1 << r)) & (R - 1)) : static_cast<uint32_t>(r);
                so[cnt[wave * R + code] + rank] = (static_cast<uint32_t>(b) * static_cast<uint32_t>(a.chunk_cols) * 4u) | low;
            }
            __syncthreads();  // the next tile rewrites the counts
        }

        // 4. this table's share of the chunk-major copy: rows (chunk, item)
        //    of P columns, a contiguous range of them per table; the row's
        //    pieces of V columns go to consecutive threads, so both sides are
        //    contiguous. Pieces past O stay unwritten (the row kernel masks
        //    those columns).
        const int pieces = a.chunk_cols / a.chunk_vec;  // S, a power of two <= 64
        const int rows_total = a.chunks * a.items;
        const int r0 = static_cast<int>(static_cast<int64_t>(rows_total) * t / gridDim.x);
        const int r1 = static_cast<int>(static_cast<int64_t>(rows_total) * (t + 1) / gridDim.x);
        const int piece = tid % pieces;
        for (int cb = r0 + tid / pieces; cb < r1; cb += kSortThreads / pieces) {
            const int chunk = cb / a.items, b = cb - chunk * a.items;
            const int col = chunk * a.chunk_cols + piece * a.chunk_vec;
            if (col >= a.out_f) continue;
            const float *src = a.grad_out + static_cast<size_t>(b) * a.out_f + col;
            float *dst = a.g_chunked + static_cast<size_t>(cb) * a.chunk_cols + piece * a.chunk_vec;
            if (a.chunk_vec % 4 == 0) {
                for (int e = 0; e < a.chunk_vec; e += 4)
                    *reinterpret_cast<vec_t<float, 4> *>(dst + e) = *reinterpret_cast<const vec_t<float, 4> *>(src + e);
            } else {
                for (int e = 0; e < a.chunk_vec; ++e) dst[e] = src[e];
            }
        }
    }

    // 5. threshold gradient: the waves' sums in wave order
    if (thr) {
        __syncthreads();
        if (tid < C) {
            float sum = tp[tid];
            for (int w = 1; w < kWaves; ++w) sum += tp[w * 8 + tid];
            a.grad_thr[t * C + tid] = sum;
        }
    }
}

// Row kernel: LUT gradient of table t over columns [chunk * S * V, + S * V),
// reading the chunk-major copy of G (an item's piece of the chunk at
// slot offset + chunk * B * P * 4; the offset's low 3 bits carry the item's
// min-margin comparison r). With DOTS the workgroup also stages the table's
// LUT chunk in LDS as f32 and, from the same grad-row pieces, forms each
// item's partial STE dot over the chunk, sum G (L[code ^ 2^r] - L[code]):
// the current row L[code] stays in registers for the row, the neighbour rows
// come from LDS, one reduce-scatter per batch completes the batch's dots, and
// the lanes holding them store them at their sorted slots,
// pdot[t][chunk][slot] (a batch's dots are contiguous). So the LUT rows of
// the STE dots are read once per (table, chunk) instead of once per (item,
// table).
// The sorted slots form batches of K = rows_batch(V), each inside one row; the
// batches are dealt to row groups (S lanes x V columns) as contiguous ranges
// of lo or lo + 1 batches, the longer ones first. Per batch a group reads its
// slots' grad-row offsets from its LDS ring (refilled a window of batches
// at a time), issues the K grad-row loads (padding slots read out of range,
// zeros) and adds them to the open row's sum in slot order; the batch's
// dots go back into the ring and leave a window at a time. A row lying
// wholly in the range is scaled and written there; a
// row crossing the range's start (end) leaves its sum in the group's slot 0
// (1), and a combine step adds the pieces in range order and writes the
// row. Empty rows are written as zeros, so grad_lut is fully overwritten.
template <typename T, int V, int S, bool DOTS, bool NBP>
__global__ __launch_bounds__(rows_threads(DOTS, sizeof(T))) void pairwise_bwd_rows_kernel(RowsArgs a) {
    constexpr int NT = rows_threads(DOTS, sizeof(T));
    constexpr int NG = NT / S;  // row groups
    constexpr int K = rows_batch(V);
    constexpr int P = S * V;  // columns of the chunk
    constexpr int KR = K <= S ? K : S;  // dots per reduce-scatter
    // a slot offset's low bits below the item offset: nb (NBP, P * 4 >= R) or r
    constexpr uint32_t kLow = NBP ? static_cast<uint32_t>(P * 4 - 1) : 7u;
    static_assert(!NBP || DOTS, "nb in the slot offsets serves the STE dots");
    // DOTS: the table's LUT chunk [R][P] in LDS, f32, or f16 for an f16 LUT
    // (the 512-thread workgroups of rows_threads)
    using LT = std::conditional_t<NT == kRowsThreads, float, _Float16>;
    // the neighbour row's LDS address from one byte permute: the LUT chunk at
    // LDS offset 0 with 256-byte rows, nb (< 256) in the slot offset's low
    // byte, the lane's column offset (< 256) in the address's low byte
    constexpr bool kNbPerm = NBP && rows_nb_perm(DOTS, sizeof(T), S, V);
    static_assert(!kNbPerm || P * sizeof(LT) == 256, "byte-permute addressing needs 256-byte LDS rows");
    extern __shared__ __align__(16) unsigned char lds[];
    int *rs = reinterpret_cast<int *>(lds + a.rs_off);            // [R + 1] row starts (slots)
    float *part = reinterpret_cast<float *>(lds + a.part_off);    // [groups][2][P] split rows
    LT *lut_s = reinterpret_cast<LT *>(lds + a.lut_off);
    // unit = chunk * T + table, each XCD taking one contiguous block of units:
    // an XCD walks its chunks one at a time over every table, so the chunk's
    // slice of G is read into its L2 once
    const int unit = xcd_block_unit(blockIdx.x, gridDim.x);
    const int chunk = unit / a.tables, t = unit - chunk * a.tables;
    const int R = a.rows, O = a.out_f;
    const int tid = threadIdx.x, g = tid / S, j = tid % S;
    const int col = chunk * P + j * V;
    const bool col_ok = col < O;  // V divides O: a lane's columns are all in or all out
    // grad-row piece of slot offset s: s + chunk base + lane offset; padding
    // (s = kSlotPad) and dead columns fall past the copy and read zeros. With
    // NBP the item offset is a multiple of P * 4 and the lane's column offset
    // j * V * 4 < P * 4 fills the bits nb leaves once masked off (one
    // and-or), the chunk base is the scalar offset, and kOutOfRange in the
    // lane term makes a dead column, or a batch past the group's range, read
    // zeros
    const uint32_t gcol = static_cast<uint32_t>(chunk) * a.chunk_bytes + static_cast<uint32_t>(j * V) * 4u;
    const uint32_t coldead = col_ok ? 0u : kOutOfRange;
    const uint32_t lane_col = static_cast<uint32_t>(j * V) * 4u | coldead;
    const int chunk_base = static_cast<int>(static_cast<uint32_t>(chunk) * a.chunk_bytes);
    const uint32_t lane_lds = static_cast<uint32_t>(j * V) * static_cast<uint32_t>(sizeof(LT));
    const __amdgpu_buffer_rsrc_t g_rsrc = buffer_rsrc(a.g_chunked, a.gc_bytes);
    const uint32_t *so = a.slot_off + static_cast<size_t>(t) * a.slots;
    const int32_t *br = a.batch_row + static_cast<size_t>(t) * (a.slots / K);
    float *gl = a.grad_lut != nullptr ? a.grad_lut + static_cast<size_t>(t) * R * O : nullptr;
    for (int k = tid; k <= R; k += NT) rs[k] = a.row_start[static_cast<size_t>(t) * (R + 1) + k];
    if constexpr (DOTS) {
        // the LUT chunk: R rows of P columns (pieces of V, columns past O zero)
        const __amdgpu_buffer_rsrc_t lut_rsrc = buffer_rsrc(a.lut, a.lut_bytes);
        for (int q = tid; q < R * S; q += NT) {
            const int row = q / S, pc = q - row * S, c0 = chunk * P + pc * V;
            float w[V];
            buffer_row<T, V>(lut_rsrc,
                             c0 < O ? static_cast<uint32_t>((static_cast<size_t>(t) * R + row) * O + c0) * sizeof(T)
                                    : kOutOfRange,
                             0, w);
            vec_t<LT, V> wv;
#pragma unroll
            for (int e = 0; e < V; ++e) wv[e] = static_cast<LT>(w[e]);  // exact: w came from T
            // whole-vector LDS accesses: element by element the lanes'
            // accesses stride by V elements and collide in the banks
            *reinterpret_cast<vec_t<LT, V> *>(lut_s + row * P + pc * V) = wv;
        }
    }
    __syncthreads();

    const int nb_all = rs[R] / K;
    const int lo = nb_all / NG, extra = nb_all - lo * NG;
    const int b_begin = g * lo + min(g, extra), b_end = b_begin + lo + (g < extra ? 1 : 0);
    int cur = -1;  // row being summed
    float acc[V];
    float lkv[V];  // DOTS: L[cur] over this lane's columns
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = lkv[e] = 0.f;
    float *pd = DOTS ? a.pdot + (static_cast<size_t>(t) * a.chunks + chunk) * a.slots : nullptr;
    auto finish = [&](int k) {  // row k's sum over this range
        if (gl == nullptr) return;
        const int fb = rs[k] / K, lb = rs[k + 1] / K - 1;
        if (fb >= b_begin && lb < b_end) {
            if (col_ok) {
                float y[V];
#pragma unroll
                for (int e = 0; e < V; ++e) y[e] = acc[e] * a.scale;
                store_f32_nt<V>(gl + static_cast<size_t>(k) * O + col, y);
            }
        } else {
            vec_t<float, V> w;
#pragma unroll
            for (int e = 0; e < V; ++e) w[e] = acc[e];
            *reinterpret_cast<vec_t<float, V> *>(part + (g * 2 + (fb < b_begin ? 0 : 1)) * P + j * V) = w;
        }
    };
    // Slot offsets come through the group's LDS ring of W batches (W * K =
    // 4 S slots, one 16-byte piece per lane), refilled from a window loaded
    // W batches ahead: a batch costs its grad-row loads only. Rows are
    // padded to whole batches, so a batch that starts at or past the open
    // row's end starts the next non-empty row (the row starts are in LDS);
    // the range's first row is the sort kernel's batch row.
    constexpr int W = S * 4 / K;
    static_assert(W * K == S * 4 && (W & (W - 1)) == 0, "a window is one 16-byte piece per lane");
    uint32_t *ring = reinterpret_cast<uint32_t *>(lds + a.ring_off) + g * (W * K);
    const __amdgpu_buffer_rsrc_t so_rsrc = buffer_rsrc(so, static_cast<uint32_t>(a.slots) * 4u);
    auto window = [&](int w) {  // lane j's piece of window w (past the table's slots: zeros)
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(
            so_rsrc, static_cast<uint32_t>((b_begin + w * W) * K + 4 * j) * 4u, 0, 0);
        return __builtin_bit_cast(vec_t<uint32_t, 4>, v);
    };
    auto ring_offsets = [&](int wi, uint32_t(&off)[K]) {  // batch wi of the ring's window
#pragma unroll
        for (int q = 0; q < K / 4; ++q) {
            const vec_t<uint32_t, 4> w = *reinterpret_cast<const vec_t<uint32_t, 4> *>(ring + wi * K + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e) off[4 * q + e] = w[e];
        }
    };
    vec_t<uint32_t, 4> wnext = window(0);
    *reinterpret_cast<vec_t<uint32_t, 4> *>(ring + 4 * j) = wnext;
    wnext = window(1);
    const int row0 = b_begin < b_end ? br[b_begin] : 0;
    int cur_end = 0;  // first slot past the open row
    // With dots, batch b's K dots go to its ring slots once its offsets are
    // read, and each window's 4 S dots (one 128-byte line at c4) are stored
    // as one 16-byte piece per lane: whole lines instead of a partial line
    // per batch.
    auto flush = [&](int w) {  // window w's dots to pdot (live batches only)
        if ((b_begin + w * W) * K + 4 * j < b_end * K)
            __builtin_nontemporal_store(*reinterpret_cast<const vec_t<uint32_t, 4> *>(ring + 4 * j),
                                        reinterpret_cast<vec_t<uint32_t, 4> *>(pd + (b_begin + w * W) * K + 4 * j));
    };
    uint32_t off[K];
    ring_offsets(0, off);
    int i = 0;
    for (; __ballot(b_begin + i < b_end) != 0; ++i) {  // wave-uniform trip count
        const int bt = b_begin + i;
        const bool live = bt < b_end;
        // a batch past the range reads zeros (its ring slots belong to
        // other groups)
        float gv[K][V];
        if constexpr (NBP) {
            const uint32_t lane_eff = lane_col | (live ? 0u : kOutOfRange);
#pragma unroll
            for (int u = 0; u < K; ++u) buffer_row<float, V>(g_rsrc, (off[u] & ~kLow) | lane_eff, chunk_base, gv[u]);
        } else {
            const uint32_t dead = coldead | (live ? 0u : kOutOfRange);
#pragma unroll
            for (int u = 0; u < K; ++u) buffer_row<float, V>(g_rsrc, ((off[u] & ~kLow) + gcol) | dead, 0, gv[u]);
        }
        if (live && bt * K >= cur_end) {
            if (cur >= 0) finish(cur);
            int k = cur < 0 ? row0 : cur + 1;
            while (rs[k + 1] <= bt * K) ++k;  // empty rows
            cur = k;
            cur_end = rs[k + 1];
#pragma unroll
            for (int e = 0; e < V; ++e) acc[e] = 0.f;
            if constexpr (DOTS) {
                const vec_t<LT, V> lv = *reinterpret_cast<const vec_t<LT, V> *>(lut_s + k * P + j * V);
#pragma unroll
                for (int e = 0; e < V; ++e) lkv[e] = static_cast<float>(lv[e]);
            }
        }
#pragma unroll
        for (int u = 0; u < K; ++u)
#pragma unroll
            for (int e = 0; e < V; ++e) acc[e] += gv[u][e];
        if constexpr (DOTS) {
            // a group past its range has cur's row (or row 0) and reads zeros
            const int kk = max(cur, 0);
            // the batch's neighbour rows, all reads issued before the dots
            vec_t<LT, V> nv[K];
#pragma unroll
            for (int u = 0; u < K; ++u) {
                if constexpr (kNbPerm) {
                    // byte 0: the lane's column offset, byte 1: nb (v_perm_b32
                    // selectors 0-3 pick bytes of the second source, 4-7 of the
                    // first, 0x0c gives zero); the LUT chunk starts at LDS
                    // address 0, so this is the LDS address itself
                    const uint32_t addr = __builtin_amdgcn_perm(off[u], lane_lds, 0x0c0c0400u);
                    nv[u] = *reinterpret_cast<const __attribute__((address_space(3))) vec_t<LT, V> *>(addr);
                } else {
                    // NBP: the sort kernel left nb in the offset's low bits (< R)
                    const int nb = NBP ? static_cast<int>(off[u] & kLow) : (kk ^ (1 << (off[u] & 7u))) & (R - 1);
                    nv[u] = *reinterpret_cast<const vec_t<LT, V> *>(lut_s + nb * P + j * V);
                }
            }
            // L[nb] - L[code] in f32: from f16, one mixed-precision fma
            // (v_fma_mix_f32) of the widened element (exact) with 1 and
            // -L[code], rounded once like the f32 subtraction; the 1 is
            // opaque, or the compiler folds the fma into a conversion and a
            // subtraction
            float one = 1.0f;
            if constexpr (sizeof(LT) == 2) __asm__("" : "+v"(one));
            float d[K];
#pragma unroll
            for (int u = 0; u < K; ++u) {
                float sd = 0.f;
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const float diff = sizeof(LT) == 2 ? __builtin_fmaf(static_cast<float>(nv[u][e]), one, -lkv[e])
                                                       : static_cast<float>(nv[u][e]) - lkv[e];
                    sd += gv[u][e] * diff;
                }
                d[u] = sd;
            }
#pragma unroll
            for (int h = 0; h < K / KR; ++h) {
                float dh[KR];
#pragma unroll
                for (int q = 0; q < KR; ++q) dh[q] = d[h * KR + q];
                const float dot = reduce_scatter<S, KR>(dh, j);
                const int q = (j / (S / KR)) & (KR - 1);  // the slot whose dot this lane holds
                if (j % (S / KR) == 0 && live)
                    ring[(i & (W - 1)) * K + h * KR + q] = __builtin_bit_cast(uint32_t, dot);
            }
        }
        // the next batch's offsets; at a window's end the ring first gives
        // up its dots, then takes the next window (one wave's LDS accesses
        // complete in order)
        if (((i + 1) & (W - 1)) == 0) {
            if constexpr (DOTS) flush(i / W);
            *reinterpret_cast<vec_t<uint32_t, 4> *>(ring + 4 * j) = wnext;
            wnext = window((i + 1) / W + 1);
        }
        ring_offsets((i + 1) & (W - 1), off);
    }
    if constexpr (DOTS)
        if ((i & (W - 1)) != 0) flush(i / W);  // the last, partial window
    if (cur >= 0) finish(cur);
    __syncthreads();

    // combine: group g writes rows g, g + groups, ...: an empty row as zeros,
    // a row split over ranges as its pieces in range order (slot 1 of its
    // first range, slot 0 of the others); rows inside one range are written
    const int bl = lo + 1;
    const float inv_bl = 1.0f / static_cast<float>(bl), inv_lo = 1.0f / static_cast<float>(max(lo, 1));
    auto range_of = [&](int bt) { return bt < extra * bl ? small_div(bt, inv_bl) : extra + small_div(bt - extra * bl, inv_lo); };
    if (gl == nullptr) return;
    for (int k = g; k < R; k += NG) {
        const int fb = rs[k] / K, nbk = rs[k + 1] / K - fb;
        vec_t<float, V> w = 0.f;
        if (nbk > 0) {
            const int gf = range_of(fb), gla = range_of(fb + nbk - 1);
            if (gf == gla) continue;
            w = *reinterpret_cast<const vec_t<float, V> *>(part + (gf * 2 + 1) * P + j * V);
            for (int gg = gf + 1; gg <= gla; ++gg) w += *reinterpret_cast<const vec_t<float, V> *>(part + gg * 2 * P + j * V);
        }
        if (col_ok) {
            float y[V];
#pragma unroll
            for (int e = 0; e < V; ++e) y[e] = w[e] * a.scale;
            store_f32_nt<V>(gl + static_cast<size_t>(k) * O + col, y);
        }
    }
}

// Reduce kernel (general path, min-margin): one workgroup per table, one
// thread per sorted slot of a tile of 1024 slots. A slot's STE dot is the
// sum of its chunks' partial dots in chunk order (contiguous reads across the
// threads); gu = dot * scale * surrogate'(u) with u from the slot item's
// route record. It stores the {gu, r} record for the scatter kernel and sums
// the threshold gradient, -gu at the item's min-margin comparison (a fixed
// tree per wave, waves in order, tiles in order: slots in sorted order).
// Padding slots carry no gu.
constexpr int kReduceThreads = 1024;
constexpr int kReduceStageBytes = 64 * 1024;  // a table's {gu, r} records staged in LDS up to 8192 items

__global__ __launch_bounds__(kReduceThreads) void pairwise_bwd_reduce_kernel(ReduceArgs a) {
    constexpr int kWaves = kReduceThreads / kWave;
    __shared__ float tp[kWaves * 8];
    // with `stage`, the table's {gu, r} records gather in LDS (in item order)
    // and leave as whole lines after the walk, instead of as scattered
    // 8-byte stores
    extern __shared__ __align__(16) uint64_t gstage[];  // [items]
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint64_t *rec_t = a.rec + static_cast<size_t>(t) * a.items;
    const uint32_t *so = a.slot_off + static_cast<size_t>(t) * a.slots;
    const float *pd = a.pdot + static_cast<size_t>(t) * a.chunks * a.slots;
    const int n_slots = a.row_start[static_cast<size_t>(t) * (a.rows + 1) + a.rows];
    if (lane < 8) tp[wave * 8 + lane] = 0.f;  // each wave its own slots
    for (int q0 = 0; q0 < n_slots; q0 += kReduceThreads) {
        const int q = q0 + tid;
        const uint32_t off = q < n_slots ? so[q] : kSlotPad;
        const bool live = off != kSlotPad;
        const int b = static_cast<int>(off >> a.item_shift);
        const uint64_t rr = live ? rec_t[b] : 0ull;
        float dot = 0.f;
        if (live) {
            constexpr int kU = 8;  // partial dots in flight
            int c = 0;
            for (; c + kU <= a.chunks; c += kU) {
                float v[kU];
#pragma unroll
                for (int u = 0; u < kU; ++u) v[u] = pd[static_cast<size_t>(c + u) * a.slots + q];
#pragma unroll
                for (int u = 0; u < kU; ++u) dot += v[u];
            }
            for (; c < a.chunks; ++c) dot += pd[static_cast<size_t>(c) * a.slots + q];
        }
        const int r = rec_r(rr) & 7;  // the slot's low bits may hold the neighbour row instead
        const float gu = live ? dot * a.scale * surrogate_grad(rec_u(rr), a.surrogate) : 0.f;
        if (live && a.gurec != nullptr) {
            const uint64_t out = static_cast<uint64_t>(__builtin_bit_cast(uint32_t, gu)) | (static_cast<uint64_t>(r) << 32);
            if (a.stage)
                gstage[b] = out;
            else
                a.gurec[static_cast<size_t>(t) * a.items + b] = out;
        }
        if (a.grad_thr != nullptr) {
            float tv[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) tv[c] = live && r == c ? -gu : 0.f;
            const float sum = reduce_scatter<kWave, 8>(tv, lane);  // lane 8c: the wave's sum for comparison c
            if ((lane & 7) == 0) tp[wave * 8 + (lane >> 3)] += sum;
        }
    }
    if (a.stage || a.grad_thr != nullptr) __syncthreads();
    if (a.stage)  // every item of the table had one live slot
        for (int k = tid; k < a.items; k += kReduceThreads) a.gurec[static_cast<size_t>(t) * a.items + k] = gstage[k];
    if (a.grad_thr != nullptr) {
        if (tid < a.comps) {
            float sum = tp[tid];
            for (int w = 1; w < kWaves; ++w) sum += tp[w * 8 + tid];
            a.grad_thr[t * a.comps + tid] = sum;
        }
    }
}

// ------------------------------------------------------------------ fused row kernel

constexpr int kFusedThreads = 1024;  // threads of a fused workgroup = items per sort tile
constexpr int kFusedFloats = 32;     // grad-row floats a lane has in flight: 32 / V items per batch
constexpr uint32_t kPadSlot = 0x80000000u;  // sorted-entry flag of a row's padding slot
// Item role: at most this many tables (so that, with one table workgroup per
// CU, at least a quarter of gfx950's 256 CUs take the item workgroups), at
// least kItemRoleMinWgs item workgroups, at most kItemChunk items in LDS.
// It gathers two LUT rows per (item, table) through the L2 on the CUs the
// table workgroups leave free, so its time grows with T / (CUs - T) x row
// bytes, while the scatter kernel it replaces costs a kernel boundary plus
// ~4 us. Measured at T = 136, B = 512 (graph-replayed steps): f32 rows of
// up to 256 bytes 17.8 -> 14.9 us per step, 384 bytes 20.1 -> 19.5 us,
// 512 bytes (c2) 20.3 -> 22.2 us; f16 rows of 256 bytes 23.6 -> 22.1 us.
// So the planner takes it while T x row bytes <= kItemRoleRowBytes x
// (kCus - T), a product between the winning 384 and the losing 512 bytes at
// T = 136.
constexpr int kItemRoleMaxTables = 192;
constexpr int kItemRoleMinWgs = 32;
constexpr int kItemChunk = 32;
constexpr int kCus = 256;               // gfx950 (MI355X)
constexpr int kItemRoleRowBytes = 448;

struct FusedArgs {
    const float *grad_out;
    const void *lut;
    const uint64_t *rec;
    float scale;
    float *grad_lut;  // or null
    float *grad_thr;  // or null
    uint64_t *gurec;  // [T][B] {gu bits, r} for the scatter kernel, or null
    uint32_t lut_bytes, g_bytes;
    uint32_t g_slice;     // bytes of G one workgroup touches (8 XCDs share the table workgroups)
    int surrogate;        // TROPNN_SURROGATE_*
    uint64_t quad_magic;  // ceil(2^32 / (out_f / CH)): staging chunk index -> LUT row
    int items, out_f, tables, comps, rows;
    int slots;  // sorted-list capacity: a tile's items plus K - 1 padding slots per row
    int lut_off, cnt_off, off_off, sorted_off, u_off, dt_off, rowbuf_off, thr_off, wtot_off, part_off, brow_off;  // LDS bytes
    // item role: workgroups table_wgs.. form the input gradient of item_n
    // items each (no scatter kernel), item_nc items at a time in LDS
    int table_wgs;  // workgroups of the table role (the first ones): T, or 0
    const int32_t *index_offsets;
    const int32_t *index_entries;
    float *grad_x;  // or null (no item role)
    int in_f, item_n, item_nc;
    int ir_rec_off, ir_g_off, ir_gud_off, ir_idx_off;  // LDS bytes
};

constexpr int kScatterThreads = 256;  // threads of a scatter-kernel workgroup (one item)

// The feature walk of feature_walk for nc items at once over nthr threads:
// unit w = (item i, feature f), i = w / in_f, with item i's gu slots at
// gud + i * gstride and its gradient row at grad_x_rows + i * in_f. A pair of
// lanes walks a unit exactly when the scatter kernel's 256 threads pair
// them (2 in_f <= 256), so each value is summed in the scatter kernel's
// order.
__device__ __forceinline__ void feature_walk_items(const float *gud, int gstride, const int *idx_s, int in_f,
                                                   int nc, float *grad_x_rows, int tid, int nthr) {
    const int *off_s = idx_s, *ent_s = idx_s + in_f + 1;
    const bool pair = in_f * 2 <= kScatterThreads;  // uniform
    const int h = pair ? tid & 1 : 0;
    const int wstep = pair ? nthr >> 1 : nthr, estep = pair ? 2 * kEntries : kEntries;
    const float inv_in = 1.0f / static_cast<float>(in_f);
    const int nunits = nc * in_f;
    // both lanes of a pair see the same w, so they leave the loop together
    for (int w = pair ? tid >> 1 : tid; w < nunits; w += wstep) {
        const int i = small_div(w, inv_in), f = w - i * in_f;
        const float *gi = gud + i * gstride;
        const int f0 = off_s[f], f1 = off_s[f + 1];
        float gx = 0.f;
        for (int eb = f0 + h * kEntries; eb < f1; eb += estep) {
            int en[kEntries];
#pragma unroll
            for (int q = 0; q < kEntries; ++q) en[q] = ent_s[eb + q];
            float v[kEntries];
#pragma unroll
            for (int q = 0; q < kEntries; ++q) v[q] = gi[en[q] >> 1];
#pragma unroll
            for (int q = 0; q < kEntries; ++q) {
                const float sv = (en[q] & 1) ? -v[q] : v[q];  // gx + (-v) rounds as gx - v
                gx = eb + q < f1 ? gx + sv : gx;
            }
        }
        if (pair) {
            const float other = dpp<kXor1>(gx);  // the partner lane's sum
            if (h == 0) __builtin_nontemporal_store(gx + other, grad_x_rows + w);
        } else {
            __builtin_nontemporal_store(gx, grad_x_rows + w);
        }
    }
}

// Item role of the fused kernel (the workgroups after the table_wgs table
// ones): the input gradient of item_n consecutive items, with no dependency
// on the table role, so the step needs no scatter kernel after it. Per chunk
// of item_nc items the route records [item][T] and G rows go to LDS (and,
// once, the inverse anchor index). Every (item, table) unit's STE dot
// s * sum_o G[b,o] (L[t,nb,o] - L[t,code,o]) is formed by a row group of S
// lanes x V columns exactly as the table role forms it (the same lane
// columns, per-lane sum and reduce-scatter, so the same bits), from LUT rows
// read through the L2 in batches of K units of one item; the lane holding a
// unit's dot forms gu = dot * surrogate'(u) and writes the item's C signed
// (table, comparison) slots (gu at r*, zeros elsewhere), and the feature walk
// sums them into grad_latent as the scatter kernel does. Batches past the
// last unit read zeros and write nothing.
template <typename T, int V, int S>
__device__ __forceinline__ void fused_item_role(const FusedArgs &a, unsigned char *lds) {
    constexpr int NG = kFusedThreads / S;  // row groups
    constexpr int K = kFusedFloats / V;    // units per batch
    constexpr int P = S * V;
    const int tid = threadIdx.x;
    const int u = static_cast<int>(blockIdx.x) - a.table_wgs;
    const int b_begin = u * a.item_n;
    const int b_end = min(a.items, b_begin + a.item_n);
    const int TT = a.tables, C = a.comps, R = a.rows, O = a.out_f;
    uint64_t *rec_s = reinterpret_cast<uint64_t *>(lds + a.ir_rec_off);  // [nc][T] route records
    float *g_s = reinterpret_cast<float *>(lds + a.ir_g_off);            // [nc][O] G rows, then P zeros
    float *gud = reinterpret_cast<float *>(lds + a.ir_gud_off);          // [nc][T * C] signed slots
    int *idx_s = reinterpret_cast<int *>(lds + a.ir_idx_off);            // the inverse anchor index
    const __amdgpu_buffer_rsrc_t lut_rsrc = buffer_rsrc(a.lut, a.lut_bytes);
    const int n_ent = 2 * TT * C;
    const int nidx = a.in_f + 1 + n_ent + kEntries;
    for (int k = tid; k < nidx; k += kFusedThreads)
        idx_s[k] = index_word(a.index_offsets, a.index_entries, a.in_f, n_ent, k);
    const int g = tid / S, j = tid % S;
    const int col = j * V;
    const bool col_ok = col < O;
    const uint32_t lane_off = (static_cast<uint32_t>(col) * static_cast<uint32_t>(sizeof(T))) | (col_ok ? 0u : kOutOfRange);
    const uint32_t row_bytes = static_cast<uint32_t>(O) * static_cast<uint32_t>(sizeof(T));
    const int nbi = (TT + K - 1) / K;  // batches per item
    const float inv_nbi = 1.0f / static_cast<float>(nbi);
    for (int c0 = b_begin; c0 < b_end; c0 += a.item_nc) {
        const int nc = min(a.item_nc, b_end - c0);
        // records: consecutive threads take consecutive items of one table
        for (int q = tid; q < nc * TT; q += kFusedThreads) {
            const int t = q / nc, i = q - t * nc;
            rec_s[i * TT + t] = a.rec[static_cast<size_t>(t) * a.items + c0 + i];
        }
        for (int q = tid; q < nc * O + P; q += kFusedThreads)
            g_s[q] = q < nc * O ? a.grad_out[static_cast<size_t>(c0) * O + q] : 0.f;
        __syncthreads();
        const int nbatch = nc * nbi;
        for (int k = 0; __ballot(g + k * NG < nbatch) != 0; ++k) {  // wave-uniform trip count
            const int bt = g + k * NG;
            const bool live = bt < nbatch;
            const int i = live ? small_div(bt, inv_nbi) : 0;
            const int tb = (bt - i * nbi) * K;
            float gv[V];
#pragma unroll
            for (int e = 0; e < V; ++e) gv[e] = g_s[i * O + col + e];
            float lc[K][V], ln[K][V];
#pragma unroll
            for (int q = 0; q < K; ++q) {
                const int t = tb + q;
                const bool ok = live && t < TT;
                const uint64_t rr = ok ? rec_s[i * TT + t] : 0ull;
                const int code = rec_code(rr) & (R - 1), r = rec_r(rr) & 7;
                const int nb = (code ^ (1 << r)) & (R - 1);
                const uint32_t tbase = static_cast<uint32_t>(t * R) * row_bytes;
                const uint32_t dead = ok ? 0u : kOutOfRange;
                buffer_row<T, V>(lut_rsrc, (tbase + static_cast<uint32_t>(code) * row_bytes + lane_off) | dead, 0, lc[q]);
                buffer_row<T, V>(lut_rsrc, (tbase + static_cast<uint32_t>(nb) * row_bytes + lane_off) | dead, 0, ln[q]);
            }
            float d[K];
#pragma unroll
            for (int q = 0; q < K; ++q) {
                float sd = 0.f;
#pragma unroll
                for (int e = 0; e < V; ++e) sd += gv[e] * (ln[q][e] - lc[q][e]);
                d[q] = sd;
            }
            const float dot = reduce_scatter<S, K>(d, j) * a.scale;
            const int q = (j / (S / K)) & (K - 1);  // the unit whose dot this lane holds
            const int t = tb + q;
            if (live && t < TT && j % (S / K) == 0) {
                const uint64_t rr = rec_s[i * TT + t];
                const int r = rec_r(rr) & 7;
                const float gu = dot * surrogate_grad(rec_u(rr), a.surrogate);
                float *slot = gud + (i * TT + t) * C;
                for (int c = 0; c < C; ++c) slot[c] = c == r ? gu : 0.f;
            }
        }
        __syncthreads();
        feature_walk_items(gud, TT * C, idx_s, a.in_f, nc, a.grad_x + static_cast<size_t>(c0) * a.in_f, tid,
                           kFusedThreads);
        __syncthreads();
    }
}

// One workgroup per table; the row group of S lanes x V columns spans the
// whole output row (S * V >= O). The table's LUT rows sit in LDS as f32.
// Per tile of 1024 items: counting sort by code (as in the sort kernel),
// then row group g owns rows g, g + groups, ... and walks each row's items
// in item order, 32 / V at a time: one grad row load per item serves both the
// LUT-gradient sum and the item's STE dot against L[nb] - L[code] (L[code]
// in registers for the whole row, L[nb] from LDS). One reduce-scatter per
// batch completes its dots, which the lanes holding them leave in the sorted
// positions' LDS slots; a pass per tile with one thread per slot then forms
// gu (the surrogate's division once per item, not once per lane of a row
// group), stores {gu, r} for the scatter kernel and reduces the threshold
// gradient.
template <typename T, int V, int S>
__global__ __launch_bounds__(kFusedThreads) void pairwise_bwd_fused_kernel(FusedArgs a) {
    constexpr int kWaves = kFusedThreads / kWave;
    constexpr int NG = kFusedThreads / S;  // row groups
    constexpr int K = kFusedFloats / V;  // items per batch
    constexpr int CH = V < 4 ? V : 4;  // elements per staging chunk: O % CH == 0, so none crosses a row
    constexpr int kStage = 4;  // LUT chunks a thread stages: R * O <= 4096 * CH
    constexpr int P = S * V;   // LDS row pitch in floats
    static_assert(K <= S, "a batch's dots are scattered over the row group");
    extern __shared__ __align__(16) unsigned char lds[];
    float *lut_s = reinterpret_cast<float *>(lds + a.lut_off);             // [R][pitch] table rows, f32
    int *cnt = reinterpret_cast<int *>(lds + a.cnt_off);                   // [R][waves] counts -> offsets
    int *off = reinterpret_cast<int *>(lds + a.off_off);                   // [R + 1] row starts
    uint2 *ent = reinterpret_cast<uint2 *>(lds + a.sorted_off);           // [slots] sorted entries (see below)
    float *us = reinterpret_cast<float *>(lds + a.u_off);                  // [slots] margin u, by position
    float *dt = reinterpret_cast<float *>(lds + a.dt_off);                 // [slots] scaled STE dot, by position
    float *rowbuf = reinterpret_cast<float *>(lds + a.rowbuf_off);         // [R][pitch] (several tiles)
    float *tp = reinterpret_cast<float *>(lds + a.thr_off);                // [waves][8]
    int *wtot = reinterpret_cast<int *>(lds + a.wtot_off);                 // [waves] scan carries, [1] sink
    float *part = reinterpret_cast<float *>(lds + a.part_off);             // [groups][2][pitch] split rows
    int *brow = reinterpret_cast<int *>(lds + a.brow_off);                 // [slots / K] row of each batch

    if (static_cast<int>(blockIdx.x) >= a.table_wgs) {  // item role (uniform per workgroup)
        fused_item_role<T, V, S>(a, lds);
        return;
    }
    const int t = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int R = a.rows, C = a.comps, O = a.out_f;
    const bool single = a.items <= kFusedThreads;
    const bool need_gu = a.grad_thr != nullptr || a.gurec != nullptr;
    const uint64_t *rec_t = a.rec + static_cast<size_t>(t) * a.items;
    const __amdgpu_buffer_rsrc_t g_rsrc = buffer_rsrc(a.grad_out, a.g_bytes);
    const __amdgpu_buffer_rsrc_t lut_rsrc = buffer_rsrc(a.lut, a.lut_bytes);

    // 1. one ballot per code bit gives each item the mask of equal codes in
    //    its wave: its rank is the count below it, and the first item of
    //    each code writes the code's count to cnt[code][wave] after the wave
    //    has zeroed its counts (one wave's LDS operations complete in order).
    //    A row's counts of all waves are contiguous: the scan reads and
    //    writes them as vectors at one base address.
    auto ballots = [&](uint64_t rr, int n_tile) -> int {
        const bool valid = tid < n_tile;
        const int code = rec_code(rr) & (R - 1);  // masks keep a corrupt record in range
        for (int k = lane; k < R; k += kWave) cnt[k * kWaves + wave] = 0;
        if (wave * kWave >= n_tile) return 0;
        uint64_t same = __ballot(valid);
        for (int c = 0; c < C; ++c) {
            const uint64_t bc = __ballot(valid && ((code >> c) & 1));
            same &= ((code >> c) & 1) ? bc : ~bc;
        }
        const int rank = __popcll(same & ((1ull << lane) - 1ull));
        if (valid && rank == 0) cnt[code * kWaves + wave] = __popcll(same);
        return rank;
    };

    // 0. first tile's record, the table's LUT rows and a touch of one slice
    //    of G per XCD (workgroups are dealt to the 8 XCDs in turn, so the
    //    grad rows the walk gathers are L2 hits by then); the first ballots
    //    need the record only, and the LUT rows go to LDS after them
    uint64_t r0 = tid < a.items ? rec_t[tid] : 0ull;
    float lv[kStage][CH];
    const int quads = R * O / CH;  // CH-element chunks
    {
        const int tbase = t * R * O * static_cast<int>(sizeof(T));
#pragma unroll
        for (int i = 0; i < kStage; ++i) {
            const int q = tid + i * kFusedThreads;
            buffer_row<T, CH>(lut_rsrc, q < quads ? static_cast<uint32_t>(q) * CH * sizeof(T) : kOutOfRange, tbase, lv[i]);
        }
    }
    const uint32_t touch = static_cast<uint32_t>(t >> 3) * a.g_slice + tid * 128u;
    const uint32_t pf = tid * 128u < a.g_slice ? __builtin_amdgcn_raw_buffer_load_b32(g_rsrc, touch, 0, 0) : 0u;
    int rank = ballots(r0, min(kFusedThreads, a.items));
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int q = tid + i * kFusedThreads;
        if (q < quads) {
            // row = q / (O / CH) by a host-computed reciprocal (exact for q < 2^16)
            const int row = static_cast<int>((static_cast<uint64_t>(q) * a.quad_magic) >> 32);
            const int col = q * CH - row * O;
            vec_t<float, CH> w;
#pragma unroll
            for (int e = 0; e < CH; ++e) w[e] = lv[i][e];
            *reinterpret_cast<vec_t<float, CH> *>(lut_s + row * P + col) = w;
        }
    }
    if (tid < R)
        for (int e = O; e < P; e += CH) *reinterpret_cast<vec_t<float, CH> *>(lut_s + tid * P + e) = 0.f;
    if (!single)
        for (int k = tid * 4; k < R * P; k += kFusedThreads * 4) *reinterpret_cast<vec_t<float, 4> *>(rowbuf + k) = 0.f;
    if (tid < kWaves * 8) tp[tid] = 0.f;
    if (tid < K) {  // sentinel slots for row groups past their row
        ent[a.slots + tid] = make_uint2(kOutOfRange, kPadSlot);
        us[a.slots + tid] = 0.f;
    }
    __syncthreads();

    for (int tile0 = 0;;) {
        const int n_tile = min(kFusedThreads, a.items - tile0);
        // per-lane values inside the loop come from an opaque copy of the
        // thread id: hoisted out of the loop (the scan's 32 LDS addresses,
        // the walk's lane offsets) they would stay live across the walk
        int tidl = tid;
        __asm__ volatile("" : "+v"(tidl));

        // 2. thread k: row k's per-wave counts -> offsets inside the row,
        //    row totals rounded up to whole batches of K slots -> exclusive
        //    scan over rows. The row's padding slots get sentinels (grad rows
        //    out of range, no gu) and its batches are recorded in brow.
        const int nscan = ((R + kWave - 1) / kWave) * kWave;  // whole waves
        int h[kWaves];
        int total = 0;
        int incl = 0;
        int padded = 0;
        if (tid < nscan) {
            const int kr = min(tidl, R - 1);  // in-bounds reads, zeroed past R
            int x[kWaves];
#pragma unroll
            for (int w = 0; w < kWaves; w += 4) {
                const vec_t<int, 4> v = *reinterpret_cast<const vec_t<int, 4> *>(cnt + kr * kWaves + w);
#pragma unroll
                for (int e = 0; e < 4; ++e) x[w + e] = v[e];
            }
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                h[w] = total;
                total += tidl < R ? x[w] : 0;
            }
            padded = (total + K - 1) / K * K;
            incl = wave_inclusive_scan(padded);
        }
        if (R > kWave) {
            if (tid < nscan && lane == kWave - 1) wtot[wave] = incl;
            __syncthreads();
            if (tid < nscan)
                for (int w = 0; w < wave; ++w) incl += wtot[w];
        }
        if (tid < R) {
            const int excl = incl - padded;
            off[tidl] = excl;
            if (tid == R - 1) off[R] = incl;
#pragma unroll
            for (int w = 0; w < kWaves; w += 4) {
                vec_t<int, 4> v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = excl + h[w + e];
                *reinterpret_cast<vec_t<int, 4> *>(cnt + tidl * kWaves + w) = v;
            }
            for (int q = excl + total; q < excl + padded; ++q) {
                ent[q] = make_uint2(kOutOfRange, kPadSlot);
                us[q] = 0.f;
            }
            for (int bb = excl / K; bb < incl / K; ++bb) brow[bb] = tidl;
        }
        __syncthreads();

        // 3. stable placement: item order inside every row. An entry holds
        //    the item's grad-row byte offset, and the LDS byte offset of its
        //    neighbour row nb | r << 18 | item << 21.
        if (tid < n_tile) {
            const int code = rec_code(r0) & (R - 1), r = rec_r(r0) & 7;
            const int pos = cnt[code * kWaves + wave] + rank;
            const uint32_t nbo = static_cast<uint32_t>((code ^ (1 << r)) & (R - 1)) * (P * 4u);
            ent[pos] = make_uint2(static_cast<uint32_t>(tile0 + tidl) * static_cast<uint32_t>(O) * 4u,
                                  nbo | (static_cast<uint32_t>(r) << 18) | (static_cast<uint32_t>(tidl) << 21));
            us[pos] = rec_u(r0);
        }
        __syncthreads();
        // the G touch's only use: a word of its own after the scan carries
        if (tile0 == 0 && tid == 0) wtot[kWaves] = static_cast<int>(pf);

        // 4. walk. The batches (rows in order, K slots each) are dealt out as
        //    contiguous ranges of lo or lo + 1 batches, the longer ones to the
        //    first row groups, so the four groups of a wave get equal counts
        //    except in one wave, however the codes are spread. A group sums
        //    each row's grad rows over its batches in registers: a row lying
        //    wholly in the range is finished there, a row crossing the
        //    range's start (end) leaves its partial sum in the group's slot 0
        //    (1) for the combine step.
        const int nb_all = off[R] / K;
        const int lo = nb_all / NG, extra = nb_all - lo * NG;
        const int g = tidl / S, j = tidl % S;
        const int b_begin = g * lo + min(g, extra), b_end = b_begin + lo + (g < extra ? 1 : 0);
        const int col = j * V;
        const bool col_ok = col < O;
        const uint32_t gcol = static_cast<uint32_t>(col) * 4u;
        const uint32_t coldead = col_ok ? 0u : kOutOfRange;
        const unsigned char *lut_b = reinterpret_cast<const unsigned char *>(lut_s) + col * 4;
        int cur = -1;  // row being summed
        vec_t<float, V> lkv = 0.f;
        float acc[V];
#pragma unroll
        for (int e = 0; e < V; ++e) acc[e] = 0.f;
        auto finish = [&](int k) {  // row k's sum over this range
            const int fb = off[k] / K, lb = off[k + 1] / K - 1;
            if (fb >= b_begin && lb < b_end) {
                if (a.grad_lut != nullptr) {
                    if (single) {
                        if (col_ok) {
                            float y[V];
#pragma unroll
                            for (int e = 0; e < V; ++e) y[e] = acc[e] * a.scale;
                            store_f32_nt<V>(a.grad_lut + (static_cast<size_t>(t) * R + k) * O + col, y);
                        }
                    } else {
                        vec_t<float, V> *rb = reinterpret_cast<vec_t<float, V> *>(rowbuf + k * P + col);
                        vec_t<float, V> w = *rb;
#pragma unroll
                        for (int e = 0; e < V; ++e) w[e] += acc[e];
                        *rb = w;
                    }
                }
            } else {
                vec_t<float, V> w;
#pragma unroll
                for (int e = 0; e < V; ++e) w[e] = acc[e];
                *reinterpret_cast<vec_t<float, V> *>(part + (g * 2 + (fb < b_begin ? 0 : 1)) * P + col) = w;
            }
        };
        for (int i = 0; __ballot(b_begin + i < b_end) != 0; ++i) {  // wave-uniform trip count
            const int bt = b_begin + i;
            const bool live = bt < b_end;
            const int k = live ? brow[bt] : cur;
            if (k != cur) {
                if (cur >= 0) finish(cur);
                cur = k;
                lkv = *reinterpret_cast<const vec_t<float, V> *>(lut_s + k * P + col);
#pragma unroll
                for (int e = 0; e < V; ++e) acc[e] = 0.f;
            }
            // a group past its range reads the K sentinel slots after the
            // list: every load out of range, no gu
            const int base = live ? bt * K : a.slots;
            uint2 en[K];
#pragma unroll
            for (int q = 0; q < K; ++q) en[q] = ent[base + q];
            float gv[K][V];
#pragma unroll
            for (int q = 0; q < K; ++q) buffer_row<float, V>(g_rsrc, (en[q].x + gcol) | coldead, 0, gv[q]);
            float d[K];
#pragma unroll
            for (int q = 0; q < K; ++q) {
                const vec_t<float, V> lnv = *reinterpret_cast<const vec_t<float, V> *>(lut_b + (en[q].y & 0x3ffffu));
                float sd = 0.f;
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    sd += gv[q][e] * (lnv[e] - lkv[e]);
                    acc[e] += gv[q][e];
                }
                d[q] = sd;
            }
            if (need_gu) {  // the slot's dot; gu is formed per slot after the walk
                const float dot = reduce_scatter<S, K>(d, j) * a.scale;
                const int q = (j / (S / K)) & (K - 1);  // the item whose dot this lane holds
                if (j % (S / K) == 0) dt[base + q] = dot;
            }
        }
        if (cur >= 0) finish(cur);
        const int next = tile0 + kFusedThreads;
        if (next < a.items) r0 = next + tid < a.items ? rec_t[next + tid] : 0ull;
        __syncthreads();
        // 5. combine: group g finishes rows g, g + groups, ...: an empty row is
        //    zero; a row split over ranges sums its pieces in range order
        //    (slot 1 of its first range, slot 0 of the others)
        if (a.grad_lut != nullptr) {
            const int bl = lo + 1;  // ranges of the first `extra` groups
            const float inv_bl = 1.0f / static_cast<float>(bl), inv_lo = 1.0f / static_cast<float>(max(lo, 1));
            auto range_of = [&](int bt) {
                return bt < extra * bl ? small_div(bt, inv_bl) : extra + small_div(bt - extra * bl, inv_lo);
            };
            for (int k = g; k < R; k += NG) {
                const int fb = off[k] / K, nbk = off[k + 1] / K - fb;
                const int gf = nbk > 0 ? range_of(fb) : 0, gl = nbk > 0 ? range_of(fb + nbk - 1) : 0;
                if (nbk > 0 && gf == gl) continue;  // finished in the walk
                vec_t<float, V> w = 0.f;
                if (nbk > 0) {
                    // a long row (codes concentrated on few rows) spans many
                    // ranges: the pieces' reads go four at a time, the adds
                    // stay in range order
                    w = *reinterpret_cast<const vec_t<float, V> *>(part + (gf * 2 + 1) * P + col);
                    int gg = gf + 1;
                    for (; gg + 3 <= gl; gg += 4) {
                        vec_t<float, V> pc[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) pc[u] = *reinterpret_cast<const vec_t<float, V> *>(part + (gg + u) * 2 * P + col);
#pragma unroll
                        for (int u = 0; u < 4; ++u) w += pc[u];
                    }
                    for (; gg <= gl; ++gg) w += *reinterpret_cast<const vec_t<float, V> *>(part + gg * 2 * P + col);
                }
                if (single) {
                    if (col_ok) {
                        float y[V];
#pragma unroll
                        for (int e = 0; e < V; ++e) y[e] = w[e] * a.scale;
                        store_f32_nt<V>(a.grad_lut + (static_cast<size_t>(t) * R + k) * O + col, y);
                    }
                } else {
                    vec_t<float, V> *rb = reinterpret_cast<vec_t<float, V> *>(rowbuf + k * P + col);
                    *rb += w;
                }
            }
        }
        // 6. one thread per sorted slot: gu = dot * surrogate'(u), the
        //    {gu, r} record for the scatter kernel, and the threshold
        //    gradient of the tile: -gu at the slot's min-margin comparison,
        //    a fixed tree per wave (lane 8c ends with the wave's sum for
        //    comparison c) added to the wave's slots. Padding slots carry no
        //    gu. The next placement rewrites the sorted list only after two
        //    barriers.
        if (need_gu) {
            const int slots = off[R];
            if (wave * kWave < slots) {
                float tv[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) tv[c] = 0.f;
                for (int q = tidl; q < slots; q += kFusedThreads) {
                    const uint32_t y = ent[q].y;
                    const int r = static_cast<int>((y >> 18) & 7u);
                    const bool pad = (y & kPadSlot) != 0;
                    const float gu = pad ? 0.f : dt[q] * surrogate_grad(us[q], a.surrogate);
                    if (!pad && a.gurec != nullptr)
                        a.gurec[static_cast<size_t>(t) * a.items + tile0 + ((y >> 21) & 1023u)] =
                            static_cast<uint64_t>(__builtin_bit_cast(uint32_t, gu)) | (static_cast<uint64_t>(r) << 32);
#pragma unroll
                    for (int c = 0; c < 8; ++c) tv[c] += r == c ? -gu : 0.f;
                }
                if (a.grad_thr != nullptr) {
                    const float tot = reduce_scatter<kWave, 8>(tv, lane);
                    if ((lane & 7) == 0) tp[wave * 8 + (lane >> 3)] += tot;
                }
            }
        }
        if (next >= a.items) break;
        tile0 = next;
        rank = ballots(r0, min(kFusedThreads, a.items - tile0));
        __syncthreads();
    }

    // 7. several tiles: the row buffer (its last rows came from the combine
    //    step of the last tile), scaled, written once
    if (!single && a.grad_lut != nullptr) {
        __syncthreads();
        constexpr int qp = P / CH;
        for (int unit = tid; unit < R * qp; unit += kFusedThreads) {
            const int k = unit / qp, c0 = (unit % qp) * CH;
            if (c0 < O) {
                float y[CH];
#pragma unroll
                for (int e = 0; e < CH; ++e) y[e] = rowbuf[k * P + c0 + e] * a.scale;
                store_f32_nt<CH>(a.grad_lut + (static_cast<size_t>(t) * R + k) * O + c0, y);
            }
        }
    }
    // 8. threshold gradient: the waves' sums in wave order
    if (a.grad_thr != nullptr) {
        __syncthreads();
        if (tid < C) {
            float sum = tp[tid];
            for (int w = 1; w < kWaves; ++w) sum += tp[w * 8 + tid];
            a.grad_thr[t * C + tid] = sum;
        }
    }
}

// Input gradient of the fused path: one workgroup per item expands the item's
// {gu, r} records (one per table) into signed slots and walks the inverse
// anchor index as the item kernel does.
struct ScatterArgs {
    const uint64_t *gurec;  // [T][B]
    const int32_t *index_offsets;
    const int32_t *index_entries;
    float *grad_x;
    int items, in_f, tables, comps;
};

constexpr int kScatterIndex = 8;  // index words per thread in flight

// BIG: an index longer than the first loads' kScatterIndex words per thread
// (c4: 9,233 words), whose rest is staged eight words per thread at a time.
template <bool BIG>
__global__ __launch_bounds__(kScatterThreads) void pairwise_bwd_scatter_kernel(ScatterArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int C = a.comps;
    float *gud = reinterpret_cast<float *>(lds);                     // [T * C]
    int *idx_s = reinterpret_cast<int *>(gud + a.tables * C);         // [in_f + 1 + 2 T C + kEntries]
    const int b = xcd_block_unit(blockIdx.x, gridDim.x), tid = threadIdx.x;  // records of adjacent items share lines
    const int n_ent = 2 * a.tables * C;
    const int nidx = a.in_f + 1 + n_ent + kEntries;
    for (int t0 = 0; t0 < a.tables; t0 += kScatterThreads) {
        const int tt = t0 + tid;
        const uint64_t rr = tt < a.tables ? a.gurec[static_cast<size_t>(tt) * a.items + b] : 0ull;
        int iv[kScatterIndex];
        const int kb = t0 == 0 ? 0 : nidx;  // the index goes out with the first records
#pragma unroll
        for (int q = 0; q < kScatterIndex; ++q) {
            const int k = kb + tid + q * kScatterThreads;
            iv[q] = k < nidx ? index_word(a.index_offsets, a.index_entries, a.in_f, n_ent, k) : 0;
        }
#pragma unroll
        for (int q = 0; q < kScatterIndex; ++q)
            if (kb + tid + q * kScatterThreads < nidx) idx_s[kb + tid + q * kScatterThreads] = iv[q];
        if (tt < a.tables) {
            const float gu = __builtin_bit_cast(float, static_cast<uint32_t>(rr));
            const int r = static_cast<int>(rr >> 32);
            for (int c = 0; c < C; ++c) gud[tt * C + c] = c == r ? gu : 0.f;
        }
    }
    if constexpr (BIG)
        stage_index(idx_s, a.index_offsets, a.index_entries, a.in_f, n_ent, kScatterIndex * kScatterThreads, nidx,
                    tid, kScatterThreads);
    __syncthreads();
    feature_walk(gud, idx_s, a.in_f, a.grad_x + static_cast<size_t>(b) * a.in_f, tid, kScatterThreads);
}

// Input gradient of inputs too wide (or tables too many) for an item's gu
// slots and the inverse index to sit in LDS: one thread per (item, feature),
// 256 consecutive features of one item per workgroup. The feature's entries
// come from the index in global memory, each entry's value from the
// records: min-margin {gu, r} [T][B] (gu where the entry's comparison is r,
// else zero), full STE gu [T][C][B]. Summed in entry order with the LDS
// walk's one-lane arithmetic (side 1 subtracts), so the values equal that
// walk's wherever both apply.
struct ScatterWideArgs {
    const uint64_t *gurec;  // min-margin
    const float *gu;        // full STE
    const int32_t *index_offsets;
    const int32_t *index_entries;
    float *grad_x;
    int items, in_f, comps, fblocks;
};

constexpr int kWideThreads = 256;

template <bool FULL>
__global__ __launch_bounds__(kWideThreads) void pairwise_bwd_scatter_wide_kernel(ScatterWideArgs a) {
    const int b = blockIdx.x / a.fblocks;
    const int f = (blockIdx.x - b * a.fblocks) * kWideThreads + threadIdx.x;
    if (f >= a.in_f) return;
    const int e0 = a.index_offsets[f], e1 = a.index_offsets[f + 1];
    float gx = 0.f;
    for (int e = e0; e < e1; ++e) {
        const int k = a.index_entries[e];
        const int tc = k >> 1;
        float v;
        if constexpr (FULL) {
            v = a.gu[static_cast<size_t>(tc) * a.items + b];
        } else {
            const int t = tc / a.comps, c = tc - t * a.comps;
            const uint64_t rr = a.gurec[static_cast<size_t>(t) * a.items + b];
            v = static_cast<int>(rr >> 32) == c ? __builtin_bit_cast(float, static_cast<uint32_t>(rr)) : 0.f;
        }
        gx = gx + ((k & 1) ? -v : v);
    }
    __builtin_nontemporal_store(gx, a.grad_x + static_cast<size_t>(b) * a.in_f + f);
}

// Inverse anchor index: for every input feature f, the entries
// ((t * C + c) << 1) | side of the anchors[t][c][side] equal to f, in
// increasing order: a stable counting sort in one workgroup, over windows of
// kIdxWindow features (one window unless the input is wider). Per window: LDS
// counts per feature (integer atomics), one wave's exclusive scan gives the
// offsets (after the entries of the windows before), and the window's entries
// are placed in chunks of 1024 in entry order: inside a wave the lanes with
// the same feature are found with one ballot per feature bit (a lane's rank
// is the number of such lanes below it), and the chunk's waves take turns,
// each advancing the features' LDS cursors, so the order is fixed. Anchors
// outside [0, in_f) are left out.
constexpr int kIdxThreads = 1024;
constexpr int kIdxWindow = 8192;  // features per pass: their cursors in LDS

__global__ __launch_bounds__(kIdxThreads) void anchor_index_kernel(const int64_t *anchors, int in_f, int tables,
                                                                  int comps, int32_t *offsets, int32_t *entries) {
    extern __shared__ __align__(16) unsigned char lds[];
    int *cursor = reinterpret_cast<int *>(lds);  // [window + 1]: counts, then each feature's next position
    const int n = tables * comps * 2, tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const uint64_t below = (1ull << lane) - 1ull, upto = below | (1ull << lane);
    int placed = 0;  // entries of the windows before
    for (int lo = 0, w = 0; lo < in_f; lo += w) {  // lo + w <= in_f: no overflow at any in_f
        w = min(kIdxWindow, in_f - lo);
        for (int f = tid; f <= w; f += kIdxThreads) cursor[f] = 0;
        __syncthreads();
        for (int k = tid; k < n; k += kIdxThreads) {
            const int64_t v = anchors[k] - lo;
            if (v >= 0 && v < w) atomicAdd(&cursor[v], 1);
        }
        __syncthreads();
        if (tid < kWave) wave_exclusive_scan(cursor, w, tid);
        __syncthreads();
        for (int f = tid; f < w; f += kIdxThreads) {
            cursor[f] += placed;
            offsets[lo + f] = cursor[f];
        }
        const int here = cursor[w];  // the window's entries (cursor[w] is left alone above)
        __syncthreads();
        const int fbits = w > 1 ? 32 - __clz(w - 1) : 0;
        for (int k0 = 0; k0 < n; k0 += kIdxThreads) {
            const int k = k0 + tid;
            int v = -1;
            if (k < n) {
                const int64_t a = anchors[k] - lo;
                v = a >= 0 && a < w ? static_cast<int>(a) : -1;
            }
            const bool valid = v >= 0;
            uint64_t same = __ballot(valid);
            for (int b = 0; b < fbits; ++b) {
                const bool bit = (v >> b) & 1;
                const uint64_t ones = __ballot(valid && bit);
                same &= bit ? ones : ~ones;
            }
            const int rank = __popcll(same & below);
            const bool last = (same & ~upto) == 0;
            for (int wv = 0; wv < kIdxThreads / kWave; ++wv) {
                if (wave == wv && valid) {
                    const int pos = cursor[v] + rank;  // every lane reads before the group's last lane writes
                    entries[pos] = k;
                    if (last) cursor[v] = pos + 1;
                }
                __syncthreads();
            }
        }
        placed += here;
    }
    if (tid == 0) offsets[in_f] = placed;
}

// Kernels that may need more than the default 64 KB of dynamic LDS opt in
// once per size.
template <typename K>
hipError_t allow_lds(K kernel, int bytes) {
    return allow_dynamic_lds(reinterpret_cast<const void *>(kernel), bytes);
}

template <typename T, int V, int S, bool DOTS>
hipError_t launch_rows_vs(const RowsArgs &args, const BackwardPlan &p, int tables, hipStream_t stream) {
    auto kernel = DOTS && p.rows_nb_pack ? pairwise_bwd_rows_kernel<T, V, S, DOTS, DOTS>
                                         : pairwise_bwd_rows_kernel<T, V, S, DOTS, false>;
    const int lds = DOTS ? p.rows_lds_dots_bytes : p.rows_lds_bytes;
    constexpr int threads = rows_threads(DOTS, sizeof(T));
    if (threads != (DOTS ? p.rows_dots_threads : kRowsThreads)) return hipErrorInvalidConfiguration;  // plan mismatch
    if constexpr (rows_nb_perm(DOTS, sizeof(T), S, V)) {
        // the byte-permute neighbour reads address the LUT chunk from LDS
        // address 0: the kernel must have no static LDS (the dynamic array
        // then starts at 0) and the chunk must open the dynamic array
        if (p.rows_nb_pack) {
            static const size_t static_lds = [kernel] {
                hipFuncAttributes at{};
                return hipFuncGetAttributes(&at, reinterpret_cast<const void *>(kernel)) == hipSuccess
                           ? at.sharedSizeBytes
                           : ~size_t{0};
            }();
            if (static_lds != 0 || args.lut_off != 0) return hipErrorInvalidConfiguration;
        }
    }
    if (hipError_t e = allow_lds(kernel, lds); e != hipSuccess) return e;
    return launch_kernel(TROPNN_KERNEL_BACKWARD_TABLE, kernel, dim3(tables * p.rows_chunks), dim3(threads), lds,
                         stream, args);
}

template <typename T, int V, bool DOTS>
hipError_t launch_rows_v(const RowsArgs &args, const BackwardPlan &p, int tables, hipStream_t stream) {
    switch (p.rows_slices) {
        case 64: return launch_rows_vs<T, V, 64, DOTS>(args, p, tables, stream);
        case 32: return launch_rows_vs<T, V, 32, DOTS>(args, p, tables, stream);
        case 16: return launch_rows_vs<T, V, 16, DOTS>(args, p, tables, stream);
        case 8: return launch_rows_vs<T, V, 8, DOTS>(args, p, tables, stream);
        default: return launch_rows_vs<T, V, 4, DOTS>(args, p, tables, stream);
    }
}

template <typename T, bool DOTS>
hipError_t launch_rows_t(const RowsArgs &args, const BackwardPlan &p, int tables, hipStream_t stream) {
    switch (p.rows_vec) {
        case 8: return launch_rows_v<T, 8, DOTS>(args, p, tables, stream);
        case 4: return launch_rows_v<T, 4, DOTS>(args, p, tables, stream);
        case 2: return launch_rows_v<T, 2, DOTS>(args, p, tables, stream);
        default: return launch_rows_v<T, 1, DOTS>(args, p, tables, stream);
    }
}

// dots: partial STE dots as well (min-margin); the LUT's element type only
// matters then
hipError_t launch_rows(const RowsArgs &args, const BackwardPlan &p, int tables, int lut_dtype, bool dots,
                       hipStream_t stream) {
    if (!dots) return launch_rows_t<float, false>(args, p, tables, stream);
    return lut_dtype == TROPNN_LUT_F16 ? launch_rows_t<_Float16, true>(args, p, tables, stream)
                                       : launch_rows_t<float, true>(args, p, tables, stream);
}

template <typename T, int N>
hipError_t launch_item_typed(const ItemArgs &args, const BackwardPlan &p, hipStream_t stream) {
    auto kernel = pairwise_bwd_full_kernel<T, N>;
    if (hipError_t e = allow_lds(kernel, p.item_lds_bytes); e != hipSuccess) return e;
    return launch_kernel(TROPNN_KERNEL_BACKWARD_ITEM, kernel, dim3(args.items), dim3(p.item_threads), p.item_lds_bytes,
                         stream, args);
}

template <typename T, int V, int S>
hipError_t launch_fused_vs(const FusedArgs &args, int wgs, const BackwardPlan &p, hipStream_t stream) {
    auto kernel = pairwise_bwd_fused_kernel<T, V, S>;
    if (hipError_t e = allow_lds(kernel, p.f_launch_lds); e != hipSuccess) return e;
    return launch_kernel(TROPNN_KERNEL_BACKWARD_FUSED, kernel, dim3(wgs), dim3(kFusedThreads), p.f_launch_lds,
                         stream, args);
}

template <typename T>
hipError_t launch_fused_typed(const FusedArgs &args, int wgs, const BackwardPlan &p, hipStream_t stream) {
    if (p.fvec == 2) return launch_fused_vs<T, 2, 16>(args, wgs, p, stream);
    if (p.fvec == 4) return launch_fused_vs<T, 4, 16>(args, wgs, p, stream);
    if (p.fslices == 16) return launch_fused_vs<T, 8, 16>(args, wgs, p, stream);
    return launch_fused_vs<T, 8, 32>(args, wgs, p, stream);
}

// Compute units of the device a stream runs on, looked up once per device
// (gfx950: 256). 0 if the runtime cannot say.
int device_cus(hipStream_t stream) {
    static std::atomic<int> cache[64];
    int dev = 0;
    if ((stream != nullptr ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev)) != hipSuccess || dev < 0 ||
        dev >= 64)
        return 0;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 0) v = 0;
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

__global__ void fill_zero_kernel(float *p, size_t n) {
    for (size_t k = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; k < n;
         k += static_cast<size_t>(gridDim.x) * blockDim.x)
        p[k] = 0.f;
}

}  // namespace

hipError_t allow_dynamic_lds(const void *kernel, int bytes) {
    static std::mutex mu;
    static std::unordered_map<const void *, int> allowed;  // the largest size each kernel opted in for
    if (bytes <= 64 * 1024) return hipSuccess;
    std::lock_guard<std::mutex> lock(mu);
    int &done = allowed[kernel];
    if (bytes <= done) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) done = bytes;
    return e;
}

hipError_t launch_fill_zero(float *p, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p, n);
    return hipGetLastError();
}

hipError_t launch_anchor_index(const int64_t *anchors, int in_f, int tables, int comps, int32_t *offsets,
                               int32_t *entries, hipStream_t stream) {
    hipLaunchKernelGGL(anchor_index_kernel, dim3(1), dim3(kIdxThreads), (min(in_f, kIdxWindow) + 1) * 4, stream,
                       anchors, in_f, tables, comps, offsets, entries);
    return hipGetLastError();
}

hipError_t launch_scatter_wide(const uint64_t *gurec, const float *gu, const int32_t *index_offsets,
                               const int32_t *index_entries, float *grad_x, const Dims &d, hipStream_t stream) {
    ScatterWideArgs s{};
    s.gurec = gurec;
    s.gu = gu;
    s.index_offsets = index_offsets;
    s.index_entries = index_entries;
    s.grad_x = grad_x;
    s.items = d.items;
    s.in_f = d.in_f;
    s.comps = d.comps;
    s.fblocks = static_cast<int>((static_cast<long long>(d.in_f) + kWideThreads - 1) / kWideThreads);
    const long long blocks = static_cast<long long>(d.items) * s.fblocks;
    if (blocks > std::numeric_limits<int>::max()) return hipErrorInvalidConfiguration;
    auto kernel = gu != nullptr ? pairwise_bwd_scatter_wide_kernel<true> : pairwise_bwd_scatter_wide_kernel<false>;
    return launch_kernel(TROPNN_KERNEL_BACKWARD_SCATTER, kernel, dim3(static_cast<unsigned>(blocks)),
                         dim3(kWideThreads), 0, stream, s);
}

hipError_t launch_scatter(const uint64_t *gurec, const int32_t *index_offsets, const int32_t *index_entries,
                          float *grad_x, const Dims &d, const BackwardPlan &p, hipStream_t stream) {
    if (p.wide_index) return launch_scatter_wide(gurec, nullptr, index_offsets, index_entries, grad_x, d, stream);
    ScatterArgs s{};
    s.gurec = gurec;
    s.index_offsets = index_offsets;
    s.index_entries = index_entries;
    s.grad_x = grad_x;
    s.items = d.items;
    s.in_f = d.in_f;
    s.tables = d.tables;
    s.comps = d.comps;
    const long long nidx = d.in_f + 1 + 2ll * d.tables * d.comps + kEntries;
    auto kernel = nidx > kScatterIndex * kScatterThreads ? pairwise_bwd_scatter_kernel<true>
                                                         : pairwise_bwd_scatter_kernel<false>;
    if (hipError_t e = allow_lds(kernel, p.scatter_lds_bytes); e != hipSuccess) return e;
    return launch_kernel(TROPNN_KERNEL_BACKWARD_SCATTER, kernel, dim3(d.items),
                         dim3(kScatterThreads), p.scatter_lds_bytes, stream, s);
}

BackwardPlan plan_backward(const Dims &d, int ste_mode) {
    BackwardPlan p{};
    p.full = (ste_mode & 0xff) == TROPNN_STE_FULL;
    const int esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    // row kernel: V columns per lane (8 for rows of 64 columns or more that
    // 8 divides, else the largest divisor of the row up to 4), S lanes per
    // row group: the smallest power of two from 4 whose S * V columns cover
    // min(O, 64); 64-column chunks keep one chunk of the grad rows within an
    // XCD's L2 while the tables of the chunk are walked. Eight columns per
    // lane halve the per-slot addressing and reduce-scatter work per column.
    p.rows_vec = d.out_f >= kRowsChunk && d.out_f % 8 == 0 ? 8 : 4;
    while (p.rows_vec > 1 && d.out_f % p.rows_vec != 0) p.rows_vec >>= 1;
    p.rows_batch = rows_batch(p.rows_vec);
    p.rows_slices = 4;
    while (p.rows_slices < 64 && p.rows_slices * p.rows_vec < (d.out_f < kRowsChunk ? d.out_f : kRowsChunk)) p.rows_slices <<= 1;
    const int rows_chunk = p.rows_slices * p.rows_vec;
    p.rows_chunk = rows_chunk;
    p.rows_chunks = (d.out_f + rows_chunk - 1) / rows_chunk;
    p.rows_part_off = ((d.rows + 1) * 4 + 15) & ~15;
    // then the row groups' slot-offset rings, 16 bytes per thread
    p.rows_ring_off = p.rows_part_off + (kRowsThreads / p.rows_slices) * 2 * rows_chunk * 4;
    p.rows_lds_bytes = p.rows_ring_off + kRowsThreads * 16;
    // with dots: the LUT chunk [R][P] f32 at offset 0 (its rows' addresses
    // are then byte permutes), then the row starts and the split-row slots
    p.rows_lut_off = 0;
    // (in the LUT's element type for an f16 LUT, with rows_threads' 512-thread
    // workgroups)
    p.rows_dots_threads = rows_threads(true, esize);
    p.rows_dots_rs_off = (d.rows * rows_chunk * esize + 15) & ~15;
    p.rows_dots_part_off = (p.rows_dots_rs_off + (d.rows + 1) * 4 + 15) & ~15;
    p.rows_dots_ring_off = p.rows_dots_part_off + (p.rows_dots_threads / p.rows_slices) * 2 * rows_chunk * 4;
    p.rows_lds_dots_bytes = p.rows_dots_ring_off + p.rows_dots_threads * 16;
    // the neighbour row fits below the item offset (a multiple of P * 4 bytes)
    p.rows_nb_pack = rows_chunk * 4 >= d.rows;
    p.sort_lds_bytes = ((kSortThreads / kWave) * d.rows + d.rows + kSortThreads / kWave) * 4 + (kSortThreads / kWave) * 8 * 4;
    // the sorted slots of a table: its items plus up to K - 1 padding slots
    // per row, rounded up to whole batches
    p.sort_slots = (d.items + d.rows * (p.rows_batch - 1) + p.rows_batch - 1) / p.rows_batch * p.rows_batch;

    // item kernel: N elements per lane as in the forward (the smallest power
    // of two whose 64-lane tile spans the row, 16 bytes at most, dividing the
    // row), waves of at most 16 tables, ~4096 waves in flight, at most 16
    // waves (so at most 256 tables)
    p.item_vec = 1;
    while (p.item_vec * esize < 16 && p.item_vec * kWave < d.out_f) p.item_vec <<= 1;
    while (p.item_vec > 1 && d.out_f % p.item_vec != 0) p.item_vec >>= 1;
    p.item_o_tiles = (d.out_f + kWave * p.item_vec - 1) / (kWave * p.item_vec);
    const int loaded = item_wave_tables(esize, p.item_vec);
    int w = (d.tables + loaded - 1) / loaded;
    const long long want = d.items > 0 ? (4096 + d.items - 1) / d.items : 16;
    if (want > w) w = static_cast<int>(want < 16 ? want : 16);
    if (w > 16) w = 16;  // more tables: each wave loops over blocks
    if (w > d.tables) w = d.tables;
    p.item_per_wave = (d.tables + w - 1) / w;
    p.item_waves = (d.tables + p.item_per_wave - 1) / p.item_per_wave;
    p.item_threads = p.item_waves * kWave;
    // an item's gu slots [T * C] f32 and the inverse anchor index in LDS; past
    // a workgroup's LDS (wide inputs, many tables) the input gradient is
    // formed by the wide scatter kernel from the index and the records in
    // global memory instead
    const long long tc = static_cast<long long>(d.tables) * d.comps;
    const long long item_lds = (tc + d.in_f + 1 + 2 * tc + kEntries) * 4;
    p.wide_index = item_lds > kMaxLdsBytes;
    p.item_lds_bytes = p.wide_index ? 0 : static_cast<int>(item_lds);
    p.scatter_lds_bytes = p.item_lds_bytes;

    // fused path: the row group spans the row, lanes own whole V-column
    // pieces of it (V = 2 for up to 32 columns with O % 4 != 0, V = 4 up to
    // 64 columns, else V = 8 and O % 8 == 0), and the table's rows fit in LDS
    p.fused = false;
    if (!p.full && ((d.out_f % 4 == 0 && (d.out_f <= 64 || (d.out_f % 8 == 0 && d.out_f <= 256))) ||
                    (d.out_f % 2 == 0 && d.out_f <= 32))) {
        p.fvec = d.out_f % 4 != 0 ? 2 : d.out_f <= 64 ? 4 : 8;
        p.fslices = d.out_f <= 128 ? 16 : 32;
        p.fpitch = p.fvec * p.fslices;
        const bool single = d.items <= kFusedThreads;
        const int waves = kFusedThreads / kWave;
        int off = 0;
        p.f_lut_off = off;
        off += d.rows * p.fpitch * 4;
        p.f_rowbuf_off = off;
        off += single ? 0 : d.rows * p.fpitch * 4;
        p.f_cnt_off = off;
        off += waves * d.rows * 4;
        p.f_off_off = off;
        off += ((d.rows + 1) * 4 + 15) & ~15;
        const int batch = kFusedFloats / p.fvec;
        p.f_slots = kFusedThreads + d.rows * (batch - 1);
        off = (off + 7) & ~7;
        p.f_sorted_off = off;
        off += (p.f_slots + batch) * 8;  // entries, then the sentinel slots
        p.f_u_off = off;
        off += (p.f_slots + batch) * 4;
        p.f_dt_off = off;
        off += (p.f_slots + batch) * 4;
        p.f_thr_off = off;
        off += waves * 8 * 4;
        p.f_wtot_off = off;
        off += (waves + 1) * 4;
        off = (off + 15) & ~15;  // 16-byte vector accesses
        p.f_part_off = off;
        off += (kFusedThreads / p.fslices) * 2 * p.fpitch * 4;
        p.f_brow_off = off;
        off += (p.f_slots / batch + 1) * 4;
        p.f_lds_bytes = off;
        p.fused = d.rows * p.fpitch * 4 <= 64 * 1024 && off <= kMaxLdsBytes;
        // item role: the most items (up to kItemChunk) whose records [nc][T]
        // u64, G rows [nc][O] (+ one row pitch of zeros) and signed slots
        // [nc][T * C] f32, with the inverse anchor index, fit the table role's
        // LDS (or, for one item, up to 160 KB)
        const long long idx_bytes = (d.in_f + 1 + 2 * tc + kEntries) * 4;
        auto a16 = [](long long v) { return (v + 15) & ~15ll; };
        auto item_bytes = [&](int nc) {
            return a16(nc * 8ll * d.tables) + a16((static_cast<long long>(nc) * d.out_f + p.fpitch) * 4) +
                   a16(nc * 4ll * tc) + idx_bytes;
        };
        const long long cap = p.f_lds_bytes > item_bytes(1) ? p.f_lds_bytes : item_bytes(1);
        int nc = 0;
        while (nc < kItemChunk && item_bytes(nc + 1) <= cap) ++nc;
        // (a caller's flag overrides the row-width rule, not the limits)
        const bool by_width = (ste_mode & TROPNN_BWD_INPUT_GRAD_FUSED) != 0 ||
                              static_cast<long long>(d.tables) * d.out_f * esize <=
                                  static_cast<long long>(kItemRoleRowBytes) * (kCus - d.tables);
        p.f_item = p.fused && d.tables <= kItemRoleMaxTables && nc >= 1 && item_bytes(1) <= kMaxLdsBytes && by_width &&
                   (ste_mode & TROPNN_BWD_INPUT_GRAD_SCATTER) == 0;
        p.f_item_nc = nc;
        p.f_ir_rec_off = 0;
        // (offsets and sizes used only with the item role, within the LDS then)
        p.f_ir_g_off = static_cast<int>(a16(nc * 8ll * d.tables));
        p.f_ir_gud_off = p.f_ir_g_off + static_cast<int>(a16((static_cast<long long>(nc) * d.out_f + p.fpitch) * 4));
        p.f_ir_idx_off = p.f_ir_gud_off + static_cast<int>(a16(nc * 4ll * tc));
        p.f_launch_lds = p.f_item ? static_cast<int>(cap) : p.f_lds_bytes;
    }
    // workspace: fused path {gu, r} [T][B] u64; general path {gu, r} [T][B]
    // u64 (min-margin) or gu [T][C][B] f32 (full STE), then the sort
    // kernel's slot offsets [T][slots] u32, row starts [T][R + 1] i32, batch
    // rows [T][slots / K] i32, the chunk-major copy of G [chunks][B][P] f32
    // and (min-margin) the row kernel's partial dots [T][chunks][slots] f32,
    // each region 16-byte aligned
    auto align16 = [](size_t v) { return (v + 15) & ~static_cast<size_t>(15); };
    if (p.fused) {
        p.workspace_bytes = p.f_item ? 0 : static_cast<size_t>(d.tables) * d.items * sizeof(uint64_t);
    } else {
        size_t off = align16(static_cast<size_t>(d.tables) * d.items * (p.full ? d.comps * sizeof(float) : sizeof(uint64_t)));
        p.ws_slot_off = off;
        off = align16(off + static_cast<size_t>(d.tables) * p.sort_slots * sizeof(uint32_t));
        p.ws_row_start = off;
        off = align16(off + static_cast<size_t>(d.tables) * (d.rows + 1) * sizeof(int32_t));
        p.ws_batch_row = off;
        off = align16(off + static_cast<size_t>(d.tables) * (p.sort_slots / p.rows_batch) * sizeof(int32_t));
        p.ws_g_chunked = off;
        off = align16(off + static_cast<size_t>(p.rows_chunks) * d.items * rows_chunk * sizeof(float));
        p.ws_pdot = off;
        if (!p.full) off = align16(off + static_cast<size_t>(d.tables) * p.rows_chunks * p.sort_slots * sizeof(float));
        p.workspace_bytes = off;
    }
    return p;
}

hipError_t launch_backward(const Dims &d, const BackwardPlan &p, const float *grad_out, const void *lut,
                           const tropnn_route_record *rec, const float *margins, const int32_t *index_offsets,
                           const int32_t *index_entries, float scale, int surrogate, float *grad_x,
                           float *grad_thr, float *grad_lut, float *workspace, hipStream_t stream) {
    const uint64_t *rec64 = reinterpret_cast<const uint64_t *>(rec);
    const int esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    const uint32_t g_bytes = static_cast<uint32_t>(static_cast<size_t>(d.items) * d.out_f * 4);
    if (p.fused) {
        if (grad_x == nullptr && grad_thr == nullptr && grad_lut == nullptr) return hipSuccess;
        // the item role forms grad_latent in the same launch (no scatter
        // kernel); otherwise the table role leaves {gu, r} records for it
        const bool item_role = p.f_item && grad_x != nullptr;
        uint64_t *gurec = grad_x != nullptr && !item_role ? reinterpret_cast<uint64_t *>(workspace) : nullptr;
        FusedArgs f{};
        f.grad_out = grad_out;
        f.lut = lut;
        f.rec = rec64;
        f.scale = scale;
        f.grad_lut = grad_lut;
        f.grad_thr = grad_thr;
        f.gurec = gurec;
        f.surrogate = surrogate;
        f.lut_bytes = static_cast<uint32_t>(static_cast<size_t>(d.tables) * d.rows * d.out_f * esize);
        f.g_bytes = g_bytes;
        f.items = d.items;
        f.out_f = d.out_f;
        f.tables = d.tables;
        f.comps = d.comps;
        f.rows = d.rows;
        f.g_slice = static_cast<uint32_t>(((g_bytes + (d.tables + 7) / 8 - 1) / ((d.tables + 7) / 8) + 127) & ~127u);
        const int per_row = d.out_f / (p.fvec < 4 ? p.fvec : 4);  // staging chunks per LUT row
        f.quad_magic = ((uint64_t{1} << 32) + per_row - 1) / per_row;
        f.part_off = p.f_part_off;
        f.brow_off = p.f_brow_off;
        f.slots = p.f_slots;
        f.lut_off = p.f_lut_off;
        f.cnt_off = p.f_cnt_off;
        f.off_off = p.f_off_off;
        f.sorted_off = p.f_sorted_off;
        f.u_off = p.f_u_off;
        f.dt_off = p.f_dt_off;
        f.rowbuf_off = p.f_rowbuf_off;
        f.thr_off = p.f_thr_off;
        f.wtot_off = p.f_wtot_off;
        // table workgroups first (one per table, unless only grad_latent is
        // asked for), then the item workgroups on the CUs the table ones
        // leave free: n items each, all resident at once on MI355X
        f.table_wgs = !item_role || grad_lut != nullptr || grad_thr != nullptr ? d.tables : 0;
        int wgs = f.table_wgs;
        if (item_role) {
            int ni = device_cus(stream) - f.table_wgs;
            if (ni < kItemRoleMinWgs) ni = kItemRoleMinWgs;
            if (ni > d.items) ni = d.items;
            const int n = (d.items + ni - 1) / ni;
            f.item_n = n;
            f.item_nc = n < p.f_item_nc ? n : p.f_item_nc;
            f.grad_x = grad_x;
            f.index_offsets = index_offsets;
            f.index_entries = index_entries;
            f.in_f = d.in_f;
            f.ir_rec_off = p.f_ir_rec_off;
            f.ir_g_off = p.f_ir_g_off;
            f.ir_gud_off = p.f_ir_gud_off;
            f.ir_idx_off = p.f_ir_idx_off;
            wgs += (d.items + n - 1) / n;
        }
        hipError_t e = d.lut_dtype == TROPNN_LUT_F16 ? launch_fused_typed<_Float16>(f, wgs, p, stream)
                                                      : launch_fused_typed<float>(f, wgs, p, stream);
        if (e != hipSuccess || grad_x == nullptr || item_role) return e;
        return launch_scatter(gurec, index_offsets, index_entries, grad_x, d, p, stream);
    }
    const bool need_gu = grad_x != nullptr || grad_thr != nullptr;
    if (p.full && need_gu) {  // full STE: per-item dots of every comparison, grad_latent
        ItemArgs a{};
        a.grad_out = grad_out;
        a.lut = lut;
        a.rec = rec64;
        a.margins = margins;
        a.index_offsets = index_offsets;
        a.index_entries = index_entries;
        a.scale = scale;
        a.surrogate = surrogate;
        // wide inputs: the kernel leaves every gu in the workspace and the
        // wide scatter kernel forms grad_latent from them
        a.grad_x = p.wide_index ? nullptr : grad_x;
        a.gu = grad_thr != nullptr || (p.wide_index && grad_x != nullptr) ? workspace : nullptr;
        a.lut_bytes = static_cast<uint32_t>(static_cast<size_t>(d.tables) * d.rows * d.out_f * esize);
        a.g_bytes = g_bytes;
        a.items = d.items;
        a.in_f = d.in_f;
        a.out_f = d.out_f;
        a.tables = d.tables;
        a.comps = d.comps;
        a.rows = d.rows;
        a.row_bytes = d.out_f * esize;
        a.table_bytes = d.rows * d.out_f * esize;
        a.per_wave = p.item_per_wave;
        a.o_tiles = p.item_o_tiles;
        hipError_t e;
        if (d.lut_dtype == TROPNN_LUT_F16) {
            switch (p.item_vec) {
                case 8: e = launch_item_typed<_Float16, 8>(a, p, stream); break;
                case 4: e = launch_item_typed<_Float16, 4>(a, p, stream); break;
                case 2: e = launch_item_typed<_Float16, 2>(a, p, stream); break;
                default: e = launch_item_typed<_Float16, 1>(a, p, stream); break;
            }
        } else {
            switch (p.item_vec) {
                case 4: e = launch_item_typed<float, 4>(a, p, stream); break;
                case 2: e = launch_item_typed<float, 2>(a, p, stream); break;
                default: e = launch_item_typed<float, 1>(a, p, stream); break;
            }
        }
        if (e != hipSuccess) return e;
        if (p.wide_index && grad_x != nullptr) {
            e = launch_scatter_wide(nullptr, workspace, index_offsets, index_entries, grad_x, d, stream);
            if (e != hipSuccess) return e;
        }
    }
    // min-margin: the row kernel forms the STE dots, so it runs whenever any
    // gradient is asked for; the full STE needs it for the LUT gradient only
    const bool dots = !p.full && need_gu;
    if (grad_lut == nullptr && !dots && !(p.full && grad_thr != nullptr)) return hipSuccess;
    unsigned char *ws = reinterpret_cast<unsigned char *>(workspace);
    SortArgs so{};
    so.rec = rec64;
    so.gu = p.full ? workspace : nullptr;
    so.slot_off = grad_lut != nullptr || dots ? reinterpret_cast<uint32_t *>(ws + p.ws_slot_off) : nullptr;
    so.row_start = reinterpret_cast<int32_t *>(ws + p.ws_row_start);
    so.batch_row = reinterpret_cast<int32_t *>(ws + p.ws_batch_row);
    so.grad_thr = p.full ? grad_thr : nullptr;
    so.grad_out = grad_out;
    so.g_chunked = reinterpret_cast<float *>(ws + p.ws_g_chunked);
    so.chunk_cols = p.rows_chunk;
    so.chunk_vec = p.rows_vec;
    so.chunks = p.rows_chunks;
    so.batch = p.rows_batch;
    so.full = p.full ? 1 : 0;
    so.nb_pack = dots && p.rows_nb_pack ? 1 : 0;
    so.items = d.items;
    so.out_f = d.out_f;
    so.comps = d.comps;
    so.rows = d.rows;
    so.slots = p.sort_slots;
    if (hipError_t e = launch_kernel(TROPNN_KERNEL_BACKWARD_SORT, pairwise_bwd_sort_kernel, dim3(d.tables),
                                     dim3(kSortThreads), p.sort_lds_bytes, stream, so);
        e != hipSuccess || so.slot_off == nullptr)
        return e;
    RowsArgs r{};
    r.g_chunked = so.g_chunked;
    r.slot_off = so.slot_off;
    r.row_start = so.row_start;
    r.batch_row = so.batch_row;
    r.grad_lut = grad_lut;
    r.scale = scale;
    r.chunk_bytes = static_cast<uint32_t>(static_cast<size_t>(d.items) * p.rows_chunk * 4);
    r.gc_bytes = static_cast<uint32_t>(static_cast<size_t>(p.rows_chunks) * r.chunk_bytes);
    r.out_f = d.out_f;
    r.rows = d.rows;
    r.tables = d.tables;
    r.slots = p.sort_slots;
    r.part_off = dots ? p.rows_dots_part_off : p.rows_part_off;
    r.ring_off = dots ? p.rows_dots_ring_off : p.rows_ring_off;
    r.rs_off = dots ? p.rows_dots_rs_off : 0;
    r.lut = lut;
    r.lut_bytes = static_cast<uint32_t>(static_cast<size_t>(d.tables) * d.rows * d.out_f * esize);
    r.pdot = dots ? reinterpret_cast<float *>(ws + p.ws_pdot) : nullptr;
    r.items = d.items;
    r.chunks = p.rows_chunks;
    r.lut_off = p.rows_lut_off;
    if (hipError_t e = launch_rows(r, p, d.tables, d.lut_dtype, dots, stream); e != hipSuccess || !dots) return e;
    ReduceArgs ra{};
    ra.pdot = r.pdot;
    ra.slot_off = so.slot_off;
    ra.row_start = so.row_start;
    ra.rows = d.rows;
    ra.slots = p.sort_slots;
    ra.item_shift = __builtin_ctz(static_cast<unsigned>(p.rows_chunk) * 4u);
    ra.rec = rec64;
    ra.gurec = grad_x != nullptr ? reinterpret_cast<uint64_t *>(workspace) : nullptr;
    ra.grad_thr = grad_thr;
    ra.scale = scale;
    ra.surrogate = surrogate;
    ra.items = d.items;
    ra.chunks = p.rows_chunks;
    ra.comps = d.comps;
    ra.stage = ra.gurec != nullptr && d.items <= kReduceStageBytes / 8;
    if (hipError_t e = launch_kernel(TROPNN_KERNEL_BACKWARD_REDUCE, pairwise_bwd_reduce_kernel, dim3(d.tables),
                                     dim3(kReduceThreads), ra.stage ? d.items * 8 : 0, stream, ra);
        e != hipSuccess || grad_x == nullptr)
        return e;
    return launch_scatter(ra.gurec, index_offsets, index_entries, grad_x, d, p, stream);
}

}  // namespace tropnn
