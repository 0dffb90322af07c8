// Internal host-side launch API between the C ABI (abi.hip) and the kernels
// (forward.hip, backward.hip). Not exported.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "tropnn_hip.h"

namespace tropnn {

// Problem dims shared by every launch.
struct Dims {
    int items;      // B (batch * seq)
    int in_f;       // I
    int out_f;      // O
    int tables;     // T
    int comps;      // C
    int rows;       // R = 2^C
    int lut_dtype;  // TROPNN_LUT_F32 / TROPNN_LUT_F16
};

// LDS of one workgroup on gfx950.
constexpr int kMaxLdsBytes = 160 * 1024;

// Launch shape of the fused route + gather + scale forward.
struct ForwardPlan {
    int vec;             // N: LUT elements per lane load (16 bytes at most)
    int lpt_log2;        // lanes per table in a route ballot (>= C)
    int o_tile;          // output columns per workgroup (64 * N)
    int o_tiles;         // grid.y
    int per_wave;        // tables per wave (contiguous block)
    int waves_per_item;  // waves of a workgroup (one item per workgroup)
    int threads;         // waves_per_item * 64
    int blocks;          // grid.x = items
    int codes_pitch;     // LDS bytes of a wave's code list
    int codes_off;       // LDS byte offsets
    int red_off;
    int lds_bytes;
    bool wide_x;         // input row beyond the LDS budget: the one-item kernel reads it from global memory
    bool multi;          // large batch: several items per workgroup (blocks = ceil(items / kMultiItems))
    // wave-item kernel (large batch, 128..1024-byte row tiles): every wave
    // owns 64 / (tile bytes / 16) items; replaces the multi-item kernel
    bool wave;
    int wave_lpr_log2;   // log2 lanes per row tile (tile bytes / 16)
    int wave_tile_bytes;
    int wave_tiles;      // grid.y
    int wave_blocks;     // grid.x
    int wave_x_off;      // LDS byte offset of the input rows (comparators at 0)
    int wave_lds_bytes;
    // streamed gather (training, large batch and LUT): a route kernel writes
    // the records, then one workgroup per (item block, 64-column chunk)
    // walks the tables with each table's LUT chunk in LDS
    bool stream_ok;
    int stream_nblk;        // item blocks
    int stream_blocks;      // workgroups
    int stream_lds;
    int route_block_items;  // items per route workgroup (their input rows in LDS)
    int route_lds;
    bool route_rec_stage;  // the route records gathered in LDS before their stores
};

// Launch shape of the backward. General path, min-margin STE: the sort kernel
// (items of each table in code order), the row kernel (LUT gradient and
// partial STE dots per column chunk), the reduce kernel (gu, threshold
// gradient) and the scatter kernel (input gradient). Full STE: the item
// kernel (every comparison's dot, gu, input gradient), the sort kernel
// (threshold gradient too) and the row kernel (LUT gradient).
struct BackwardPlan {
    // row kernel
    int rows_vec;       // V: columns per lane (divides the row: 8, 4, 2 or 1)
    int rows_batch;     // sorted slots per row-kernel batch (rows padded to whole batches)
    int rows_slices;    // S: lanes per row group (4 to 64)
    int rows_chunk;     // P = S * V columns per workgroup
    int rows_chunks;    // column chunks of P
    int rows_part_off;  // LDS byte offset of the split-row slots
    int rows_ring_off;  // LDS byte offset of the row groups' slot-offset rings
    int rows_lds_bytes;
    int rows_lut_off;   // with partial STE dots: LDS byte offset of the LUT chunk (0)
    int rows_dots_rs_off, rows_dots_part_off, rows_dots_ring_off;  // with partial STE dots: row starts, split-row slots, rings
    int rows_lds_dots_bytes;
    int rows_dots_threads;  // threads of the row kernel's workgroup with dots (512 for an f16 LUT, else 1024)
    bool rows_nb_pack;       // slot offsets carry the neighbour row (min-margin dots, P * 4 >= R)
    // sort kernel
    int sort_lds_bytes;
    int sort_slots;     // sorted-slot capacity of a table (items + padding to whole batches)
    size_t ws_slot_off, ws_row_start, ws_batch_row, ws_g_chunked, ws_pdot;  // workspace byte offsets (general path)
    // item kernel
    int item_vec;       // N: LUT / grad elements per lane load (16 bytes at most)
    int item_o_tiles;   // 64 * N column tiles per row
    int item_per_wave;  // tables per wave
    int item_waves;     // waves per workgroup (one item per workgroup)
    int item_threads;
    bool wide_index;    // gu slots and index past one workgroup's LDS: the wide scatter kernel forms grad_latent
    int item_lds_bytes; // the item's gu slots [T * C] f32 + the inverse anchor index (0 with wide_index)
    bool full;          // full STE (every comparison): item kernel variant, general path only
    // fused path (O a multiple of 4 up to 64, or of 8 up to 256, a table's LUT
    // rows within 64 KB as f32): one kernel per table does the LUT gradient, the
    // STE dots and the threshold gradient; a scatter kernel per item the input
    // gradient. Otherwise the item, sort and row kernels above.
    bool fused;
    int fvec;           // V: columns per lane
    int fslices;        // S: lanes per row group, S * V >= O
    int fpitch;         // S * V: LDS row pitch in floats
    int f_lut_off, f_cnt_off, f_off_off, f_sorted_off, f_u_off, f_dt_off, f_rowbuf_off, f_thr_off, f_wtot_off;  // LDS bytes
    int f_part_off, f_brow_off;
    int f_slots;        // sorted-list capacity of a tile (items + padding to whole batches)
    int f_lds_bytes;
    // item role of the fused launch (tables <= kItemRoleMaxTables): workgroups
    // after the table ones form the input gradient, so no scatter kernel runs
    // and the fused path needs no workspace
    bool f_item;
    int f_item_nc;      // items of an item-role workgroup held in LDS at once
    int f_ir_rec_off, f_ir_g_off, f_ir_gud_off, f_ir_idx_off;  // LDS bytes
    int f_launch_lds;   // the launch's dynamic LDS: max of the two roles'
    int scatter_lds_bytes;   // gu slots [T * C] f32 + the inverse anchor index
    size_t workspace_bytes;  // fused: none with the item role, else {gu, r} [T][B] u64; general: gu, then the sort kernel's output
};

// Row loads a forward wave keeps in flight (its gather chunk), by LUT element
// size and elements per lane; sized to stay within 128 VGPRs.
constexpr int gather_chunk(int esize, int vec) { return esize == 2 && vec == 8 ? 8 : 16; }

// rows16: the LUT and the output start on 16-byte boundaries (the wave-item
// kernel moves whole 16-byte pieces of rows; without it the other kernels,
// whose loads need only the plan's vec * element alignment, serve the shape)
ForwardPlan plan_forward(const Dims &d, bool rows16 = true);
// Tables whose two LUT rows an item-kernel wave keeps in flight, by LUT
// element size and elements per lane: about 48 VGPRs of rows, so the kernel
// stays within 80 VGPRs and two workgroups share a CU.
constexpr int item_wave_tables(int esize, int vec) {
    return esize * vec <= 4 ? 16 : (esize * vec == 8 ? 12 : (esize == 4 ? 6 : 3));
}

// ste_mode: TROPNN_STE_MIN_MARGIN or TROPNN_STE_FULL (general path only),
// optionally with one TROPNN_BWD_INPUT_GRAD_* flag (fused path's item role).
BackwardPlan plan_backward(const Dims &d, int ste_mode);

hipError_t launch_forward(const Dims &d, const ForwardPlan &p, const float *x, const int64_t *anchors,
                          const float *thr, const void *lut, float scale, float *out, tropnn_route_record *rec,
                          int64_t *indices, float *margins, uint8_t *codes, hipStream_t stream);

// Route only: codes (uint8 and / or int64) and margins, no gather.
hipError_t launch_route(const Dims &d, const float *x, const int64_t *anchors, const float *thr, uint8_t *codes,
                        int64_t *indices, float *margins, hipStream_t stream);

hipError_t launch_backward(const Dims &d, const BackwardPlan &p, const float *grad_out, const void *lut,
                           const tropnn_route_record *rec, const float *margins, const int32_t *index_offsets,
                           const int32_t *index_entries, float scale, int surrogate, float *grad_x,
                           float *grad_thr, float *grad_lut, float *workspace, hipStream_t stream);

// Inverse anchor index (see tropnn_hip_build_anchor_index).
hipError_t launch_anchor_index(const int64_t *anchors, int in_f, int tables, int comps, int32_t *offsets,
                               int32_t *entries, hipStream_t stream);

// Events armed by tropnn_hip_arm_kernel_events for the next launch of a
// kernel; take_armed_events clears them.
struct ArmedEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
ArmedEvents take_armed_events(int kernel);
void arm_events(int kernel, hipEvent_t start, hipEvent_t stop);

// Launches `kernel`; when events are armed for `kernel_id`, the dispatch
// itself stamps them with the kernel's start and end (hipExtLaunchKernel), so
// they time the kernel alone, without marker packets around it.
template <typename F, typename... Args>
hipError_t launch_kernel(int kernel_id, F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t stream,
                         Args... args) {
    const ArmedEvents ev = take_armed_events(kernel_id);
    if (ev.start != nullptr)
        hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, ev.start, ev.stop, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    return hipGetLastError();
}

// Writes n zeros with a kernel (no hipMemsetAsync node in captured graphs).
hipError_t launch_fill_zero(float *p, size_t n, hipStream_t stream);

// Adam / AdamW step over n f32 tensors (host arrays of device pointers),
// kAdamGroup tensors per launch, then launches advancing each tensor's device
// step counter.
constexpr int kAdamGroup = 16;
hipError_t launch_adam(int n, float *const *params, const float *const *grads, float *const *exp_avgs,
                       float *const *exp_avg_sqs, const int64_t *numels, float *const *steps, double lr,
                       double beta1, double beta2, double eps, double weight_decay, int decoupled,
                       hipStream_t stream);

// Mean cross entropy over `rows` rows of `classes` f32 logits and its
// gradient, in one launch.
hipError_t launch_cross_entropy(const float *logits, const int64_t *target, int64_t rows, int classes,
                                int64_t ignore_index, float *loss, float *grad_logits, hipStream_t stream);

// Opts `kernel` into `bytes` of dynamic LDS when that is above the default
// 64 KB, once per kernel and size (thread-safe; keyed by the kernel's address).
hipError_t allow_dynamic_lds(const void *kernel, int bytes);

}  // namespace tropnn
