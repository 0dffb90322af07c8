// Internal host-side launch API between the C ABI (abi.hip) and the kernels
// (forward.hip, backward.hip). Not exported.
#pragma once

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

// Launch shape of the fused route + gather + scale forward.
struct ForwardPlan {
    int vec;             // LUT elements per lane load (16 bytes at most)
    int lpt_log2;        // lanes per table in a route ballot (>= C)
    int lpr_log2;        // lanes per LUT row in the gather
    int o_tile;          // output columns per workgroup
    int o_tiles;         // grid.y
    int items_per_wg;    // items per workgroup
    int waves_per_item;  // waves sharing one item's tables
    int threads;         // items_per_wg * waves_per_item * 64
    int blocks;          // grid.x
    int codes_off;       // LDS byte offsets
    int red_off;
    int lds_bytes;
};

// Launch shape of the table-major backward (LUT gradient + STE dot) and of
// the input-side backward (input / threshold gradients).
struct BackwardPlan {
    int vec;            // elements per lane load of grad_output / LUT rows
    int o_chunk;        // output columns per table workgroup
    int o_chunks;       // grid.y of the table kernel
    int pitch;          // LDS row pitch (floats) of the LUT slab
    int slices_log2;    // lanes (vec-wide column slices) per gradient row
    int lut_threads;    // threads of a table workgroup = items per sort tile
    int lut_lds_bytes;  // slab + histograms + bucket starts + sorted tile
    int in_items_per_wg;
    int in_threads;
    int in_lds_bytes;
    size_t workspace_bytes;  // partial STE dots [o_chunks][T][B] f32
};

ForwardPlan plan_forward(const Dims &d);
BackwardPlan plan_backward(const Dims &d);

hipError_t launch_forward(const Dims &d, const ForwardPlan &p, const float *x, const int64_t *anchors,
                          const float *thr, const void *lut, float scale, float *out, tropnn_route_record *rec,
                          int64_t *indices, float *margins, hipStream_t stream);

hipError_t launch_backward(const Dims &d, const BackwardPlan &p, const float *grad_out, const void *lut,
                           const tropnn_route_record *rec, const int32_t *index_offsets,
                           const int32_t *index_entries, float scale, float *grad_x, float *grad_thr,
                           float *grad_lut, float *workspace, hipStream_t stream);

// Inverse anchor index (see tropnn_hip_build_anchor_index).
hipError_t launch_anchor_index(const int64_t *anchors, int in_f, int tables, int comps, int32_t *offsets,
                               int32_t *entries, hipStream_t stream);

// Events armed by tropnn_hip_arm_kernel_events for the next launch of a
// kernel; take_armed_events clears them. record_event tolerates NULL.
struct ArmedEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
ArmedEvents take_armed_events(int kernel);
void arm_events(int kernel, hipEvent_t start, hipEvent_t stop);
inline void record_event(hipEvent_t e, hipStream_t s) {
    if (e != nullptr) (void)hipEventRecord(e, s);
}

// Writes n zeros with a kernel (no hipMemsetAsync node in captured graphs).
hipError_t launch_fill_zero(float *p, size_t n, hipStream_t stream);

}  // namespace tropnn
