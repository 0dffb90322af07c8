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
    int lpr_log2;       // lanes per item row in the table kernel
    int lut_threads;    // threads of a table workgroup
    int lut_lds_bytes;  // slab + gradient slab
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

hipError_t launch_backward(const Dims &d, const BackwardPlan &p, const float *grad_out, const int64_t *anchors,
                           const void *lut, const tropnn_route_record *rec, float scale, float *grad_x,
                           float *grad_thr, float *grad_lut, float *workspace, hipStream_t stream);

// Writes n zeros with a kernel (no hipMemsetAsync node in captured graphs).
hipError_t launch_fill_zero(float *p, size_t n, hipStream_t stream);

}  // namespace tropnn
