// C ABI of libtropnn_hip.so (declared in include/tropnn_hip.h): argument
// validation, the per-thread error channel, launch planning and dispatch.
// Nothing here allocates memory or synchronises the device.
//
// The allocation-free backward (tropnn_hip_pairwise_backward_noalloc) takes
// its workspace from `scratch` below, a file-scope device array: every GPU
// that loads the library holds its own copy, at its own address, until the
// process ends. In host code the name `scratch` is only a handle for the HIP
// runtime; the copy's device address comes from hipGetSymbolAddress, once per
// device, with that device current, and only that address reaches a kernel.
#include <stdarg.h>
#include <stdio.h>

#include <limits>
#include <mutex>
#include <string>

#include "launch.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return TROPNN_OK;
}

int hip_fail(const char *where, hipError_t e) {
    return fail(TROPNN_ERR_HIP, "%s: %s (%s)", where, hipGetErrorName(e), hipGetErrorString(e));
}

bool fits_int(int64_t v) { return v >= 0 && v <= std::numeric_limits<int>::max(); }

// Shape checks shared by every entry point. Returns TROPNN_OK or an error code
// (message set) and fills `d`.
int make_dims(int64_t items, int64_t in_f, int64_t out_f, int64_t tables, int64_t comps, int lut_dtype,
              tropnn::Dims &d) {
    if (items < 0) return fail(TROPNN_ERR_INVALID_ARGUMENT, "items must be >= 0, got %lld", (long long)items);
    if (in_f < 1) return fail(TROPNN_ERR_INVALID_ARGUMENT, "in_features must be >= 1, got %lld", (long long)in_f);
    if (out_f < 1) return fail(TROPNN_ERR_INVALID_ARGUMENT, "out_features must be >= 1, got %lld", (long long)out_f);
    if (tables < 1) return fail(TROPNN_ERR_INVALID_ARGUMENT, "tables must be >= 1, got %lld", (long long)tables);
    if (comps < 1) return fail(TROPNN_ERR_INVALID_ARGUMENT, "comparisons must be >= 1, got %lld", (long long)comps);
    if (comps > TROPNN_MAX_COMPARISONS)
        return fail(TROPNN_ERR_UNSUPPORTED, "comparisons=%lld exceeds the supported maximum %d", (long long)comps,
                    TROPNN_MAX_COMPARISONS);
    if (lut_dtype != TROPNN_LUT_F32 && lut_dtype != TROPNN_LUT_F16)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "lut_dtype must be TROPNN_LUT_F32 or TROPNN_LUT_F16, got %d",
                    lut_dtype);
    if (!fits_int(items) || !fits_int(in_f) || !fits_int(out_f) || !fits_int(tables))
        return fail(TROPNN_ERR_UNSUPPORTED, "a dimension exceeds INT_MAX");
    const int64_t rows = int64_t{1} << comps;
    if (items * tables > std::numeric_limits<int>::max() || tables * rows > std::numeric_limits<int>::max())
        return fail(TROPNN_ERR_UNSUPPORTED, "items*tables or tables*2^comparisons exceeds INT_MAX");
    d.items = static_cast<int>(items);
    d.in_f = static_cast<int>(in_f);
    d.out_f = static_cast<int>(out_f);
    d.tables = static_cast<int>(tables);
    d.comps = static_cast<int>(comps);
    d.rows = static_cast<int>(rows);
    d.lut_dtype = lut_dtype;
    return TROPNN_OK;
}

bool misaligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) != 0; }

int check_forward_ptrs(const tropnn::Dims &d, const tropnn::ForwardPlan &p, const float *x, const int64_t *anchors,
                       const float *thr, const void *lut, const float *out) {
    if (d.items == 0) return TROPNN_OK;
    if (!x || !anchors || !thr || !lut || !out)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "latent, anchors, thresholds, lut and output must be non-NULL");
    const size_t esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    if (misaligned(lut, p.vec * esize) || misaligned(out, p.vec * 4) || misaligned(x, 4) || misaligned(thr, 4) ||
        misaligned(anchors, 8))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "a device pointer is not aligned to its element/vector size");
    return TROPNN_OK;
}

std::mutex g_events_mu;
tropnn::ArmedEvents g_armed[TROPNN_KERNEL_FORWARD_ROUTE + 1];

}  // namespace

// Workspace of the allocation-free backward, one copy per GPU. Never zeroed:
// every byte of it that a backward reads, the same backward wrote first.
static __device__ __align__(256) unsigned char scratch[TROPNN_NOALLOC_WORKSPACE_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of each GPU's copy of `scratch`

// The device address of `scratch` on the GPU that `stream` runs on, looked up
// on the first call for that GPU (with the GPU made current for the lookup)
// and kept. No allocation: the array is part of the loaded code object.
int scratch_for_stream(hipStream_t stream, void **out) {
    int dev = 0;
    hipError_t e = stream != nullptr ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail("device of the stream", e);
    if (dev < 0 || dev >= kMaxDevices)
        return fail(TROPNN_ERR_UNSUPPORTED, "device %d: the allocation-free entry point serves devices 0-%d", dev,
                    kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        // the lookup is a runtime call of its own, not stream work: it is
        // made outside any capture, so a first call under capture is refused
        if (stream != nullptr) {
            hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
            if ((e = hipStreamIsCapturing(stream, &st)) != hipSuccess) return hip_fail("hipStreamIsCapturing", e);
            if (st != hipStreamCaptureStatusNone)
                return fail(TROPNN_ERR_UNSUPPORTED,
                            "the first allocation-free backward on device %d is under stream capture; make one call "
                            "on that device outside capture first (it looks up the device buffer's address)",
                            dev);
        }
        int cur = 0;
        if ((e = hipGetDevice(&cur)) != hipSuccess) return hip_fail("hipGetDevice", e);
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return hip_fail("hipSetDevice", e);
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur != dev) {
            const hipError_t back = hipSetDevice(cur);
            if (e == hipSuccess) e = back;
        }
        if (e != hipSuccess) return hip_fail("hipGetSymbolAddress(scratch)", e);
        if (ptr == nullptr) return fail(TROPNN_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return TROPNN_OK;
}

}  // namespace

namespace tropnn {

ArmedEvents take_armed_events(int kernel) {
    std::lock_guard<std::mutex> lock(g_events_mu);
    ArmedEvents e = g_armed[kernel];
    g_armed[kernel] = ArmedEvents{};
    return e;
}

void arm_events(int kernel, hipEvent_t start, hipEvent_t stop) {
    std::lock_guard<std::mutex> lock(g_events_mu);
    g_armed[kernel].start = start;
    g_armed[kernel].stop = stop;
}

}  // namespace tropnn

extern "C" {

int tropnn_hip_arm_kernel_events(int kernel, void *start_event, void *stop_event) {
    if (kernel < TROPNN_KERNEL_FORWARD || kernel > TROPNN_KERNEL_FORWARD_ROUTE)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "unknown kernel id %d", kernel);
    if ((start_event == nullptr) != (stop_event == nullptr))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "arm both events or neither");
    tropnn::arm_events(kernel, static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
    return ok();
}


int tropnn_hip_adam_step(int n_tensors, float *const *params, const float *const *grads, float *const *exp_avgs,
                         float *const *exp_avg_sqs, const int64_t *numels, float *const *steps, double lr,
                         double beta1, double beta2, double eps, double weight_decay, int decoupled_weight_decay,
                         tropnn_stream_t stream) {
    if (n_tensors < 0) return fail(TROPNN_ERR_INVALID_ARGUMENT, "n_tensors must be >= 0, got %d", n_tensors);
    if (n_tensors > 0 && (!params || !grads || !exp_avgs || !exp_avg_sqs || !numels || !steps))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "params, grads, exp_avgs, exp_avg_sqs, numels and steps must be non-NULL");
    if (!(lr >= 0.0) || !(beta1 >= 0.0 && beta1 < 1.0) || !(beta2 >= 0.0 && beta2 < 1.0) || !(eps >= 0.0) ||
        !(weight_decay >= 0.0))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "need lr >= 0, 0 <= beta1, beta2 < 1, eps >= 0, weight_decay >= 0");
    for (int k = 0; k < n_tensors; ++k) {
        if (!steps[k] || misaligned(steps[k], 4))
            return fail(TROPNN_ERR_INVALID_ARGUMENT, "steps[%d] must be a 4-byte aligned device float", k);
        if (numels[k] < 0) return fail(TROPNN_ERR_INVALID_ARGUMENT, "numels[%d] < 0", k);
        if (numels[k] == 0) continue;
        if (!params[k] || !grads[k] || !exp_avgs[k] || !exp_avg_sqs[k])
            return fail(TROPNN_ERR_INVALID_ARGUMENT, "tensor %d has a NULL pointer", k);
        if (misaligned(params[k], 4) || misaligned(grads[k], 4) || misaligned(exp_avgs[k], 4) ||
            misaligned(exp_avg_sqs[k], 4))
            return fail(TROPNN_ERR_INVALID_ARGUMENT, "tensor %d is not 4-byte aligned", k);
    }
    hipError_t e = tropnn::launch_adam(n_tensors, params, grads, exp_avgs, exp_avg_sqs, numels, steps, lr, beta1,
                                       beta2, eps, weight_decay, decoupled_weight_decay, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("adam launch", e);
    return ok();
}

int tropnn_hip_cross_entropy(int64_t rows, int64_t classes, const float *logits, const int64_t *target,
                             int64_t ignore_index, float *loss, float *grad_logits, tropnn_stream_t stream) {
    if (rows < 1) return fail(TROPNN_ERR_INVALID_ARGUMENT, "rows must be >= 1, got %lld", (long long)rows);
    if (classes < 1 || classes > (1 << 20))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "classes must be in [1, 2^20], got %lld", (long long)classes);
    if (!logits || !target || !loss || !grad_logits)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "logits, target, loss and grad_logits must be non-NULL");
    if (misaligned(logits, 4) || misaligned(target, 8) || misaligned(loss, 4) || misaligned(grad_logits, 4))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "logits, loss and grad_logits need 4-byte, target 8-byte alignment");
    hipError_t e = tropnn::launch_cross_entropy(logits, target, rows, static_cast<int>(classes), ignore_index, loss,
                                                grad_logits, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("cross entropy launch", e);
    return ok();
}

int tropnn_hip_abi_version(void) { return TROPNN_HIP_ABI_VERSION; }

const char *tropnn_hip_last_error(void) { return g_last_error.c_str(); }

int tropnn_hip_pairwise_forward(int64_t items, int64_t in_features, int64_t out_features, int64_t tables,
                                int64_t comparisons, const float *latent, const int64_t *anchors,
                                const float *thresholds, const void *lut, int lut_dtype, float output_scale,
                                float *output, tropnn_route_record *route_record, int64_t *indices, float *margins,
                                uint8_t *codes, tropnn_stream_t stream) {
    tropnn::Dims d{};
    if (int rc = make_dims(items, in_features, out_features, tables, comparisons, lut_dtype, d)) return rc;
    // a LUT or output off a 16-byte boundary (a view with a storage offset)
    // takes a kernel whose loads need only the element-vector alignment
    const tropnn::ForwardPlan p = tropnn::plan_forward(d, !misaligned(lut, 16) && !misaligned(output, 16));
    if (int rc = check_forward_ptrs(d, p, latent, anchors, thresholds, lut, output)) return rc;
    if (d.items == 0) return ok();
    if ((route_record && misaligned(route_record, 8)) || (indices && misaligned(indices, 8)) ||
        (margins && misaligned(margins, 4)))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "route_record, indices and margins must be aligned to their element size");
    if (p.lds_bytes > tropnn::kMaxLdsBytes)
        return fail(TROPNN_ERR_UNSUPPORTED, "forward needs more than %d bytes of LDS per workgroup (tables too many)",
                    tropnn::kMaxLdsBytes);
    // the gather addresses the LUT through one buffer resource with 32-bit offsets
    const int64_t lut_bytes = int64_t{d.tables} * d.rows * d.out_f * (d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4);
    if (lut_bytes > (int64_t{1} << 31))
        return fail(TROPNN_ERR_UNSUPPORTED, "LUT of %lld bytes exceeds the forward's 2 GiB limit",
                    (long long)lut_bytes);
    hipError_t e = tropnn::launch_forward(d, p, latent, anchors, thresholds, lut, output_scale, output, route_record,
                                          indices, margins, codes, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("pairwise forward launch", e);
    return ok();
}

int tropnn_hip_lut_forward_batch_f32(size_t batch, size_t tables, size_t comparisons, size_t input_dim,
                                     size_t output_dim, const float *weights, const int64_t *anchors,
                                     const float *offsets, const float *inputs, float *outputs, float output_scale,
                                     tropnn_stream_t stream) {
    return tropnn_hip_pairwise_forward((int64_t)batch, (int64_t)input_dim, (int64_t)output_dim, (int64_t)tables,
                                       (int64_t)comparisons, inputs, anchors, offsets, weights, TROPNN_LUT_F32,
                                       output_scale, outputs, nullptr, nullptr, nullptr, nullptr, stream);
}

int tropnn_hip_lut_forward_batch_f16(size_t batch, size_t tables, size_t comparisons, size_t input_dim,
                                     size_t output_dim, const uint16_t *weights_f16, const int64_t *anchors,
                                     const float *offsets, const float *inputs, float *outputs, float output_scale,
                                     tropnn_stream_t stream) {
    return tropnn_hip_pairwise_forward((int64_t)batch, (int64_t)input_dim, (int64_t)output_dim, (int64_t)tables,
                                       (int64_t)comparisons, inputs, anchors, offsets, weights_f16, TROPNN_LUT_F16,
                                       output_scale, outputs, nullptr, nullptr, nullptr, nullptr, stream);
}

int tropnn_hip_pairwise_route(int64_t items, int64_t in_features, int64_t tables, int64_t comparisons,
                              const float *latent, const int64_t *anchors, const float *thresholds, uint8_t *codes,
                              int64_t *indices, float *margins, tropnn_stream_t stream) {
    tropnn::Dims d{};
    if (int rc = make_dims(items, in_features, 1, tables, comparisons, TROPNN_LUT_F32, d)) return rc;
    if (d.items == 0 || (!codes && !indices && !margins)) return ok();
    if (!latent || !anchors || !thresholds)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "latent, anchors and thresholds must be non-NULL");
    if (misaligned(latent, 4) || misaligned(thresholds, 4) || misaligned(anchors, 8) || (indices && misaligned(indices, 8)) ||
        (margins && misaligned(margins, 4)))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "a device pointer is not aligned to its element size");
    hipError_t e = tropnn::launch_route(d, latent, anchors, thresholds, codes, indices, margins,
                                        static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("pairwise route launch", e);
    return ok();
}

// ste_mode: TROPNN_STE_MIN_MARGIN or TROPNN_STE_FULL in the low byte, at
// most one TROPNN_BWD_INPUT_GRAD_* flag above it.
static constexpr int kSteModeMask = 0xff;
static int check_ste_mode(int ste_mode) {
    const int mode = ste_mode & kSteModeMask, flags = ste_mode & ~kSteModeMask;
    if (mode != TROPNN_STE_MIN_MARGIN && mode != TROPNN_STE_FULL)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "ste_mode must be TROPNN_STE_MIN_MARGIN or TROPNN_STE_FULL, "
                    "optionally with one TROPNN_BWD_INPUT_GRAD_* flag, got %d", ste_mode);
    if (flags != 0 && flags != TROPNN_BWD_INPUT_GRAD_FUSED && flags != TROPNN_BWD_INPUT_GRAD_SCATTER)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "ste_mode carries unknown or conflicting flags: %d", ste_mode);
    return TROPNN_OK;
}

size_t tropnn_hip_pairwise_backward_workspace_size(int64_t items, int64_t in_features, int64_t out_features,
                                                   int64_t tables, int64_t comparisons, int lut_dtype, int ste_mode) {
    tropnn::Dims d{};
    if (make_dims(items, in_features, out_features, tables, comparisons, lut_dtype, d) != TROPNN_OK) return 0;
    if (check_ste_mode(ste_mode) != TROPNN_OK) return 0;
    ok();
    return tropnn::plan_backward(d, ste_mode).workspace_bytes;
}

int tropnn_hip_build_anchor_index(int64_t in_features, int64_t tables, int64_t comparisons, const int64_t *anchors,
                                  int32_t *offsets, int32_t *entries, tropnn_stream_t stream) {
    tropnn::Dims d{};
    if (int rc = make_dims(0, in_features, 1, tables, comparisons, TROPNN_LUT_F32, d)) return rc;
    if (tables * comparisons * 2 >= (int64_t{1} << 27))
        return fail(TROPNN_ERR_UNSUPPORTED, "tables*comparisons too large for the anchor index");
    if (!anchors || !offsets || !entries)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "anchors, offsets and entries must be non-NULL");
    if (misaligned(anchors, 8) || misaligned(offsets, 4) || misaligned(entries, 4))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "a device pointer is not aligned to its element size");
    hipError_t e = tropnn::launch_anchor_index(anchors, d.in_f, d.tables, d.comps, offsets, entries,
                                               static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("anchor index launch", e);
    return ok();
}

int tropnn_hip_pairwise_backward(int64_t items, int64_t in_features, int64_t out_features, int64_t tables,
                                 int64_t comparisons, const float *grad_output, const void *lut, int lut_dtype,
                                 const tropnn_route_record *route_record, const float *margins,
                                 const int32_t *index_offsets, const int32_t *index_entries, float output_scale,
                                 int ste_mode, int surrogate, float *grad_latent, float *grad_thresholds,
                                 float *grad_lut, void *workspace, size_t workspace_bytes, tropnn_stream_t stream) {
    tropnn::Dims d{};
    if (int rc = make_dims(items, in_features, out_features, tables, comparisons, lut_dtype, d)) return rc;
    if (int rc = check_ste_mode(ste_mode)) return rc;
    if (surrogate != TROPNN_SURROGATE_FAST_SIGMOID_ODD && surrogate != TROPNN_SURROGATE_IZHIKEVICH)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "surrogate must be a TROPNN_SURROGATE_* value");
    const tropnn::BackwardPlan p = tropnn::plan_backward(d, ste_mode);
    if (d.items == 0) {
        // no items: the parameter gradients are zero (a fill kernel, not a
        // memset, so the call stays capturable in a HIP graph)
        hipError_t e = hipSuccess;
        if (grad_thresholds)
            e = tropnn::launch_fill_zero(grad_thresholds, static_cast<size_t>(d.tables) * d.comps,
                                         static_cast<hipStream_t>(stream));
        if (e == hipSuccess && grad_lut)
            e = tropnn::launch_fill_zero(grad_lut, static_cast<size_t>(d.tables) * d.rows * d.out_f,
                                         static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail("zero fill launch", e);
        return ok();
    }
    if (!grad_output || !lut || !route_record)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "grad_output, lut and route_record must be non-NULL");
    if (grad_latent && (!index_offsets || !index_entries))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "grad_latent needs the anchor index (tropnn_hip_build_anchor_index)");
    if ((ste_mode & kSteModeMask) == TROPNN_STE_FULL && (grad_latent || grad_thresholds) && !margins)
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "the full STE needs the forward's margins [items, tables, comparisons]");
    if (margins && misaligned(margins, 4))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "margins must be 4-byte aligned");
    const size_t esize = d.lut_dtype == TROPNN_LUT_F16 ? 2 : 4;
    // fused path: LUT chunks, grad-row and LUT-grad-row pieces of min(V, 4)
    // elements; general path: the item kernel's and the row kernel's pieces
    const size_t fchunk = p.fvec < 4 ? static_cast<size_t>(p.fvec) : 4;
    const size_t lut_align = p.fused ? fchunk * esize : static_cast<size_t>(p.rows_vec > p.item_vec ? p.rows_vec : p.item_vec) * esize;
    const size_t gvec = p.fused ? fchunk : static_cast<size_t>(p.rows_vec > p.item_vec ? p.rows_vec : p.item_vec);
    const size_t lut_grad_vec = p.fused ? fchunk : static_cast<size_t>(p.rows_vec);
    if (misaligned(lut, lut_align) || misaligned(grad_output, gvec * 4) ||
        (grad_lut && misaligned(grad_lut, lut_grad_vec * 4)) || misaligned(route_record, 8))
        return fail(TROPNN_ERR_INVALID_ARGUMENT, "a device pointer is not aligned to its element/vector size");
    if (grad_latent || grad_thresholds || grad_lut) {
        if (p.workspace_bytes > 0 && (!workspace || workspace_bytes < p.workspace_bytes))
            return fail(TROPNN_ERR_INVALID_ARGUMENT, "workspace of %zu bytes required, got %zu", p.workspace_bytes,
                        workspace_bytes);
        if (p.workspace_bytes > 0 && misaligned(workspace, 16))
            return fail(TROPNN_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    }
    // grad rows and the LUT are addressed through buffer resources with 32-bit offsets
    const int64_t lut_bytes = int64_t{d.tables} * d.rows * d.out_f * esize;
    const int64_t g_bytes = int64_t{d.items} * d.out_f * 4;
    if (lut_bytes > (int64_t{1} << 31) || g_bytes > (int64_t{1} << 31))
        return fail(TROPNN_ERR_UNSUPPORTED, "LUT (%lld bytes) or grad_output (%lld bytes) exceeds the 2 GiB limit",
                    (long long)lut_bytes, (long long)g_bytes);
    // the general path's chunk-major copy of grad_output (rows rounded up to
    // whole column chunks) is addressed the same way
    const int64_t gc_bytes = int64_t{p.rows_chunks} * p.rows_chunk * d.items * 4;
    if (!p.fused && grad_lut && gc_bytes > (int64_t{1} << 31))
        return fail(TROPNN_ERR_UNSUPPORTED, "grad_output in column chunks (%lld bytes) exceeds the 2 GiB limit",
                    (long long)gc_bytes);
    hipError_t e = tropnn::launch_backward(d, p, grad_output, lut, route_record, margins, index_offsets,
                                           index_entries, output_scale, surrogate, grad_latent, grad_thresholds,
                                           grad_lut, static_cast<float *>(workspace), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("pairwise backward launch", e);
    return ok();
}

int tropnn_hip_pairwise_backward_noalloc(int64_t items, int64_t in_features, int64_t out_features, int64_t tables,
                                         int64_t comparisons, const float *grad_output, const void *lut,
                                         int lut_dtype, const tropnn_route_record *route_record, const float *margins,
                                         const int32_t *index_offsets, const int32_t *index_entries,
                                         float output_scale, int ste_mode, int surrogate, float *grad_latent,
                                         float *grad_thresholds, float *grad_lut, tropnn_stream_t stream) {
    tropnn::Dims d{};
    if (int rc = make_dims(items, in_features, out_features, tables, comparisons, lut_dtype, d)) return rc;
    if (int rc = check_ste_mode(ste_mode)) return rc;
    const size_t need = tropnn::plan_backward(d, ste_mode).workspace_bytes;
    if (need > sizeof scratch)
        return fail(TROPNN_ERR_UNSUPPORTED,
                    "this backward needs %zu bytes of workspace, over the %zu bytes of the allocation-free entry "
                    "point's device buffer; call tropnn_hip_pairwise_backward with a workspace of that size",
                    need, sizeof scratch);
    void *ws = nullptr;
    if (d.items > 0 && (grad_latent || grad_thresholds || grad_lut)) {
        if (int rc = scratch_for_stream(static_cast<hipStream_t>(stream), &ws)) return rc;
    }
    return tropnn_hip_pairwise_backward(items, in_features, out_features, tables, comparisons, grad_output, lut,
                                        lut_dtype, route_record, margins, index_offsets, index_entries, output_scale,
                                        ste_mode, surrogate, grad_latent, grad_thresholds, grad_lut, ws,
                                        ws != nullptr ? sizeof scratch : 0, stream);
}

}  // extern "C"
