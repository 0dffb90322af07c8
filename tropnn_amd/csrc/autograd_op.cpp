// torch.ops.tropnn_hip.pairwise: the autograd operator behind pairwise_hip,
// in C++ so that an eager training step pays no Python on its per-call path
// (validation, output and gradient allocation, the kernel calls, and the
// backward node, which then runs on autograd's device thread without the
// GIL). It is host code only: every launch goes through the C ABI of
// libtropnn_hip.so (include/tropnn_hip.h), whose entry-point addresses the
// Python package hands over once, after it has loaded that library and
// checked its ABI version (bind_abi below), so this operator and the ctypes
// bindings always drive one and the same library.
//
// Contract: that of _PairwiseTileLangFunction (backends/pairwise_tilelang.py:460-534)
// as wrapped by pairwise_tilelang (backends/pairwise_tilelang.py:537-549):
// outputs (output [B,S,O], indices, margins), indices and margins
// non-differentiable; gradients flow to latent, thresholds (both through the
// STE, when `ste`) and lut; anchors, lut_read and the anchor index get none.

#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/library.h>

#include <atomic>
#include <cstdint>
#include <optional>
#include <tuple>

#include "tropnn_hip.h"

namespace {

using at::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

struct Abi {
    decltype(&tropnn_hip_pairwise_forward) forward = nullptr;
    decltype(&tropnn_hip_pairwise_backward) backward = nullptr;
    decltype(&tropnn_hip_pairwise_backward_workspace_size) workspace_size = nullptr;
    decltype(&tropnn_hip_last_error) last_error = nullptr;
};
Abi g_abi;
std::atomic<bool> g_bound{false};

// The Python package passes the addresses of the entry points of the
// libtropnn_hip.so it loaded (ctypes), with that library's ABI version.
void bind_abi(int64_t forward, int64_t backward, int64_t workspace_size, int64_t last_error, int64_t abi_version) {
    TORCH_CHECK(abi_version == TROPNN_HIP_ABI_VERSION, "libtropnn_hip.so has ABI version ", abi_version,
                ", the autograd operator was built for ", TROPNN_HIP_ABI_VERSION);
    TORCH_CHECK(forward != 0 && backward != 0 && workspace_size != 0 && last_error != 0,
                "bind_abi: NULL entry point");
    g_abi.forward = reinterpret_cast<decltype(g_abi.forward)>(static_cast<intptr_t>(forward));
    g_abi.backward = reinterpret_cast<decltype(g_abi.backward)>(static_cast<intptr_t>(backward));
    g_abi.workspace_size = reinterpret_cast<decltype(g_abi.workspace_size)>(static_cast<intptr_t>(workspace_size));
    g_abi.last_error = reinterpret_cast<decltype(g_abi.last_error)>(static_cast<intptr_t>(last_error));
    g_bound.store(true, std::memory_order_release);
}

// Status codes of the C ABI to the exception types of the ctypes bindings:
// invalid argument -> ValueError, unsupported -> NotImplementedError,
// HIP error -> RuntimeError.
void check_rc(int rc, const char *what) {
    if (rc == TROPNN_OK) return;
    const char *msg = g_abi.last_error();
    TORCH_CHECK_VALUE(rc != TROPNN_ERR_INVALID_ARGUMENT, what, ": ", msg);
    TORCH_CHECK_NOT_IMPLEMENTED(rc != TROPNN_ERR_UNSUPPORTED, what, ": ", msg);
    TORCH_CHECK(false, what, ": ", rc == TROPNN_ERR_HIP ? std::string("HIP error") : "error " + std::to_string(rc),
                ": ", msg);
}

hipStream_t current_stream(const Tensor &t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

struct Dims {
    int64_t batch, steps, in_f, tables, comps, out_f;
};

// Shapes and dtypes, with the messages and exception types of the ctypes
// path's checks (pairwise_tilelang.py:423-436 raises ValueError / TypeError
// alike).
Dims validate(const Tensor &latent, const Tensor &anchors, const Tensor &thresholds, const Tensor &lut) {
    TORCH_CHECK_VALUE(latent.dim() == 3, "latent must have shape [batch, steps, in_features], got ", latent.sizes());
    TORCH_CHECK_TYPE(latent.scalar_type() == at::kFloat && thresholds.scalar_type() == at::kFloat,
                     "Pairwise HIP backend expects float32 latent and thresholds, got ", latent.scalar_type(), ", ",
                     thresholds.scalar_type());
    TORCH_CHECK_TYPE(anchors.scalar_type() == at::kLong, "anchors must be int64, got ", anchors.scalar_type());
    TORCH_CHECK_TYPE(lut.scalar_type() == at::kFloat || lut.scalar_type() == at::kHalf,
                     "lut must be float32 or float16, got ", lut.scalar_type());
    TORCH_CHECK_VALUE(anchors.dim() == 3 && anchors.size(2) == 2,
                      "anchors must have shape [tables, comparisons, 2], got ", anchors.sizes());
    Dims d{latent.size(0), latent.size(1), latent.size(2), anchors.size(0), anchors.size(1), 0};
    TORCH_CHECK_VALUE(thresholds.dim() == 2 && thresholds.size(0) == d.tables && thresholds.size(1) == d.comps,
                      "thresholds must have shape (", d.tables, ", ", d.comps, "), got ", thresholds.sizes());
    TORCH_CHECK_NOT_IMPLEMENTED(d.comps <= TROPNN_MAX_COMPARISONS, "Pairwise HIP backend supports comparisons <= ",
                                TROPNN_MAX_COMPARISONS, ", got ", d.comps);
    TORCH_CHECK_VALUE(lut.dim() == 3 && lut.size(0) == d.tables && lut.size(1) == (int64_t{1} << d.comps),
                      "lut must have shape [", d.tables, ", ", int64_t{1} << d.comps, ", out_features], got ",
                      lut.sizes());
    d.out_f = lut.size(2);
    const auto dev = latent.device();
    TORCH_CHECK_VALUE(dev.is_cuda() && anchors.device() == dev && thresholds.device() == dev && lut.device() == dev,
                      "all tensors must be on one GPU, got ", latent.device(), ", ", anchors.device(), ", ",
                      thresholds.device(), ", ", lut.device());
    return d;
}

constexpr int64_t kRouteNone = 0, kRouteFull = 1, kRouteCodes = 2;
// Where the backward forms the latent gradient of narrow rows: by the
// library's row-width rule, in the fused launch, or in a kernel after it.
constexpr int64_t kInputGradAuto = 0, kInputGradFused = 1, kInputGradScatter = 2;
int input_grad_flag(int64_t input_grad) {
    return input_grad == kInputGradFused ? TROPNN_BWD_INPUT_GRAD_FUSED
                                         : input_grad == kInputGradScatter ? TROPNN_BWD_INPUT_GRAD_SCATTER : 0;
}

// One forward launch and the tensors it writes.
struct Forward {
    Tensor out, indices, margins, record, saved_margins;
    Tensor lut_read;  // the contiguous LUT the kernels read
};

// Validation, allocation and the forward launch. want_record: the backward
// will read the route record; want_margins: the full-STE backward will read
// every comparison's margin.
Forward run_forward(const Dims &d, const Tensor &latent, const Tensor &anchors, const Tensor &thresholds,
                    const Tensor &lut_read, double output_scale, int64_t route_mode, bool want_record,
                    bool want_margins) {
    const int64_t items = d.batch * d.steps;
    const bool full_route = route_mode == kRouteFull;
    const Tensor x = latent.contiguous();  // [B,S,I] is [items, I] row-major
    const Tensor anc = anchors.contiguous(), thr = thresholds.contiguous(), lut_c = lut_read.contiguous();
    const auto f32 = latent.options();
    Forward f;
    f.lut_read = lut_c;
    f.out = at::empty({d.batch, d.steps, d.out_f}, f32);
    if (want_record) f.record = at::empty({d.tables, items}, f32.dtype(at::kLong));
    if (full_route) {
        f.indices = at::empty({d.batch, d.steps, d.tables}, f32.dtype(at::kLong));
        f.margins = at::empty({d.batch, d.steps, d.tables, d.comps}, f32);
    } else {
        f.indices = at::empty({d.batch, d.steps, route_mode == kRouteCodes ? d.tables : 0},
                              f32.dtype(route_mode == kRouteCodes ? at::kByte : at::kLong));
        f.margins = at::empty({d.batch, d.steps, 0}, f32);
    }
    // the margins the full-STE backward reads
    if (want_margins) f.saved_margins = full_route ? f.margins : at::empty({items, d.tables, d.comps}, f32);

    TORCH_CHECK(g_bound.load(std::memory_order_acquire), "tropnn_hip.pairwise: the C ABI is not bound");
    const int lut_dtype = lut_c.scalar_type() == at::kHalf ? TROPNN_LUT_F16 : TROPNN_LUT_F32;
    const int rc = g_abi.forward(
        items, d.in_f, d.out_f, d.tables, d.comps, x.const_data_ptr<float>(), anc.const_data_ptr<int64_t>(),
        thr.const_data_ptr<float>(), lut_c.const_data_ptr(), lut_dtype, static_cast<float>(output_scale),
        f.out.mutable_data_ptr<float>(),
        want_record ? reinterpret_cast<tropnn_route_record *>(f.record.mutable_data_ptr()) : nullptr,
        full_route ? f.indices.mutable_data_ptr<int64_t>() : nullptr,
        full_route ? f.margins.mutable_data_ptr<float>()
                   : (want_margins ? f.saved_margins.mutable_data_ptr<float>() : nullptr),
        route_mode == kRouteCodes ? f.indices.mutable_data_ptr<uint8_t>() : nullptr, current_stream(x));
    check_rc(rc, "tropnn_hip_pairwise_forward");
    return f;
}

struct PairwiseFunction : public torch::autograd::Function<PairwiseFunction> {
    // Argument order fixes the input-edge numbering of needs_input_grad:
    // tensors latent 0, anchors 1, thresholds 2, lut 3, lut_read 4 (the
    // anchor index follows, as optionals: an absent one is no input at all).
    static variable_list forward(AutogradContext *ctx, const Tensor &latent, const Tensor &anchors,
                                 const Tensor &thresholds, const Tensor &lut, const Tensor &lut_read,
                                 const std::optional<Tensor> &index_offsets,
                                 const std::optional<Tensor> &index_entries, bool ste, bool min_margin,
                                 int64_t surrogate, double output_scale, int64_t route_mode, int64_t input_grad,
                                 bool recorded) {
        const Dims d = validate(latent, anchors, thresholds, lut_read);
        // What the backward may be asked for: every input that requires a
        // gradient, when autograd records this call. (needs_input_grad is
        // narrower inside a backward pass, e.g. a checkpoint recompute under
        // autograd.grad(inputs=...), and the record must cover any later
        // backward of this node.)
        const bool g_x = recorded && latent.requires_grad();
        const bool g_thr = recorded && thresholds.requires_grad();
        const bool g_lut = recorded && lut.requires_grad();
        const bool needs_route = ste && (g_x || g_thr);
        const bool want_record = g_lut || needs_route;
        const bool want_margins = needs_route && !min_margin;
        if (ste && g_x)
            TORCH_CHECK(index_offsets.has_value() && index_entries.has_value(),
                        "the latent gradient needs the inverse anchor index");
        Forward f = run_forward(d, latent, anchors, thresholds, lut_read, output_scale, route_mode, want_record,
                                want_margins);
        Tensor &out = f.out, &indices = f.indices, &margins = f.margins, &record = f.record,
               &saved_margins = f.saved_margins, &lut_c = f.lut_read;

        ctx->set_materialize_grads(false);
        ctx->mark_non_differentiable({indices, margins});
        if (recorded) {
            ctx->save_for_backward({record, lut_c, saved_margins});
            if (ste && g_x) {
                ctx->saved_data["index_offsets"] = *index_offsets;
                ctx->saved_data["index_entries"] = *index_entries;
            }
            ctx->saved_data["dims"] = std::vector<int64_t>{d.batch, d.steps, d.in_f, d.tables, d.comps, d.out_f};
            ctx->saved_data["ste"] = ste;
            ctx->saved_data["ste_mode"] =
                static_cast<int64_t>((min_margin ? TROPNN_STE_MIN_MARGIN : TROPNN_STE_FULL) | input_grad_flag(input_grad));
            ctx->saved_data["surrogate"] = surrogate;
            ctx->saved_data["output_scale"] = output_scale;
        }
        return {out, indices, margins};
    }

    // Computes only the gradients this backward pass asks for (a subset of
    // those the forward recorded for).
    static variable_list backward(AutogradContext *ctx, variable_list grad_outputs) {
        variable_list grads(14);  // one per forward argument
        const Tensor &grad_output = grad_outputs[0];
        if (!grad_output.defined()) return grads;
        const bool ste = ctx->saved_data["ste"].toBool();
        const bool want_x = ste && ctx->needs_input_grad(0);
        const bool want_thr = ste && ctx->needs_input_grad(2);
        const bool want_lut = ctx->needs_input_grad(3);
        if (!(want_x || want_thr || want_lut)) return grads;
        const auto saved = ctx->get_saved_variables();
        const Tensor &record = saved[0], &lut_read = saved[1], &margins = saved[2];
        const auto dims = ctx->saved_data["dims"].toIntVector();
        const int64_t batch = dims[0], steps = dims[1], in_f = dims[2], tables = dims[3], comps = dims[4],
                      out_f = dims[5];
        const int64_t items = batch * steps;
        const int ste_mode = static_cast<int>(ctx->saved_data["ste_mode"].toInt());
        const Tensor g = grad_output.reshape({items, out_f}).to(at::kFloat).contiguous();
        const auto f32 = g.options();
        Tensor grad_x = want_x ? at::empty({batch, steps, in_f}, f32) : Tensor();
        Tensor grad_thr = want_thr ? at::empty({tables, comps}, f32) : Tensor();
        Tensor grad_lut = want_lut ? at::empty({tables, int64_t{1} << comps, out_f}, f32) : Tensor();
        const int lut_dtype = lut_read.scalar_type() == at::kHalf ? TROPNN_LUT_F16 : TROPNN_LUT_F32;
        const size_t ws_bytes = g_abi.workspace_size(items, in_f, out_f, tables, comps, lut_dtype, ste_mode);
        Tensor workspace = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, f32.dtype(at::kByte));
        Tensor offsets, entries;
        if (want_x) {
            offsets = ctx->saved_data["index_offsets"].toTensor();
            entries = ctx->saved_data["index_entries"].toTensor();
        }
        const int rc = g_abi.backward(
            items, in_f, out_f, tables, comps, g.const_data_ptr<float>(), lut_read.const_data_ptr(), lut_dtype,
            reinterpret_cast<const tropnn_route_record *>(record.const_data_ptr()),
            margins.defined() ? margins.const_data_ptr<float>() : nullptr,
            want_x ? offsets.const_data_ptr<int32_t>() : nullptr, want_x ? entries.const_data_ptr<int32_t>() : nullptr,
            static_cast<float>(ctx->saved_data["output_scale"].toDouble()), ste_mode,
            static_cast<int>(ctx->saved_data["surrogate"].toInt()), want_x ? grad_x.mutable_data_ptr<float>() : nullptr,
            want_thr ? grad_thr.mutable_data_ptr<float>() : nullptr,
            want_lut ? grad_lut.mutable_data_ptr<float>() : nullptr, workspace.mutable_data_ptr(), ws_bytes,
            current_stream(g));
        check_rc(rc, "tropnn_hip_pairwise_backward");
        grads[0] = grad_x;
        grads[2] = grad_thr;
        grads[3] = grad_lut;
        return grads;
    }
};

std::tuple<Tensor, Tensor, Tensor> pairwise(const Tensor &latent, const Tensor &anchors, const Tensor &thresholds,
                                            const Tensor &lut, const Tensor &lut_read,
                                            const std::optional<Tensor> &index_offsets,
                                            const std::optional<Tensor> &index_entries, bool ste, bool min_margin,
                                            int64_t surrogate, double output_scale, int64_t route_mode,
                                            int64_t input_grad) {
    TORCH_CHECK_VALUE(surrogate == TROPNN_SURROGATE_FAST_SIGMOID_ODD || surrogate == TROPNN_SURROGATE_IZHIKEVICH,
                      "unknown surrogate id ", surrogate);
    TORCH_CHECK_VALUE(route_mode == kRouteNone || route_mode == kRouteFull || route_mode == kRouteCodes,
                      "unknown route mode ", route_mode);
    TORCH_CHECK_VALUE(input_grad == kInputGradAuto || input_grad == kInputGradFused || input_grad == kInputGradScatter,
                      "unknown input-gradient form ", input_grad);
    const bool recorded =
        at::GradMode::is_enabled() && (latent.requires_grad() || thresholds.requires_grad() || lut.requires_grad());
    if (!recorded) {
        // no backward node: the launch alone (inference, torch.no_grad)
        const Dims d = validate(latent, anchors, thresholds, lut_read);
        Forward f = run_forward(d, latent, anchors, thresholds, lut_read, output_scale, route_mode, false, false);
        return {f.out, f.indices, f.margins};
    }
    auto outs = PairwiseFunction::apply(latent, anchors, thresholds, lut, lut_read.detach(), index_offsets,
                                        index_entries, ste, min_margin, surrogate, output_scale, route_mode,
                                        input_grad, recorded);
    return {outs[0], outs[1], outs[2]};
}

}  // namespace

TORCH_LIBRARY(tropnn_hip, m) {
    m.def("bind_abi(int forward, int backward, int workspace_size, int last_error, int abi_version) -> ()",
          &bind_abi);
    m.def("pairwise(Tensor latent, Tensor anchors, Tensor thresholds, Tensor lut, Tensor lut_read, "
          "Tensor? index_offsets, Tensor? index_entries, bool ste, bool min_margin, int surrogate, "
          "float output_scale, int route_mode, int input_grad=0) -> (Tensor, Tensor, Tensor)",
          &pairwise);
}
