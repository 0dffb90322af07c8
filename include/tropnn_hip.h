/*
 * tropnn_hip.h -- C ABI of libtropnn_hip.so, the MI355X (gfx950) PairwiseLinear
 * hot path: comparator route, LUT row gather-sum, min-margin STE backward.
 *
 * Conventions (the precedent is the reference's Zig C ABI, kernels/src/lut.zig:248-318,
 * bound with ctypes at backends/pairwise_zig.py:19-32):
 *   - the caller owns every buffer; all tensor pointers are DEVICE pointers to
 *     contiguous row-major arrays; the library never allocates;
 *   - dims are passed by value; anchors are int64 [tables, comparisons, 2]
 *     (the torch buffer's dtype, layers/pairwise.py:57);
 *   - every call is asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream) and never synchronises the device;
 *   - every entry point returns TROPNN_OK (0) or an error code, and
 *     tropnn_hip_last_error() returns the calling thread's last message
 *     (the reference's Zig ABI has no error channel; its Python wrappers
 *     validate first, and so does this library, before any launch);
 *   - stateless and re-entrant: calls on different streams may overlap as
 *     long as they write disjoint buffers (the one exception is
 *     tropnn_hip_pairwise_backward_noalloc, whose calls on one GPU share a
 *     library-held buffer).
 */
#ifndef TROPNN_HIP_H
#define TROPNN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TROPNN_HIP_ABI_VERSION 11

/* status codes */
#define TROPNN_OK 0
#define TROPNN_ERR_INVALID_ARGUMENT 1 /* bad shape, pointer, enum or size */
#define TROPNN_ERR_UNSUPPORTED 2      /* valid for the reference, not implemented here */
#define TROPNN_ERR_HIP 3              /* a HIP runtime call failed */

/* element type of the LUT the kernels read */
#define TROPNN_LUT_F32 0
#define TROPNN_LUT_F16 1 /* IEEE binary16, rows converted to f32, f32 accumulation */

/* surrogate gradient of the Heaviside step (layers/surrogate.py:9-25) */
#define TROPNN_SURROGATE_FAST_SIGMOID_ODD 0
#define TROPNN_SURROGATE_IZHIKEVICH 1

/* which comparisons carry the STE gradient (layers/pairwise.py:137-200) */
#define TROPNN_STE_MIN_MARGIN 0
#define TROPNN_STE_FULL 1
/* Flags ORed into ste_mode (of the backward and of its workspace size, alike)
 * that choose where the min-margin backward of narrow rows (out_features a
 * multiple of 4 up to 64 or of 8 up to 256) forms grad_latent. Neither: by the
 * row width, the crossover measured on independent inputs. The choice changes
 * no result bit (both forms sum in the same order), only the time and the
 * workspace size (none with FUSED). No counterpart in the reference. */
#define TROPNN_BWD_INPUT_GRAD_FUSED 0x100   /* in the backward's first launch, whenever the shape allows
                                               (pays where the items' codes concentrate on few LUT rows,
                                               e.g. a layer fed by another PairwiseLinear) */
#define TROPNN_BWD_INPUT_GRAD_SCATTER 0x200 /* in a per-item kernel after it */

/* Largest `comparisons` the kernels take (LUT rows per table = 2^comparisons). */
#define TROPNN_MAX_COMPARISONS 8

/* Route record: one 8-byte entry per (table, item), laid out [tables][items].
 * Written by the training forward, read by the backward.
 *   bytes 0-3  float    u     the margin with the smallest |margin| (first on ties)
 *   bytes 4-5  uint16   code  the LUT row index (bit c = [margin_c > 0])
 *   byte  6    uint8    r     the comparison index of u
 *   byte  7    uint8    0
 */
typedef struct tropnn_route_record {
    float u;
    uint16_t code;
    uint8_t r;
    uint8_t reserved;
} tropnn_route_record;

typedef void *tropnn_stream_t; /* hipStream_t */

/* ABI version of the loaded library; callers compare with TROPNN_HIP_ABI_VERSION. */
int tropnn_hip_abi_version(void);

/* Last error message of the calling thread ("" after a successful call). */
const char *tropnn_hip_last_error(void);

/*
 * Eval forward with f32 / f16 weights. Replaces the Zig exports
 * lut_forward_batch_with_offsets_no_cache and lut_forward_batch_f16_no_cache
 * (kernels/src/lut.zig:255-285, 288-318): same argument order and meaning
 * (weights [tables, 2^comparisons, output_dim], anchors [tables, comparisons, 2],
 * offsets = thresholds [tables, comparisons], inputs [batch, input_dim],
 * outputs [batch, output_dim], fully overwritten), plus the output scale the
 * module applies afterwards (layers/base.py:76-77) and the stream.
 */
int tropnn_hip_lut_forward_batch_f32(size_t batch, size_t tables, size_t comparisons, size_t input_dim,
                                     size_t output_dim, const float *weights, const int64_t *anchors,
                                     const float *offsets, const float *inputs, float *outputs, float output_scale,
                                     tropnn_stream_t stream);
int tropnn_hip_lut_forward_batch_f16(size_t batch, size_t tables, size_t comparisons, size_t input_dim,
                                     size_t output_dim, const uint16_t *weights_f16, const int64_t *anchors,
                                     const float *offsets, const float *inputs, float *outputs, float output_scale,
                                     tropnn_stream_t stream);

/*
 * Forward of the training / debug path. Replaces the TileLang route and
 * forward kernels with their launcher _run_forward
 * (backends/pairwise_tilelang.py:17-115, 413-457), fused into one launch:
 *   output[b,:]       = output_scale * sum_t lut[t, code[b,t], :]      [items, out_features]
 *   route_record      = per (table, item) record above, or NULL         [tables, items]
 *   indices[b,t]      = code as int64, or NULL                          [items, tables]
 *   margins[b,t,c]    = (x[b,a] - x[b,b']) - thr[t,c], or NULL          [items, tables, comparisons]
 *   codes[b,t]        = code as uint8, or NULL                          [items, tables]
 * lut_dtype selects float (TROPNN_LUT_F32) or binary16 (TROPNN_LUT_F16) rows.
 * indices and margins are the route-debug tensors of the reference's shell
 * (layers/base.py:78-83); codes is their compact form (comparisons <= 8), one
 * byte per (item, table) instead of 8 + 4 * comparisons.
 */
int tropnn_hip_pairwise_forward(int64_t items, int64_t in_features, int64_t out_features, int64_t tables,
                                int64_t comparisons, const float *latent, const int64_t *anchors,
                                const float *thresholds, const void *lut, int lut_dtype, float output_scale,
                                float *output, tropnn_route_record *route_record, int64_t *indices, float *margins,
                                uint8_t *codes, tropnn_stream_t stream);

/*
 * Route only: the comparator codes and margins of every (item, table), with
 * no LUT access. Replaces PairwiseLinear._compute_indices
 * (layers/pairwise.py:127-135), which returns (indices, margins). Writes any
 * of codes (uint8 [items, tables]), indices (int64 [items, tables]) and
 * margins (f32 [items, tables, comparisons]); NULL skips one. The margins are
 * bit-identical to the forward's. Used to materialise route-debug tensors
 * after a forward that wrote only codes.
 */
int tropnn_hip_pairwise_route(int64_t items, int64_t in_features, int64_t tables, int64_t comparisons,
                              const float *latent, const int64_t *anchors, const float *thresholds, uint8_t *codes,
                              int64_t *indices, float *margins, tropnn_stream_t stream);

/* Bytes of device workspace tropnn_hip_pairwise_backward needs for these dims
 * and STE mode (0 and an error message for invalid arguments). */
size_t tropnn_hip_pairwise_backward_workspace_size(int64_t items, int64_t in_features, int64_t out_features,
                                                   int64_t tables, int64_t comparisons, int lut_dtype, int ste_mode);

/*
 * Inverse anchor index used by the input-gradient backward: for every input
 * feature f, offsets[f] .. offsets[f+1] delimit its entries in `entries`,
 * each ((t * comparisons + c) << 1) | side, the flat position of an
 * anchors[t][c][side] equal to f, in increasing order (a fixed summation
 * order, so grad_latent is deterministic). offsets: in_features + 1 int32; entries: 2 * tables *
 * comparisons int32. Depends on the anchors only: build once, rebuild when
 * the anchors change. No counterpart in the reference, whose input gradient
 * is an index_put accumulate (layers/pairwise.py:131-132) or an atomic add
 * (backends/pairwise_tilelang.py:279-284).
 */
int tropnn_hip_build_anchor_index(int64_t in_features, int64_t tables, int64_t comparisons, const int64_t *anchors,
                                  int32_t *offsets, int32_t *entries, tropnn_stream_t stream);

/*
 * Backward of the training forward. Replaces _PairwiseTileLangFunction.backward
 * and its LUT-scatter, min-STE and full-STE kernels
 * (backends/pairwise_tilelang.py:118-410, 481-534); the math is the autograd
 * of the torch path (layers/pairwise.py:137-200, layers/surrogate.py:9-38):
 *   g[b,:]            = output_scale * grad_output[b,:]
 *   grad_lut[t,r,:]   = sum_{b: code[b,t]=r} g[b,:]                      (fully overwritten)
 * ste_mode = TROPNN_STE_MIN_MARGIN (r = the record's min-margin comparison,
 * u = its margin):
 *   D[b,t]            = sum_o g[b,o] * (lut[t,nb,o] - lut[t,code,o]),   nb = code ^ (1 << r)
 *   gu[b,t]           = D[b,t] * surrogate'(u[b,t])
 *   grad_latent[b,i]  = sum_t gu[b,t] * ([i = a(t,r)] - [i = b'(t,r)])   (fully overwritten)
 *   grad_thresholds[t,c] = -sum_b [r[b,t] = c] * gu[b,t]                (fully overwritten)
 * ste_mode = TROPNN_STE_FULL: every comparison c contributes, with its own
 * margin margins[b,t,c] (the forward's margins output, required when
 * grad_latent or grad_thresholds is asked for) and nb = code ^ (1 << c):
 *   gu[b,t,c] = D[b,t,c] * surrogate'(margins[b,t,c]); grad_latent and
 *   grad_thresholds sum gu[b,t,c] over every c.
 * surrogate: TROPNN_SURROGATE_FAST_SIGMOID_ODD or TROPNN_SURROGATE_IZHIKEVICH.
 * Every sum runs in a fixed order: the results are deterministic.
 * Any of the three gradient pointers may be NULL to skip that gradient;
 * grad_latent needs the anchor index (index_offsets / index_entries from
 * tropnn_hip_build_anchor_index), the others accept NULL index pointers.
 * workspace: device memory of at least
 * tropnn_hip_pairwise_backward_workspace_size() bytes (same ste_mode), 16-byte
 * aligned, whenever a gradient is asked for.
 */
int tropnn_hip_pairwise_backward(int64_t items, int64_t in_features, int64_t out_features, int64_t tables,
                                 int64_t comparisons, const float *grad_output, const void *lut, int lut_dtype,
                                 const tropnn_route_record *route_record, const float *margins,
                                 const int32_t *index_offsets, const int32_t *index_entries, float output_scale,
                                 int ste_mode, int surrogate, float *grad_latent, float *grad_thresholds,
                                 float *grad_lut, void *workspace, size_t workspace_bytes, tropnn_stream_t stream);

/*
 * Allocation-free variant of tropnn_hip_pairwise_backward. It has no
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving or training loops,
 * harnesses that forbid hipMalloc. Same arguments, results and errors, minus
 * the workspace: the kernels use a device buffer of
 * TROPNN_NOALLOC_WORKSPACE_BYTES that the library holds, one per GPU, from
 * the first call on that GPU until the process ends. The call allocates
 * nothing. A shape whose workspace (tropnn_hip_pairwise_backward_workspace_size)
 * is larger fails with TROPNN_ERR_UNSUPPORTED before any launch. Every call
 * on one GPU shares that GPU's buffer: calls that overlap on one GPU (other
 * streams, other threads, without ordering between them) race on it and give
 * wrong gradients; serialise them. The buffer needs no clearing between calls.
 * The first call on a GPU looks up that GPU's buffer address (a runtime call,
 * not stream work), so it must not be under stream capture: it fails with
 * TROPNN_ERR_UNSUPPORTED if it is. Once one call on the GPU has run outside
 * capture, calls under capture record only kernel launches (no memset, no
 * allocation) and replay correctly.
 */
#define TROPNN_NOALLOC_WORKSPACE_BYTES (32u << 20)
int tropnn_hip_pairwise_backward_noalloc(int64_t items, int64_t in_features, int64_t out_features, int64_t tables,
                                         int64_t comparisons, const float *grad_output, const void *lut,
                                         int lut_dtype, const tropnn_route_record *route_record, const float *margins,
                                         const int32_t *index_offsets, const int32_t *index_entries,
                                         float output_scale, int ste_mode, int surrogate, float *grad_latent,
                                         float *grad_thresholds, float *grad_lut, tropnn_stream_t stream);

/*
 * Adam / AdamW step over n_tensors f32 tensors: the optimizer of the
 * classifier's training step. The reference trains it with
 * torch.optim.AdamW(weight_decay=0) (examples/emnist.py:310), i.e. torch's
 * Adam update; this is that update (non-amsgrad, op order of torch's
 * single-tensor Adam) in one launch over all the tensors' elements:
 *   weight_decay != 0: decoupled ? p *= 1 - lr * wd : g += wd * p
 *   m = lerp(m, g, 1 - beta1);  v = v beta2 + (1 - beta2) g^2
 *   p -= (lr / (1 - beta1^t)) * (m / (sqrt(v) / sqrt(1 - beta2^t) + eps))
 * with t = *steps[k] + 1 read from device memory, after which *steps[k] = t
 * (a second launch): a step captured in a HIP graph replays with the current
 * counts. lr and the other scalars are taken by value; as in torch, the bias
 * corrections are formed in f64 and each per-element op is one f32 op (no
 * fused multiply-adds).
 * params, grads, exp_avgs, exp_avg_sqs, steps: HOST arrays of n_tensors
 * DEVICE pointers (f32, 4-byte aligned; numels[k] elements each, one float
 * for steps[k]); the steps pointers must be distinct. exp_avgs and
 * exp_avg_sqs start at zero and the step counters at 0.
 */
int tropnn_hip_adam_step(int n_tensors, float *const *params, const float *const *grads, float *const *exp_avgs,
                         float *const *exp_avg_sqs, const int64_t *numels, float *const *steps, double lr,
                         double beta1, double beta2, double eps, double weight_decay, int decoupled_weight_decay,
                         tropnn_stream_t stream);

/*
 * Mean cross entropy of the classifier's training step (the reference's
 * F.cross_entropy(logits, y), examples/emnist.py:221) and its gradient, in
 * one launch: loss[0] = sum over rows i with target[i] != ignore_index of
 * (logsumexp(logits[i]) - logits[i][target[i]]), divided by their count;
 * grad_logits[i][j] = (softmax(logits[i])[j] - [j == target[i]]) / count
 * (0 on ignored rows), i.e. d loss / d logits. logits f32 [rows][classes],
 * target int64 [rows], loss f32 [1], grad_logits f32 [rows][classes]: DEVICE
 * pointers, 4-byte (target 8-byte) aligned. A target outside [0, classes)
 * that is not ignore_index gives a NaN loss; every row ignored gives NaN
 * (0 / 0), as torch.
 */
int tropnn_hip_cross_entropy(int64_t rows, int64_t classes, const float *logits, const int64_t *target,
                             int64_t ignore_index, float *loss, float *grad_logits, tropnn_stream_t stream);

/*
 * Profiling hook (no counterpart in the reference, whose harness times whole
 * calls, tools/benchmarking/benchmark.py:91-118). Arms two caller-created
 * hipEvent_t handles to be recorded on the launch stream immediately before
 * and after the NEXT launch of one kernel:
 *   TROPNN_KERNEL_FORWARD           the fused route + gather + scale kernel (large training
 *                                   shapes: the streamed gather + scale kernel)
 *   TROPNN_KERNEL_FORWARD_ROUTE     the route-record kernel before the streamed gather (training
 *                                   forward with at least 4096 items, LUT rows of whole 128-byte
 *                                   chunks, comparisons <= 8 and a LUT of at least 32 MiB)
 *   TROPNN_KERNEL_BACKWARD_TABLE    the per-(table, column chunk) LUT-gradient kernel (with the
 *                                   min-margin STE: also each chunk's partial STE dots)
 *   TROPNN_KERNEL_BACKWARD_ITEM     the per-item STE-dot / input-gradient kernel of the full STE
 *   TROPNN_KERNEL_BACKWARD_SORT     the per-table code sort kernel before the row kernel
 *                                   (full STE: also the threshold gradient)
 *   TROPNN_KERNEL_BACKWARD_REDUCE   the per-table kernel after it (min-margin): partial dots ->
 *                                   gu, threshold gradient, {gu, r} records
 *   TROPNN_KERNEL_BACKWARD_FUSED    the per-table LUT-gradient / STE-dot / threshold-gradient
 *                                   kernel of narrow rows (out_features a multiple of 4 up to 64
 *                                   or of 8 up to 256, one table's rows within 64 KB as f32)
 *   TROPNN_KERNEL_BACKWARD_SCATTER  the per-item input-gradient kernel after FUSED or REDUCE
 * A backward launches FUSED then SCATTER (narrow rows), or SORT, TABLE, REDUCE and
 * SCATTER (other rows, min-margin STE), or ITEM, SORT and TABLE (other rows, full STE).
 * One-shot and process-global (not for concurrent use from several threads).
 * Passing NULL events disarms. Lets a benchmark time one kernel per step with
 * events on the exact stream the kernel runs on.
 */
#define TROPNN_KERNEL_FORWARD 0
#define TROPNN_KERNEL_BACKWARD_TABLE 1
#define TROPNN_KERNEL_BACKWARD_ITEM 2
#define TROPNN_KERNEL_BACKWARD_FUSED 3
#define TROPNN_KERNEL_BACKWARD_SCATTER 4
#define TROPNN_KERNEL_BACKWARD_SORT 5
#define TROPNN_KERNEL_BACKWARD_REDUCE 6
#define TROPNN_KERNEL_FORWARD_ROUTE 7
int tropnn_hip_arm_kernel_events(int kernel, void *start_event, void *stop_event);

#ifdef __cplusplus
}
#endif

#endif /* TROPNN_HIP_H */
