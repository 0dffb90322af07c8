"""HIP backend of PairwiseLinear: ctypes binding of libtropnn_hip.so plus the
autograd operator around it.

Public entry points mirror the reference's backend wrappers:
  * pairwise_hip(...)          -- like pairwise_tilelang (backends/pairwise_tilelang.py:537-549):
                                  autograd operator, returns (output, indices, margins)
  * pairwise_hip_forward(...)  -- like pairwise_zig_forward (backends/pairwise_zig.py:35-103):
                                  eval-only forward with an f32 or f16 LUT
  * has_pairwise_hip()         -- capability probe like has_pairwise_zig / has_tilelang
                                  (backend.py:15-42)

Errors follow the reference wrappers: RuntimeError when the native library or
a GPU is missing (pairwise_tilelang.py:421-422, zig_runtime.py:81-87),
ValueError for a non-GPU tensor or a bad shape, TypeError for a wrong dtype
(pairwise_tilelang.py:423-436, pairwise_zig.py:43-61). There is no CPU
fallback: every call runs the HIP kernels or raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path
from typing import Any

import torch
from torch import Tensor

ABI_VERSION = 11
LUT_F32, LUT_F16 = 0, 1
SURROGATE_IDS = {"fast_sigmoid_odd": 0, "izhikevich": 1}
STE_MIN_MARGIN, STE_FULL = 0, 1
BWD_INPUT_GRAD_FUSED, BWD_INPUT_GRAD_SCATTER = 0x100, 0x200  # flags ORed into the STE mode
MAX_COMPARISONS = 8
ERR_NAMES = {1: "invalid argument", 2: "unsupported", 3: "HIP error"}

_PKG_DIR = Path(__file__).resolve().parent.parent
DEFAULT_LIBRARY = _PKG_DIR / "libtropnn_hip.so"
# host-only torch operator library (csrc/autograd_op.cpp): the autograd
# operator behind pairwise_hip, which calls the C ABI of the library above
OPS_LIBRARY = _PKG_DIR / "libtropnn_hip_torch.so"
_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None
_PAIRWISE_OP: Any = None
_ROUTE_MODES = {False: 0, True: 1, "codes": 2}
# where the backward forms the latent gradient of narrow rows (the operator's
# input_grad argument): the library's row-width rule, the fused launch, or a
# kernel after it
INPUT_GRAD_FORMS = {"auto": 0, "fused": 1, "scatter": 2}
# Per-anchors-tensor caches live as attributes of the anchors tensor object
# itself (not in a table keyed by address: the caching allocator reuses the
# addresses of freed tensors), validated by the tensor's version counter,
# which every in-place write bumps.
_CHECKED_ATTR = "_tropnn_hip_checked"
_INDEX_ATTR = "_tropnn_hip_anchor_index"

EXPORTED_SYMBOLS = (
    "tropnn_hip_abi_version",
    "tropnn_hip_last_error",
    "tropnn_hip_lut_forward_batch_f32",
    "tropnn_hip_lut_forward_batch_f16",
    "tropnn_hip_pairwise_forward",
    "tropnn_hip_pairwise_route",
    "tropnn_hip_pairwise_backward_workspace_size",
    "tropnn_hip_pairwise_backward",
    "tropnn_hip_pairwise_backward_noalloc",
    "tropnn_hip_build_anchor_index",
    "tropnn_hip_arm_kernel_events",
    "tropnn_hip_adam_step",
    "tropnn_hip_cross_entropy",
)
KERNEL_IDS = {
    "forward": 0,
    "backward_table": 1,
    "backward_item": 2,
    "backward_fused": 3,
    "backward_scatter": 4,
    "backward_sort": 5,
    "backward_reduce": 6,
    "forward_route": 7,
}


def library_path() -> Path:
    """TROPNN_HIP_LIB overrides the in-tree build location."""
    env = os.environ.get("TROPNN_HIP_LIB")
    return Path(env) if env else DEFAULT_LIBRARY


def _declare(lib: ctypes.CDLL) -> None:
    i64, sz, p, f, i = ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float, ctypes.c_int
    lib.tropnn_hip_abi_version.argtypes = []
    lib.tropnn_hip_abi_version.restype = i
    lib.tropnn_hip_last_error.argtypes = []
    lib.tropnn_hip_last_error.restype = ctypes.c_char_p
    for name in ("tropnn_hip_lut_forward_batch_f32", "tropnn_hip_lut_forward_batch_f16"):
        fn = getattr(lib, name)
        fn.argtypes = [sz, sz, sz, sz, sz, p, p, p, p, p, f, p]
        fn.restype = i
    lib.tropnn_hip_pairwise_forward.argtypes = [i64, i64, i64, i64, i64, p, p, p, p, i, f, p, p, p, p, p, p]
    lib.tropnn_hip_pairwise_forward.restype = i
    lib.tropnn_hip_pairwise_route.argtypes = [i64, i64, i64, i64, p, p, p, p, p, p, p]
    lib.tropnn_hip_pairwise_route.restype = i
    lib.tropnn_hip_pairwise_backward_workspace_size.argtypes = [i64, i64, i64, i64, i64, i, i]
    lib.tropnn_hip_pairwise_backward_workspace_size.restype = sz
    lib.tropnn_hip_build_anchor_index.argtypes = [i64, i64, i64, p, p, p, p]
    lib.tropnn_hip_build_anchor_index.restype = i
    lib.tropnn_hip_pairwise_backward.argtypes = [i64, i64, i64, i64, i64, p, p, i, p, p, p, p, f, i, i, p, p, p, p, sz, p]
    lib.tropnn_hip_pairwise_backward.restype = i
    lib.tropnn_hip_pairwise_backward_noalloc.argtypes = [i64, i64, i64, i64, i64, p, p, i, p, p, p, p, f, i, i, p, p, p, p]
    lib.tropnn_hip_pairwise_backward_noalloc.restype = i
    lib.tropnn_hip_arm_kernel_events.argtypes = [i, p, p]
    lib.tropnn_hip_arm_kernel_events.restype = i
    d = ctypes.c_double
    lib.tropnn_hip_adam_step.argtypes = [i, p, p, p, p, p, p, d, d, d, d, d, i, p]
    lib.tropnn_hip_adam_step.restype = i
    lib.tropnn_hip_cross_entropy.argtypes = [i64, i64, p, p, i64, p, p, p]
    lib.tropnn_hip_cross_entropy.restype = i


def load_library() -> ctypes.CDLL:
    """Load libtropnn_hip.so once (under a lock), after torch's HIP runtime,
    so both share one libamdhip64 instance. Raises RuntimeError if the file is
    missing or its ABI version differs."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"PairwiseLinear backend='hip' needs {path}, which is not built; "
                "build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C tropnn_amd/csrc`"
            )
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as exc:
            raise RuntimeError(f"cannot load {path}: {exc}") from exc
        missing = [s for s in EXPORTED_SYMBOLS if not hasattr(lib, s)]
        if missing:
            raise RuntimeError(f"{path} lacks symbols {missing}")
        _declare(lib)
        version = lib.tropnn_hip_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, this package expects {ABI_VERSION}")
        _LIB = lib
    return _LIB


def _pairwise_op() -> Any:
    """torch.ops.tropnn_hip.pairwise, loaded once and bound to the entry
    points of the libtropnn_hip.so that load_library() loaded and checked.
    Raises RuntimeError if the operator library is not built."""
    global _PAIRWISE_OP
    if _PAIRWISE_OP is not None:
        return _PAIRWISE_OP
    lib = load_library()
    with _LOCK:
        if _PAIRWISE_OP is not None:
            return _PAIRWISE_OP
        if not OPS_LIBRARY.exists():
            raise RuntimeError(
                f"PairwiseLinear backend='hip' needs {OPS_LIBRARY}, which is not built; "
                "build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C tropnn_amd/csrc`"
            )
        if not hasattr(torch.ops.tropnn_hip, "bind_abi"):
            try:
                torch.ops.load_library(str(OPS_LIBRARY))
            except OSError as exc:
                raise RuntimeError(f"cannot load {OPS_LIBRARY}: {exc}") from exc

        def addr(name: str) -> int:
            return ctypes.cast(getattr(lib, name), ctypes.c_void_p).value

        torch.ops.tropnn_hip.bind_abi(
            addr("tropnn_hip_pairwise_forward"),
            addr("tropnn_hip_pairwise_backward"),
            addr("tropnn_hip_pairwise_backward_workspace_size"),
            addr("tropnn_hip_last_error"),
            lib.tropnn_hip_abi_version(),
        )
        _PAIRWISE_OP = torch.ops.tropnn_hip.pairwise.default
    return _PAIRWISE_OP


def has_pairwise_hip() -> bool:
    """True when the native libraries load and a GPU is visible."""
    if not torch.cuda.is_available():
        return False
    try:
        load_library()
        _pairwise_op()
    except RuntimeError:
        return False
    return True


def _check(rc: int, what: str) -> None:
    if rc == 0:
        return
    msg = load_library().tropnn_hip_last_error().decode(errors="replace")
    if rc == 2:
        raise NotImplementedError(f"{what}: {msg}")
    if rc == 1:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {ERR_NAMES.get(rc, rc)}: {msg}")


def arm_kernel_events(kernel: str, start: "torch.cuda.Event | None", stop: "torch.cuda.Event | None") -> None:
    """Record `start` / `stop` (torch.cuda.Event objects that have been
    recorded once, so their handles exist) around the next launch of `kernel`
    (a key of KERNEL_IDS); None disarms."""
    lib = load_library()
    h0 = None if start is None else start.cuda_event
    h1 = None if stop is None else stop.cuda_event
    _check(lib.tropnn_hip_arm_kernel_events(KERNEL_IDS[kernel], h0, h1), "tropnn_hip_arm_kernel_events")


def _stream(device: torch.device) -> int:
    """The raw hipStream_t of the device's current stream (no Stream object)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_gpu(*tensors: Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            if not torch.cuda.is_available():
                raise RuntimeError(
                    "PairwiseLinear backend='hip' requires a visible AMD GPU (torch.cuda.is_available() is False)"
                )
            raise ValueError("PairwiseLinear backend='hip' requires GPU tensors")


def check_anchors(anchors: Tensor, in_features: int) -> None:
    """Every anchor must index the input row. Checked once per anchors tensor
    and version because it reads the tensor back to the host."""
    key = (anchors._version, in_features)
    if getattr(anchors, _CHECKED_ATTR, None) == key:
        return
    if anchors.numel() > 0:
        lo, hi = int(anchors.min().item()), int(anchors.max().item())
        if lo < 0 or hi >= in_features:
            raise ValueError(f"anchors must lie in [0, {in_features}), got range [{lo}, {hi}]")
    setattr(anchors, _CHECKED_ATTR, key)


def anchor_index(anchors: Tensor, in_features: int) -> tuple[Tensor, Tensor]:
    """(offsets [I+1], entries [2TC]) int32 inverse anchor index on the
    anchors' device, built by tropnn_hip_build_anchor_index and cached per
    anchors tensor and version: the anchors are a buffer that training never
    changes, so this runs once per layer."""
    key = (anchors._version, in_features)
    hit = getattr(anchors, _INDEX_ATTR, None)
    if hit is not None and hit[0] == key:
        return hit[1], hit[2]
    if anchors.dtype != torch.int64:
        raise TypeError(f"anchors must be int64, got {anchors.dtype}")
    if anchors.ndim != 3 or anchors.shape[2] != 2:
        raise ValueError(f"anchors must have shape [tables, comparisons, 2], got {tuple(anchors.shape)}")
    _require_gpu(anchors)
    tables, comps, _ = anchors.shape
    offsets = torch.empty(in_features + 1, device=anchors.device, dtype=torch.int32)
    entries = torch.empty(max(2 * tables * comps, 1), device=anchors.device, dtype=torch.int32)
    anc = anchors.contiguous()
    rc = load_library().tropnn_hip_build_anchor_index(
        in_features, tables, comps, _ptr(anc), _ptr(offsets), _ptr(entries), _stream(anchors.device)
    )
    _check(rc, "tropnn_hip_build_anchor_index")
    setattr(anchors, _INDEX_ATTR, (key, offsets, entries))
    return offsets, entries


def _validate(latent: Tensor, anchors: Tensor, thresholds: Tensor, lut: Tensor) -> tuple[int, int, int, int, int, int]:
    if latent.ndim != 3:
        raise ValueError(f"latent must have shape [batch, steps, in_features], got {tuple(latent.shape)}")
    if latent.dtype != torch.float32 or thresholds.dtype != torch.float32:
        raise TypeError(f"Pairwise HIP backend expects float32 latent and thresholds, got {latent.dtype}, {thresholds.dtype}")
    if anchors.dtype != torch.int64:
        raise TypeError(f"anchors must be int64, got {anchors.dtype}")
    if lut.dtype not in (torch.float32, torch.float16):
        raise TypeError(f"lut must be float32 or float16, got {lut.dtype}")
    batch, steps, in_features = latent.shape
    if anchors.ndim != 3 or anchors.shape[2] != 2:
        raise ValueError(f"anchors must have shape [tables, comparisons, 2], got {tuple(anchors.shape)}")
    tables, comps, _ = anchors.shape
    if thresholds.shape != (tables, comps):
        raise ValueError(f"thresholds must have shape {(tables, comps)}, got {tuple(thresholds.shape)}")
    if lut.ndim != 3 or lut.shape[0] != tables or lut.shape[1] != (1 << comps):
        raise ValueError(f"lut must have shape [{tables}, {1 << comps}, out_features], got {tuple(lut.shape)}")
    if comps > MAX_COMPARISONS:
        raise NotImplementedError(f"Pairwise HIP backend supports comparisons <= {MAX_COMPARISONS}, got {comps}")
    devs = {t.device for t in (latent, anchors, thresholds, lut)}
    if len(devs) != 1:
        raise ValueError(f"all tensors must be on one device, got {sorted(map(str, devs))}")
    return batch, steps, in_features, tables, comps, lut.shape[2]


def _route_forward(
    latent: Tensor,
    anchors: Tensor,
    thresholds: Tensor,
    lut_read: Tensor,
    *,
    output_scale: float,
    want_record: bool,
    return_route: bool | str,
    want_margins: bool = False,
) -> tuple[Tensor, Tensor | None, Tensor, Tensor, Tensor | None]:
    """One fused forward launch. Returns (output, record, indices, margins,
    saved_margins); saved_margins [items, tables, comparisons] is the margins
    tensor the full-STE backward reads (want_margins), else None.
    return_route: True = int64 indices and f32 margins; "codes" = uint8 codes
    in place of indices and empty margins; False = both empty."""
    batch, steps, in_features, tables, comps, out_features = _validate(latent, anchors, thresholds, lut_read)
    check_anchors(anchors, in_features)
    items = batch * steps
    dev = latent.device
    x = latent.reshape(items, in_features).contiguous()
    anc, thr, lut_c = anchors.contiguous(), thresholds.contiguous(), lut_read.contiguous()
    out = torch.empty((items, out_features), device=dev, dtype=torch.float32)
    record = torch.empty((tables, items), device=dev, dtype=torch.int64) if want_record else None
    full_route = return_route is True
    codes = torch.empty((items, tables), device=dev, dtype=torch.uint8) if return_route == "codes" else None
    if full_route:
        indices = torch.empty((items, tables), device=dev, dtype=torch.int64)
        margins = torch.empty((items, tables, comps), device=dev, dtype=torch.float32)
    else:
        indices = torch.empty((items, 0), device=dev, dtype=torch.int64)
        margins = torch.empty((items, 0), device=dev, dtype=torch.float32)
    saved = None  # margins the full-STE backward reads
    if want_margins:
        saved = margins if full_route else torch.empty((items, tables, comps), device=dev, dtype=torch.float32)
    lib = load_library()
    rc = lib.tropnn_hip_pairwise_forward(
        items,
        in_features,
        out_features,
        tables,
        comps,
        _ptr(x),
        _ptr(anc),
        _ptr(thr),
        _ptr(lut_c),
        LUT_F16 if lut_c.dtype == torch.float16 else LUT_F32,
        float(output_scale),
        _ptr(out),
        _ptr(record),
        _ptr(indices) if full_route else None,
        _ptr(margins) if full_route else _ptr(saved),
        _ptr(codes),
        _stream(dev),
    )
    _check(rc, "tropnn_hip_pairwise_forward")
    if full_route:
        idx_view = indices.view(batch, steps, tables)
        mar_view = margins.view(batch, steps, tables, comps)
    elif codes is not None:
        idx_view = codes.view(batch, steps, tables)
        mar_view = margins.view(batch, steps, 0)
    else:
        idx_view = indices.view(batch, steps, 0)
        mar_view = margins.view(batch, steps, 0)
    return out.view(batch, steps, out_features), record, idx_view, mar_view, saved


def pairwise_hip(
    latent: Tensor,
    anchors: Tensor,
    thresholds: Tensor,
    lut: Tensor,
    *,
    use_min_margin_ste: bool = True,
    surrogate: str = "fast_sigmoid_odd",
    output_scale: float = 1.0,
    lut_read: Tensor | None = None,
    ste: bool = True,
    return_route: bool | str = True,
    input_grad: str = "auto",
) -> tuple[Tensor, Tensor, Tensor]:
    """HIP counterpart of pairwise_tilelang (backends/pairwise_tilelang.py:537-549).

    latent [B,S,I] f32, anchors [T,C,2] int64, thresholds [T,C] f32,
    lut [T,2^C,O] f32 (the parameter gradients flow to). Returns
    (output [B,S,O] = output_scale * sum_t lut[t, code], indices [B,S,T] int64,
    margins [B,S,T,C] f32); with return_route=False the last two are empty
    [B,S,0] tensors, as the Zig path returns (layers/pairwise.py:223-225);
    with return_route="codes" the second is the uint8 codes [B,S,T] and the
    third is empty (pairwise_hip_route computes margins on demand).

    lut_read: the tensor the kernels read, e.g. an f16 copy of lut (f32 by
    default = lut itself). ste: carry the STE gradient (min-margin, or every
    comparison with use_min_margin_ste=False) to latent and
    thresholds (the torch path does so only in training,
    layers/pairwise.py:245-247). output_scale defaults to 1.0, the
    pairwise_tilelang contract (the module scales afterwards); the package's
    PairwiseLinear passes its 1/sqrt(T) here so the scale is fused.

    The autograd operator (torch.ops.tropnn_hip.pairwise, csrc/autograd_op.cpp)
    has the contract of _PairwiseTileLangFunction
    (backends/pairwise_tilelang.py:460-534): gradients flow to latent,
    thresholds and lut; indices and margins are non-differentiable. Forward:
    one fused route + gather + scale launch, which also writes the per-(table,
    item) route record the backward reads when a gradient will be asked for
    (none under torch.no_grad). Backward: table-major LUT gradient + min-margin
    or full STE (fast_sigmoid_odd or izhikevich surrogate), then input /
    threshold gradients; only the gradients the backward pass asks for are
    computed. The full STE needs every comparison's margin, which the forward
    then keeps.

    input_grad: "auto", "fused" or "scatter", where the min-margin backward of
    narrow rows forms the latent gradient (no counterpart in the reference;
    the results are the same bits either way, see PairwiseLinear).
    """
    surrogate_id = SURROGATE_IDS.get(surrogate)
    if surrogate_id is None:
        raise ValueError(f"Pairwise HIP backend does not support surrogate={surrogate!r}")
    route_mode = _ROUTE_MODES.get(return_route) if isinstance(return_route, (bool, str)) else None
    if route_mode is None:
        raise ValueError(f"return_route must be True, False or 'codes', got {return_route!r}")
    input_grad_id = INPUT_GRAD_FORMS.get(input_grad) if isinstance(input_grad, str) else None
    if input_grad_id is None:
        raise ValueError(f"input_grad must be 'auto', 'fused' or 'scatter', got {input_grad!r}")
    _require_gpu(latent, anchors, thresholds, lut)
    op = _pairwise_op()
    if latent.ndim != 3:
        raise ValueError(f"latent must have shape [batch, steps, in_features], got {tuple(latent.shape)}")
    in_features = latent.shape[2]
    check_anchors(anchors, in_features)
    offsets = entries = None
    if ste and latent.requires_grad and torch.is_grad_enabled():
        # built once per anchors version, at forward time (outside any
        # backward-pass graph capture)
        offsets, entries = anchor_index(anchors, in_features)
    return op(
        latent,
        anchors,
        thresholds,
        lut,
        lut if lut_read is None else lut_read,
        offsets,
        entries,
        bool(ste),
        bool(use_min_margin_ste),
        surrogate_id,
        float(output_scale),
        route_mode,
        input_grad_id,
    )


def pairwise_hip_route(
    latent: Tensor,
    anchors: Tensor,
    thresholds: Tensor,
    *,
    codes: bool = False,
    indices: bool = True,
    margins: bool = True,
) -> tuple[Tensor | None, Tensor | None, Tensor | None]:
    """Route only, the HIP counterpart of PairwiseLinear._compute_indices
    (layers/pairwise.py:127-135): returns (codes [B,S,T] uint8, indices
    [B,S,T] int64, margins [B,S,T,C] f32), None for each one not asked for.
    No LUT access and no autograd; the margins are bit-identical to the
    forward's."""
    _require_gpu(latent, anchors, thresholds)
    if latent.ndim != 3:
        raise ValueError(f"latent must have shape [batch, steps, in_features], got {tuple(latent.shape)}")
    if latent.dtype != torch.float32 or thresholds.dtype != torch.float32:
        raise TypeError(f"Pairwise HIP backend expects float32 latent and thresholds, got {latent.dtype}, {thresholds.dtype}")
    if anchors.dtype != torch.int64:
        raise TypeError(f"anchors must be int64, got {anchors.dtype}")
    if anchors.ndim != 3 or anchors.shape[2] != 2:
        raise ValueError(f"anchors must have shape [tables, comparisons, 2], got {tuple(anchors.shape)}")
    batch, steps, in_features = latent.shape
    tables, comps, _ = anchors.shape
    if thresholds.shape != (tables, comps):
        raise ValueError(f"thresholds must have shape {(tables, comps)}, got {tuple(thresholds.shape)}")
    if comps > MAX_COMPARISONS:
        raise NotImplementedError(f"Pairwise HIP backend supports comparisons <= {MAX_COMPARISONS}, got {comps}")
    check_anchors(anchors, in_features)
    items = batch * steps
    dev = latent.device
    x = latent.detach().reshape(items, in_features).contiguous()
    c_out = torch.empty((batch, steps, tables), device=dev, dtype=torch.uint8) if codes else None
    i_out = torch.empty((batch, steps, tables), device=dev, dtype=torch.int64) if indices else None
    m_out = torch.empty((batch, steps, tables, comps), device=dev, dtype=torch.float32) if margins else None
    rc = load_library().tropnn_hip_pairwise_route(
        items,
        in_features,
        tables,
        comps,
        _ptr(x),
        _ptr(anchors.contiguous()),
        _ptr(thresholds.detach().contiguous()),
        _ptr(c_out),
        _ptr(i_out),
        _ptr(m_out),
        _stream(dev),
    )
    _check(rc, "tropnn_hip_pairwise_route")
    return c_out, i_out, m_out


def pairwise_hip_forward(
    latent: Tensor,
    anchors: Tensor,
    thresholds: Tensor,
    lut: Tensor,
    *,
    lut_dtype: str = "f32",
    output_scale: float = 1.0,
) -> Tensor:
    """Eval-only forward, the HIP counterpart of pairwise_zig_forward
    (backends/pairwise_zig.py:35-103): no autograd, no route outputs, the LUT
    read as f32 or as an RNE f16 copy. Calls the Zig-ABI-shaped entry points
    tropnn_hip_lut_forward_batch_f32 / _f16."""
    if lut_dtype not in ("f32", "f16"):
        raise ValueError(f"lut_dtype must be 'f32' or 'f16', got {lut_dtype!r}")
    _require_gpu(latent, anchors, thresholds, lut)
    weights = lut.detach().to(torch.float16 if lut_dtype == "f16" else torch.float32)
    batch, steps, in_features, tables, comps, out_features = _validate(latent, anchors, thresholds.detach(), weights)
    check_anchors(anchors, in_features)
    items = batch * steps
    x = latent.detach().reshape(items, in_features).contiguous()
    out = torch.empty((items, out_features), device=latent.device, dtype=torch.float32)
    lib = load_library()
    fn = lib.tropnn_hip_lut_forward_batch_f16 if lut_dtype == "f16" else lib.tropnn_hip_lut_forward_batch_f32
    w = weights.contiguous()
    thr = thresholds.detach().contiguous()
    anc = anchors.contiguous()
    rc = fn(items, tables, comps, in_features, out_features, _ptr(w), _ptr(anc), _ptr(thr), _ptr(x), _ptr(out),
            float(output_scale), _stream(latent.device))
    _check(rc, fn.__name__)
    return out.view(batch, steps, out_features)
