"""The C ABI of libtropnn_hip.so without a GPU: the library loads, exports
exactly what include/tropnn_hip.h declares, and rejects bad arguments with
the documented codes before any launch (these calls touch no device)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

import importlib

ph = importlib.import_module("tropnn_amd.backends.pairwise_hip")

HEADER = Path(__file__).resolve().parent.parent / "include" / "tropnn_hip.h"


def header_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(tropnn_hip_[a-z0-9_]+)\s*\(", text)))


def header_define(name: str) -> int:
    m = re.search(rf"#define {name} (0x[0-9a-fA-F]+|\d+)", HEADER.read_text())
    assert m, name
    return int(m.group(1), 0)


@pytest.fixture(scope="module")
def lib():
    path = ph.library_path()
    if not path.exists():
        pytest.skip("libtropnn_hip.so not built (run __graft_entry__.build())")
    return ph.load_library()


def test_exports_match_header(lib):
    declared = header_functions()
    assert sorted(ph.EXPORTED_SYMBOLS) == declared
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.tropnn_hip_abi_version() == header_define("TROPNN_HIP_ABI_VERSION") == ph.ABI_VERSION


def test_constants_match_header():
    assert header_define("TROPNN_LUT_F32") == ph.LUT_F32
    assert header_define("TROPNN_LUT_F16") == ph.LUT_F16
    assert header_define("TROPNN_SURROGATE_FAST_SIGMOID_ODD") == ph.SURROGATE_IDS["fast_sigmoid_odd"]
    assert header_define("TROPNN_SURROGATE_IZHIKEVICH") == ph.SURROGATE_IDS["izhikevich"]
    assert header_define("TROPNN_MAX_COMPARISONS") == ph.MAX_COMPARISONS
    assert header_define("TROPNN_STE_MIN_MARGIN") == ph.STE_MIN_MARGIN
    assert header_define("TROPNN_STE_FULL") == ph.STE_FULL
    assert header_define("TROPNN_BWD_INPUT_GRAD_FUSED") == ph.BWD_INPUT_GRAD_FUSED
    assert header_define("TROPNN_BWD_INPUT_GRAD_SCATTER") == ph.BWD_INPUT_GRAD_SCATTER
    for name, kid in ph.KERNEL_IDS.items():
        assert header_define("TROPNN_KERNEL_" + name.upper()) == kid


def test_workspace_size(lib):
    ws = lib.tropnn_hip_pairwise_backward_workspace_size
    # min-margin, fused path: the scatter kernel reads {gu, r} records
    # [T][B] x 8 bytes, unless the fused launch's item role forms the input
    # gradient itself (no workspace): at most 192 tables and T x row bytes
    # <= 448 (256 - T)
    assert ws(512, 128, 128, 136, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 136 * 512 * 8  # c2: 512-byte rows
    assert ws(512, 128, 96, 136, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 0  # 384-byte rows
    assert ws(512, 128, 128, 136, 6, ph.LUT_F16, ph.STE_MIN_MARGIN) == 0  # f16: 256-byte rows
    assert ws(512, 128, 10, 136, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 0  # c5's last layer
    assert ws(512, 128, 8, 192, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 0
    assert ws(512, 128, 8, 193, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 193 * 512 * 8
    assert ws(512, 128, 64, 300, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 300 * 512 * 8
    # general path: {gu, r} [T][B] u64 (full STE: gu [T][C][B] f32), then
    # the sort kernel's slot offsets [T][slots] (slots = B + R (K - 1),
    # rounded up to whole batches of K: K = 4 when the row kernel takes 8
    # columns per lane, O >= 64 and 8 | O, else 8), row starts [T][R + 1],
    # batch rows [T][slots / K], the chunk-major copy of G [chunks][B][P]
    # (P = 64 columns, or the row's width rounded up to the row kernel's
    # lanes) and, min-margin, the row kernel's partial STE dots
    # [T][chunks][slots] f32
    def general(b, o, t, r, c, p, full):
        a16 = lambda v: (v + 15) // 16 * 16
        k = 4 if o >= 64 and o % 8 == 0 else 8
        slots = (b + r * (k - 1) + k - 1) // k * k
        chunks = (o + p - 1) // p
        head = a16(a16(a16(t * b * (4 * c if full else 8)) + t * slots * 4) + t * (r + 1) * 4)
        tail = a16(a16(head + t * (slots // k) * 4) + chunks * b * p * 4)
        return tail if full else a16(tail + t * chunks * slots * 4)

    assert ws(64, 1024, 4096, 512, 8, ph.LUT_F16, ph.STE_MIN_MARGIN) == general(64, 4096, 512, 256, 8, 64, False)
    assert ws(512, 128, 128, 136, 6, ph.LUT_F32, ph.STE_FULL) == general(512, 128, 136, 64, 6, 64, True)
    assert ws(33, 20, 10, 7, 3, ph.LUT_F32, ph.STE_MIN_MARGIN) == 0  # fused (item role), 2 columns per lane
    assert ws(33, 20, 34, 7, 3, ph.LUT_F32, ph.STE_MIN_MARGIN) == general(33, 34, 7, 8, 3, 64, False)
    assert ws(33, 20, 5, 7, 3, ph.LUT_F32, ph.STE_MIN_MARGIN) == general(33, 5, 7, 8, 3, 8, False)
    # 8 columns per lane below 64 columns: no (batches of 8)
    assert ws(33, 20, 40, 7, 3, ph.LUT_F32, ph.STE_FULL) == general(33, 40, 7, 8, 3, 64, True)
    assert ws(512, 128, 128, 136, 9, ph.LUT_F32, ph.STE_MIN_MARGIN) == 0
    assert ws(512, 128, 128, 136, 6, ph.LUT_F32, 7) == 0 and "ste_mode" in _err(lib)
    # the caller's input-gradient flags: FUSED takes the item role past the
    # row-width rule (not past its limits), SCATTER keeps the scatter kernel
    fused, scatter = ph.BWD_INPUT_GRAD_FUSED, ph.BWD_INPUT_GRAD_SCATTER
    assert ws(512, 128, 128, 136, 6, ph.LUT_F32, ph.STE_MIN_MARGIN | fused) == 0  # c2 rows in the fused launch
    assert ws(512, 128, 10, 136, 6, ph.LUT_F32, ph.STE_MIN_MARGIN | scatter) == 136 * 512 * 8
    assert ws(512, 128, 8, 193, 6, ph.LUT_F32, ph.STE_MIN_MARGIN | fused) == 193 * 512 * 8  # over 192 tables
    assert ws(512, 128, 128, 136, 6, ph.LUT_F32, ph.STE_FULL | fused) == general(512, 128, 136, 64, 6, 64, True)
    assert ws(512, 128, 128, 136, 6, ph.LUT_F32, ph.STE_MIN_MARGIN | fused | scatter) == 0 and "flags" in _err(lib)
    assert ws(512, 128, 128, 136, 6, ph.LUT_F32, ph.STE_MIN_MARGIN | 0x400) == 0 and "flags" in _err(lib)
    # wide inputs and many tables: past 160 KB of gu slots plus inverse index
    # per item the item role is off and the wide scatter kernel reads the
    # {gu, r} records (the FUSED flag does not lift that limit); below it the
    # item role holds an 80 KB index
    assert ws(300, 20000, 64, 24, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 0
    assert ws(200, 50000, 64, 24, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 24 * 200 * 8
    assert ws(200, 50000, 64, 24, 6, ph.LUT_F32, ph.STE_MIN_MARGIN | fused) == 24 * 200 * 8
    assert ws(64, 64, 32, 3000, 6, ph.LUT_F32, ph.STE_MIN_MARGIN) == 3000 * 64 * 8
    assert ws(150, 50000, 48, 20, 5, ph.LUT_F32, ph.STE_FULL) == general(150, 48, 20, 32, 5, 64, True)


def _err(lib) -> str:
    return lib.tropnn_hip_last_error().decode()


def test_forward_rejects_bad_arguments(lib):
    fwd = lib.tropnn_hip_pairwise_forward
    # tables < 1
    assert fwd(4, 8, 5, 0, 3, 8, 8, 8, 8, 0, 1.0, 8, None, None, None, None, None) == 1
    assert "tables" in _err(lib)
    # comparisons above the supported maximum: unsupported, not invalid
    assert fwd(4, 8, 5, 3, 9, 8, 8, 8, 8, 0, 1.0, 8, None, None, None, None, None) == 2
    assert "comparisons" in _err(lib)
    # no in_features limit of its own: a 100,000-feature input is checked like
    # any other (here: its NULL latent)
    assert fwd(4, 100000, 5, 3, 3, None, 8, 8, 8, 0, 1.0, 8, None, None, None, None, None) == 1
    assert "non-NULL" in _err(lib)
    # unknown LUT dtype
    assert fwd(4, 8, 5, 3, 3, 8, 8, 8, 8, 7, 1.0, 8, None, None, None, None, None) == 1
    # NULL buffers
    assert fwd(4, 8, 5, 3, 3, None, 8, 8, 8, 0, 1.0, 8, None, None, None, None, None) == 1
    assert "non-NULL" in _err(lib)
    # empty batch is a no-op success
    assert fwd(0, 8, 5, 3, 3, None, None, None, None, 0, 1.0, None, None, None, None, None, None) == 0
    assert _err(lib) == ""


def test_forward_rejects_misaligned_debug_outputs(lib):
    fwd = lib.tropnn_hip_pairwise_forward
    # int64 indices at an odd address (never dereferenced: validation fails first)
    assert fwd(4, 8, 8, 3, 3, 16, 16, 16, 16, 0, 1.0, 16, None, 12, None, None, None) == 1
    assert "aligned" in _err(lib)


def test_route_rejects_bad_arguments(lib):
    route = lib.tropnn_hip_pairwise_route
    # items, in, tables, comps, latent, anchors, thresholds, codes, indices, margins, stream
    assert route(4, 8, 0, 3, 16, 16, 16, 16, None, None, None) == 1 and "tables" in _err(lib)
    assert route(4, 8, 3, 9, 16, 16, 16, 16, None, None, None) == 2 and "comparisons" in _err(lib)
    assert route(4, 8, 3, 3, None, 16, 16, 16, None, None, None) == 1 and "non-NULL" in _err(lib)
    assert route(4, 8, 3, 3, 16, 16, 16, None, 12, None, None) == 1 and "aligned" in _err(lib)
    # nothing asked for, or an empty batch: a no-op success without a launch
    assert route(4, 8, 3, 3, None, None, None, None, None, None, None) == 0 and _err(lib) == ""
    assert route(0, 8, 3, 3, None, None, None, 16, 16, 16, None) == 0 and _err(lib) == ""


def test_backward_rejects_bad_arguments(lib):
    bwd = lib.tropnn_hip_pairwise_backward
    # items, in, out, tables, comps, G, lut, dtype, record, margins, offsets,
    # entries, scale, ste_mode, surrogate, grad_x, grad_thr, grad_lut,
    # workspace, workspace_bytes, stream (pointers are never dereferenced:
    # every case fails validation before a launch)
    args = [4, 8, 5, 3, 3, 16, 16, 0, 16, None, 16, 16, 1.0, 0, 0, 16, 16, 16, 16, 1 << 20, None]
    bad_mode = list(args)
    bad_mode[13] = 2
    assert bwd(*bad_mode) == 1 and "ste_mode" in _err(lib)
    bad_surr = list(args)
    bad_surr[14] = 5
    assert bwd(*bad_surr) == 1 and "surrogate" in _err(lib)
    full_no_margins = list(args)
    full_no_margins[13] = 1
    assert bwd(*full_no_margins) == 1 and "margins" in _err(lib)
    no_index = list(args)
    no_index[10] = None
    assert bwd(*no_index) == 1 and "anchor index" in _err(lib)
    small_ws = list(args)
    small_ws[19] = 4
    assert bwd(*small_ws) == 1 and "workspace" in _err(lib)
    # the LUT gradient alone needs the workspace too (the general path sorts into it)
    lut_only = list(args)
    lut_only[15], lut_only[16], lut_only[18] = None, None, None
    assert bwd(*lut_only) == 1 and "workspace" in _err(lib)


def test_event_hook_rejects_bad_kernel(lib):
    assert lib.tropnn_hip_arm_kernel_events(8, None, None) == 1
    assert lib.tropnn_hip_arm_kernel_events(0, ctypes.c_void_p(8), None) == 1
    assert lib.tropnn_hip_arm_kernel_events(0, None, None) == 0


def test_adam_rejects_bad_arguments(lib):
    fn = lib.tropnn_hip_adam_step
    one = ctypes.c_void_p * 1
    good = one(256)
    numel = (ctypes.c_int64 * 1)(4)
    base = [1, good, good, good, good, numel, good, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0, None]
    assert fn(-1, *base[1:]) == 1
    assert fn(0, None, None, None, None, None, None, *base[7:]) == 0  # nothing to do, no launch
    for k in range(1, 7):
        args = list(base)
        args[k] = None
        assert fn(*args) == 1, k
    for k, bad in ((7, -1.0), (8, 1.0), (9, -0.1), (10, -1e-8), (11, -0.5)):
        args = list(base)
        args[k] = bad
        assert fn(*args) == 1 and "beta" in _err(lib), k
    args = list(base)
    args[6] = one(258)  # misaligned step counter
    assert fn(*args) == 1 and "steps[0]" in _err(lib)
    args = list(base)
    args[1] = one(258)  # misaligned parameter
    assert fn(*args) == 1 and "aligned" in _err(lib)
    args = list(base)
    args[2] = one(None)  # NULL gradient of a non-empty tensor
    assert fn(*args) == 1 and "NULL" in _err(lib)
    args = list(base)
    args[5] = (ctypes.c_int64 * 1)(-4)
    assert fn(*args) == 1 and "numels" in _err(lib)


def test_cross_entropy_rejects_bad_arguments(lib):
    fn = lib.tropnn_hip_cross_entropy
    base = [512, 10, 256, 256, -100, 256, 256, None]
    assert fn(0, *base[1:]) == 1 and "rows" in _err(lib)
    assert fn(512, 0, *base[2:]) == 1 and "classes" in _err(lib)
    for k in (2, 3, 5, 6):
        args = list(base)
        args[k] = None
        assert fn(*args) == 1 and "NULL" in _err(lib), k
    args = list(base)
    args[3] = 260  # int64 targets need 8-byte alignment
    assert fn(*args) == 1 and "align" in _err(lib)


def test_noalloc_backward_rejects_before_any_launch(lib):
    """The allocation-free backward refuses a shape whose workspace exceeds its
    TROPNN_NOALLOC_WORKSPACE_BYTES buffer (c4's layer needs ~1.2 GB) and bad
    enums, with the documented codes, before it looks up its device buffer."""
    m = re.search(r"#define TROPNN_NOALLOC_WORKSPACE_BYTES \((\d+)u << (\d+)\)", HEADER.read_text())
    assert m
    limit = int(m.group(1)) << int(m.group(2))
    dims = (8192, 1024, 4096, 512, 8)
    assert lib.tropnn_hip_pairwise_backward_workspace_size(*dims, ph.LUT_F16, ph.STE_MIN_MARGIN) > limit
    fake = 1 << 20
    rc = lib.tropnn_hip_pairwise_backward_noalloc(*dims, fake, fake, ph.LUT_F16, fake, None, fake, fake, 1.0,
                                                  ph.STE_MIN_MARGIN, 0, fake, fake, fake, None)
    assert rc == 2 and b"allocation-free" in lib.tropnn_hip_last_error()
    assert lib.tropnn_hip_pairwise_backward_noalloc(4, 8, 8, 2, 2, fake, fake, 0, fake, None, fake, fake, 1.0,
                                                    7, 0, fake, fake, fake, None) == 1
    assert lib.tropnn_hip_pairwise_backward_noalloc(4, 8, 8, 2, 99, fake, fake, 0, fake, None, fake, fake, 1.0,
                                                    0, 0, fake, fake, fake, None) == 2


def test_autograd_operator_loads_and_binds(lib):
    """The autograd operator library loads without a GPU, is bound to this
    library's entry points, refuses another ABI version, and rejects CPU
    tensors before any call into the library."""
    import torch

    if not ph.OPS_LIBRARY.exists():
        pytest.skip("libtropnn_hip_torch.so not built (run __graft_entry__.build())")
    op = ph._pairwise_op()
    args = [a.name for a in op._schema.arguments]
    assert args == ["latent", "anchors", "thresholds", "lut", "lut_read", "index_offsets", "index_entries",
                    "ste", "min_margin", "surrogate", "output_scale", "route_mode", "input_grad"]
    assert len(op._schema.returns) == 3
    addr = ctypes.cast(lib.tropnn_hip_pairwise_forward, ctypes.c_void_p).value
    with pytest.raises(RuntimeError, match="ABI version"):
        torch.ops.tropnn_hip.bind_abi(addr, addr, addr, addr, ph.ABI_VERSION + 1)
    x = torch.zeros(2, 1, 8)
    anchors = torch.zeros(3, 2, 2, dtype=torch.int64)
    with pytest.raises(ValueError, match="one GPU"):
        op(x, anchors, torch.zeros(3, 2), torch.zeros(3, 4, 5), torch.zeros(3, 4, 5), None, None,
           True, True, 0, 1.0, 0)
    with pytest.raises(ValueError, match="surrogate"):
        op(x, anchors, torch.zeros(3, 2), torch.zeros(3, 4, 5), torch.zeros(3, 4, 5), None, None,
           True, True, 7, 1.0, 0)
    with pytest.raises(ValueError, match="input-gradient"):
        op(x, anchors, torch.zeros(3, 2), torch.zeros(3, 4, 5), torch.zeros(3, 4, 5), None, None,
           True, True, 0, 1.0, 0, 3)
