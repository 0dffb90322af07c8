"""tropnn_hip_pairwise_backward_noalloc, the allocation-free backward, against
tropnn_hip_pairwise_backward with a caller workspace, through the C ABI.

Both run the same kernels in the same order, so their gradients are
bit-identical (torch.equal; the kernels are deterministic). Each case makes
two calls in a row, the second with fewer items, so the second call finds the
library's buffer holding the first call's contents. The outputs start as NaN,
so an element either entry point leaves unwritten shows.
"""
from __future__ import annotations

import importlib

import pytest
import torch

ph = importlib.import_module("tropnn_amd.backends.pairwise_hip")

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    yield
    torch.cuda.synchronize()


def _inputs(items, i, o, t, c, lut_dtype, full, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(items, 1, i, generator=gen).to(DEV)
    anchors = torch.randint(0, i, (t, c, 2), generator=gen).to(DEV)
    thr = (0.3 * torch.randn(t, c, generator=gen)).to(DEV)
    lut = (0.02 * torch.randn(t, 1 << c, o, generator=gen)).to(DEV)
    lut = lut.to(torch.float16) if lut_dtype == "f16" else lut
    g = torch.randn(items, o, generator=gen).to(DEV)
    _, rec, _, _, margins = ph._route_forward(
        x, anchors, thr, lut, output_scale=0.125, want_record=True, return_route=False, want_margins=full
    )
    offsets, entries = ph.anchor_index(anchors, i)
    return g, lut, rec, margins, offsets, entries


def _backward(noalloc, dims, g, lut, rec, margins, offsets, entries, ste_mode):
    items, i, o, t, c = dims
    lib = ph.load_library()
    lut_dtype = ph.LUT_F16 if lut.dtype == torch.float16 else ph.LUT_F32
    nan = float("nan")
    gx = torch.full((items, i), nan, device=DEV)
    gthr = torch.full((t, c), nan, device=DEV)
    glut = torch.full((t, 1 << c, o), nan, device=DEV)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    args = (items, i, o, t, c, g.data_ptr(), lut.data_ptr(), lut_dtype, rec.data_ptr(),
            None if margins is None else margins.data_ptr(), offsets.data_ptr(), entries.data_ptr(), 0.125,
            ste_mode, ph.SURROGATE_IDS["fast_sigmoid_odd"], gx.data_ptr(), gthr.data_ptr(), glut.data_ptr())
    if noalloc:
        rc = lib.tropnn_hip_pairwise_backward_noalloc(*args, stream)
    else:
        ws_bytes = lib.tropnn_hip_pairwise_backward_workspace_size(items, i, o, t, c, lut_dtype, ste_mode)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        rc = lib.tropnn_hip_pairwise_backward(*args, ws.data_ptr(), ws_bytes, stream)
    ph._check(rc, "noalloc" if noalloc else "backward")
    torch.cuda.synchronize()
    return gx, gthr, glut


@pytest.mark.parametrize(
    "i,o,t,c,lut_dtype,full,sizes,flag",
    [
        (128, 128, 136, 6, "f32", False, (512, 200), 0),  # c2's layer: fused table kernel + scatter
        (128, 128, 136, 6, "f32", False, (512, 200), ph.BWD_INPUT_GRAD_FUSED),  # item role, no workspace
        (128, 64, 40, 6, "f32", False, (300, 77), ph.BWD_INPUT_GRAD_SCATTER),  # narrow rows sent to the scatter
        (96, 300, 24, 6, "f16", False, (700, 257), 0),  # general path: sort, row, reduce, scatter
        (64, 48, 20, 5, "f32", True, (600, 130), 0),  # full STE: item, sort, row
    ],
)
def test_noalloc_backward_matches_workspace_backward(i, o, t, c, lut_dtype, full, sizes, flag):
    ste_mode = (ph.STE_FULL if full else ph.STE_MIN_MARGIN) | flag
    lib = ph.load_library()
    for call, items in enumerate(sizes):
        ws_bytes = lib.tropnn_hip_pairwise_backward_workspace_size(items, i, o, t, c, 0, ste_mode)
        assert ws_bytes <= 32 << 20  # 0 for the fused path whose item role forms grad_latent
        print(f"[noalloc] call {call}: items={items} i={i} o={o} t={t} c={c} {lut_dtype} full={full} flag={flag:#x}",
              flush=True)
        inputs = _inputs(items, i, o, t, c, lut_dtype, full, seed=17 * call + items)
        dims = (items, i, o, t, c)
        ref = _backward(False, dims, *inputs, ste_mode)
        got = _backward(True, dims, *inputs, ste_mode)
        for name, a, b in zip(("grad_latent", "grad_thresholds", "grad_lut"), got, ref):
            assert not torch.isnan(b).any(), f"call {call}: {name} of the workspace entry point has unwritten elements"
            assert torch.equal(a, b), f"call {call}: {name} differs, max {float((a - b).abs().max()):.3e}"


def test_noalloc_rejects_a_workspace_over_its_buffer():
    lib = ph.load_library()
    dims = (8192, 1024, 4096, 512, 8)  # c4's layer: ~1.2 GB of workspace
    need = lib.tropnn_hip_pairwise_backward_workspace_size(*dims, ph.LUT_F16, ph.STE_MIN_MARGIN)
    assert need > 32 << 20
    rc = lib.tropnn_hip_pairwise_backward_noalloc(*dims, None, None, ph.LUT_F16, None, None, None, None, 1.0,
                                                  ph.STE_MIN_MARGIN, 0, None, None, None,
                                                  torch.cuda.current_stream(DEV).cuda_stream)
    assert rc == 2
    assert b"allocation-free" in lib.tropnn_hip_last_error()


def _noalloc_args(dims, g, lut, rec, margins, offsets, entries, ste_mode, outs):
    items, i, o, t, c = dims
    lut_dtype = ph.LUT_F16 if lut.dtype == torch.float16 else ph.LUT_F32
    gx, gthr, glut = outs
    return (items, i, o, t, c, g.data_ptr(), lut.data_ptr(), lut_dtype, rec.data_ptr(),
            None if margins is None else margins.data_ptr(), offsets.data_ptr(), entries.data_ptr(), 0.125,
            ste_mode, ph.SURROGATE_IDS["fast_sigmoid_odd"], gx.data_ptr(), gthr.data_ptr(), glut.data_ptr())


def test_noalloc_backward_replayed_from_a_graph():
    """The allocation-free backward captured in a HIP graph (after one call
    on the device outside capture) and replayed three times, with eager work
    and synchronisation between the replays: before each replay the upstream
    gradient is rewritten in place and the outputs are filled with NaN; each
    replay must equal the workspace entry point run eagerly on the same
    inputs, bit for bit."""
    i, o, t, c, items = 128, 128, 136, 6, 512
    dims = (items, i, o, t, c)
    g, lut, rec, margins, offsets, entries = _inputs(items, i, o, t, c, "f32", False, seed=5)
    lib = ph.load_library()
    _backward(True, dims, g, lut, rec, margins, offsets, entries, ph.STE_MIN_MARGIN)  # outside capture first
    outs = tuple(torch.empty(s, device=DEV) for s in ((items, i), (t, c), (t, 1 << c, o)))
    args = _noalloc_args(dims, g, lut, rec, margins, offsets, entries, ph.STE_MIN_MARGIN, outs)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.tropnn_hip_pairwise_backward_noalloc(*args, torch.cuda.current_stream(DEV).cuda_stream)
    ph._check(rc, "noalloc under capture")
    gen = torch.Generator().manual_seed(9)
    for replay in range(3):
        g.copy_(torch.randn(g.shape, generator=gen).to(DEV))
        for out in outs:
            out.fill_(float("nan"))
        torch.cuda.synchronize()
        print(f"[noalloc graph] replay {replay}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        ref = _backward(False, dims, g, lut, rec, margins, offsets, entries, ph.STE_MIN_MARGIN)
        for name, a, b in zip(("grad_latent", "grad_thresholds", "grad_lut"), outs, ref):
            assert torch.equal(a, b), f"replay {replay}: {name} differs, max {float((a - b).abs().max()):.3e}"


_FIRST_CALL_UNDER_CAPTURE = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch
import tests.test_zz_no_alloc as t
ph = t.ph
items, i, o, k, c = 64, 32, 16, 8, 4
inputs = t._inputs(items, i, o, k, c, "f32", False, seed=1)
outs = tuple(torch.empty(s, device=t.DEV) for s in ((items, i), (k, c), (k, 1 << c, o)))
args = t._noalloc_args((items, i, o, k, c), *inputs, ph.STE_MIN_MARGIN, outs)
lib = ph.load_library()
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = lib.tropnn_hip_pairwise_backward_noalloc(*args, torch.cuda.current_stream(t.DEV).cuda_stream)
    msg = lib.tropnn_hip_last_error()
assert rc == 2, rc
assert b"under stream capture" in msg, msg
rc = lib.tropnn_hip_pairwise_backward_noalloc(*args, torch.cuda.current_stream(t.DEV).cuda_stream)
assert rc == 0, lib.tropnn_hip_last_error()
torch.cuda.synchronize()
print("first call under capture refused; the next call outside capture ran")
"""


def test_noalloc_first_call_under_capture_is_refused():
    """In a fresh process the first allocation-free backward on the device,
    made under stream capture, fails with TROPNN_ERR_UNSUPPORTED and a clear
    message before enqueuing anything (its buffer's address lookup is not
    stream work); a later call outside capture runs."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    proc = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, str(root)], capture_output=True,
                          text=True, timeout=240, cwd=str(root))
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-2000:]
    assert "refused" in proc.stdout
