"""The wave-item forward kernel: batches of >= 2048 items giving >= 1024 waves,
LUT rows (or 1024-byte column tiles of them) of 128 to 1024 bytes, each wave
routing and gathering whole items. Against the CPU oracle: codes and margin
bits exact, outputs and training gradients within the north-star tolerance;
against the one-item kernel (the same items in calls below 2048 items, which
sum the same 16-table blocks): outputs bit-identical."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import routing_np
from test_gpu_parity import DEV, F16_TOL, F32_TOL, assert_train_parity, make_pair, rel_err, seeded, train_step

pytestmark = pytest.mark.gpu


def one_item_calls(hip, xd):
    """The same items through the one-item kernel: calls of 1024 items, the
    last one taking the remainder (every call below 2048 items)."""
    b = xd.shape[0]
    cuts = [1024 * k for k in range(max(1, b // 1024))] + [b]
    return torch.cat([hip(xd[lo:hi]) for lo, hi in zip(cuts[:-1], cuts[1:])])


@pytest.mark.parametrize(
    "lut_dtype,o,b",
    [
        ("f16", 128, 4100),  # c3's row: 256 bytes, 4 items per wave
        ("f32", 128, 2053),  # 512-byte rows, 2 items per wave
        ("f16", 256, 2100),
        ("f32", 64, 4111),
        ("f32", 512, 2050),  # two 1024-byte column tiles, 1 item per wave
        ("f16", 64, 8200),  # 128-byte rows, 8 items per wave
    ],
)
def test_wave_forward_against_oracle_and_one_item_kernel(lut_dtype, o, b):
    i, t, c = 128, 136, 6
    ref, hip = make_pair(i, o, t, c, seed=5, thr_std=0.3, lut_dtype=lut_dtype)
    x = seeded((b, i), seed=31)
    xd = x.to(DEV)
    hip.eval()
    with torch.no_grad():
        y = hip(xd)
        idx, mar = hip._last_indices.clone(), hip._last_margins.clone()
        y_one = one_item_calls(hip, xd)
        y_ref = ref.eval()(x)
    torch.cuda.synchronize()
    assert torch.equal(y, y_one)
    codes = routing_np.route_codes(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    margins = routing_np.margins_f32(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    np.testing.assert_array_equal(idx.cpu().reshape(b, t).numpy(), codes)
    np.testing.assert_array_equal(mar.cpu().reshape(b, t, c).numpy().view(np.uint32), margins.view(np.uint32))
    assert rel_err(y, y_ref) <= (F16_TOL if lut_dtype == "f16" else F32_TOL)


@pytest.mark.parametrize(
    "i,o,t,c,b,lut_dtype",
    [
        (33, 64, 20, 8, 4100, "f32"),  # input rows not a multiple of 4; blocks of 10 tables; 8 comparisons
        (40, 128, 3, 1, 4097, "f16"),  # one comparison, three tables
        (300, 128, 70, 7, 4099, "f16"),
    ],
)
def test_wave_forward_edge_shapes(i, o, t, c, b, lut_dtype):
    ref, hip = make_pair(i, o, t, c, seed=t + c, thr_std=0.4, lut_dtype=lut_dtype)
    x = seeded((b, i), seed=i + b)
    hip.eval()
    with torch.no_grad():
        y = hip(x.to(DEV))
        idx, mar = hip._last_indices, hip._last_margins
        y_ref = ref.eval()(x)
    codes = routing_np.route_codes(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    margins = routing_np.margins_f32(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    np.testing.assert_array_equal(idx.cpu().reshape(b, t).numpy(), codes)
    np.testing.assert_array_equal(mar.cpu().reshape(b, t, c).numpy().view(np.uint32), margins.view(np.uint32))
    assert rel_err(y, y_ref) <= (F16_TOL if lut_dtype == "f16" else F32_TOL)


def test_wave_forward_lazy_codes():
    """cache_route_debug='lazy': the wave kernel writes the uint8 codes only."""
    i, o, t, c, b = 128, 128, 136, 6, 4100
    ref, hip = make_pair(i, o, t, c, seed=9, thr_std=0.3, lut_dtype="f16")
    x = seeded((b, i), seed=7)
    hip.eval()
    hip.cache_route_debug = "lazy"
    with torch.no_grad():
        hip(x.to(DEV))
    expect = routing_np.route_codes(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    np.testing.assert_array_equal(hip._last_codes.cpu().reshape(b, t).numpy(), expect)


@pytest.mark.parametrize(
    "i,o,t,c,b,min_margin,surrogate",
    [
        (64, 32, 20, 5, 8200, True, "fast_sigmoid_odd"),  # 128-byte rows: 8 items per wave
        (48, 64, 17, 6, 4100, False, "izhikevich"),  # full STE (margins saved by the forward)
        (128, 128, 136, 6, 2053, True, "fast_sigmoid_odd"),  # c2's layer at 2053 items
    ],
)
def test_wave_forward_training(i, o, t, c, b, min_margin, surrogate):
    """Training steps whose forward is the wave kernel: the route records it
    writes drive the backward; every gradient against the oracle."""
    ref, hip = make_pair(i, o, t, c, seed=2, thr_std=0.4, use_min_margin_ste=min_margin, surrogate=surrogate)
    x = seeded((b, i), seed=13)
    g = seeded((b, 1, o), seed=14)
    yx_ref, yx_hip = train_step(ref, hip, x, g)
    assert_train_parity(ref, hip, yx_ref, yx_hip)


@pytest.mark.parametrize("lut_dtype,o,lut_off,out_off", [("f16", 64, 1, 1), ("f32", 128, 2, 2), ("f16", 128, 4, 0)])
def test_wave_shapes_with_lut_or_output_off_16_bytes(lut_dtype, o, lut_off, out_off):
    """A LUT or output that starts off a 16-byte boundary (views with a
    storage offset, aligned to the element vector the other kernels load)
    takes the multi-item kernel instead of the wave-item kernel, whose loads
    and stores move whole 16-byte pieces: the output equals the aligned
    call's bit for bit (both kernels sum the one-item kernel's 16-table
    blocks in order), and the aligned call is within the bar of the oracle."""
    from tropnn_amd.backends.pairwise_hip import _check, load_library

    i, t, c, b = 128, 136, 6, 8200
    ref, hip = make_pair(i, o, t, c, seed=4, thr_std=0.3, lut_dtype=lut_dtype)
    dt = torch.float16 if lut_dtype == "f16" else torch.float32
    x = seeded((b, i), seed=3)
    xd = x.to(DEV)
    lut = hip.lut.detach().to(dt).contiguous()
    anchors = hip.anchors.contiguous()
    thr = hip.thresholds.detach().contiguous()
    lib = load_library()
    fn = lib.tropnn_hip_lut_forward_batch_f16 if lut_dtype == "f16" else lib.tropnn_hip_lut_forward_batch_f32
    stream = torch.cuda.current_stream(DEV).cuda_stream

    def call(lut_view, out_view):
        rc = fn(b, t, c, i, o, lut_view.data_ptr(), anchors.data_ptr(), thr.data_ptr(), xd.data_ptr(),
                out_view.data_ptr(), 1.0, stream)
        _check(rc, fn.__name__)

    aligned = torch.full((b, o), float("nan"), device=DEV)
    call(lut, aligned)
    lbuf = torch.empty(lut.numel() + lut_off, dtype=dt, device=DEV)
    lut_v = lbuf[lut_off:].view(lut.shape)
    lut_v.copy_(lut)
    obuf = torch.full((b * o + out_off,), float("nan"), device=DEV)
    out_v = obuf[out_off:].view(b, o)
    assert (lut_v.data_ptr() % 16 != 0) or (out_v.data_ptr() % 16 != 0)
    call(lut_v, out_v)
    torch.cuda.synchronize()
    assert torch.equal(out_v, aligned)
    with torch.no_grad():
        y_ref = ref.eval()(x).reshape(b, o) / ref.output_scale
    assert rel_err(aligned, y_ref) <= (F16_TOL if lut_dtype == "f16" else F32_TOL)
