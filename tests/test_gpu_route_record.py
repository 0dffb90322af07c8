"""The training forward's route record (include/tropnn_hip.h: one 8-byte
{u f32, code u16, r u8, 0} per (table, item), laid out [tables][items]),
read back from tropnn_hip_pairwise_forward through the C ABI and compared bit
for bit with the oracle's restatement of the reference's route
(oracle/routing_np.py: layers/pairwise.py:131-140): code = sum_c [m > 0] << c,
r = the first argmin_c |m| with a NaN |m| first (torch.argmin), u = m[r].
Every forward kernel that writes records is covered: the one-item kernel,
the multi-item and wave-item kernels of large batches, and the route kernel
before the streamed gather; with P = 1, 2, 4 and 8 lanes per table in the
ballot kernels (C = 1, 2, 3 .. 4, 5 .. 8), margins at ties, exact zeros,
signed zeros, subnormals, infinities and NaN."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from oracle import routing_np

# the module (the package re-exports the function of the same name)
ph = importlib.import_module("tropnn_amd.backends.pairwise_hip")

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    yield
    torch.cuda.synchronize()


def forward_record(x: np.ndarray, anchors: np.ndarray, thr: np.ndarray, o: int, lut_dtype: str = "f32",
                   debug: bool = False) -> np.ndarray:
    """Route record [T][B] as uint64 from the C ABI's training forward."""
    b, i = x.shape
    t, c = thr.shape
    lib = ph.load_library()
    gen = torch.Generator().manual_seed(7)
    lut = (0.02 * torch.randn(t, 1 << c, o, generator=gen)).to(torch.float16 if lut_dtype == "f16" else torch.float32)
    xd = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    ad = torch.from_numpy(np.ascontiguousarray(anchors)).to(DEV)
    td = torch.from_numpy(np.ascontiguousarray(thr)).to(DEV)
    ld = lut.to(DEV).contiguous()
    out = torch.empty(b, o, device=DEV)
    rec = torch.full((t, b), -1, dtype=torch.int64, device=DEV)  # every entry must be written
    idx = torch.empty(b, t, dtype=torch.int64, device=DEV) if debug else None
    codes = torch.empty(b, t, dtype=torch.uint8, device=DEV) if debug else None
    rc = lib.tropnn_hip_pairwise_forward(
        b, i, o, t, c, xd.data_ptr(), ad.data_ptr(), td.data_ptr(), ld.data_ptr(),
        ph.LUT_F16 if lut_dtype == "f16" else ph.LUT_F32, 1.0, out.data_ptr(), rec.data_ptr(),
        idx.data_ptr() if debug else None, None, codes.data_ptr() if debug else None,
        torch.cuda.current_stream(DEV).cuda_stream)
    assert rc == 0, lib.tropnn_hip_last_error()
    torch.cuda.synchronize()
    r = rec.cpu().numpy().view(np.uint64)
    if debug:
        expect = routing_np.route_codes(x, anchors, thr)
        np.testing.assert_array_equal(idx.cpu().numpy(), expect)
        np.testing.assert_array_equal(codes.cpu().numpy().astype(np.int64), expect)
    return r


def check_record(rec: np.ndarray, x: np.ndarray, anchors: np.ndarray, thr: np.ndarray) -> None:
    m = routing_np.margins_f32(x, anchors, thr)              # [B,T,C]
    code = routing_np.codes_from_margins(m).T                # [T,B]
    r = routing_np.min_margin_index(m).T                     # [T,B]
    u = np.take_along_axis(m, r.T[..., None], axis=-1)[..., 0].T.astype(np.float32)
    got_u = (rec & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    got_code = ((rec >> np.uint64(32)) & np.uint64(0xFFFF)).astype(np.int64)
    got_r = ((rec >> np.uint64(48)) & np.uint64(0xFF)).astype(np.int64)
    got_pad = (rec >> np.uint64(56)).astype(np.int64)
    np.testing.assert_array_equal(got_code, code)
    np.testing.assert_array_equal(got_r, r)
    # u bit for bit, except that a NaN the subtraction creates (inf - inf)
    # carries the platform's default payload (x86's has the sign bit set,
    # the GPU's not): NaN for NaN there
    nan = np.isnan(u)
    np.testing.assert_array_equal(np.isnan(got_u.view(np.float32)), nan)
    np.testing.assert_array_equal(got_u[~nan], u.view(np.uint32)[~nan])
    assert not got_pad.any()


def random_case(b, i, t, c, seed, sparse=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, i)).astype(np.float32)
    if sparse:  # c5-like: ~80 % exact zeros, so many margins are exactly -thr or 0
        x = (rng.random((b, i)) * (rng.random((b, i)) >= 0.8)).astype(np.float32)
    anchors = rng.integers(0, i, size=(t, c, 2)).astype(np.int64)
    thr = (0.3 * rng.standard_normal((t, c))).astype(np.float32)
    if sparse:
        thr[:, ::2] = 0.0
    return x, anchors, thr


@pytest.mark.parametrize(
    "b,i,o,t,c,lut_dtype,sparse,debug",
    [
        (512, 128, 128, 136, 6, "f32", False, False),   # c2: one-item kernel, 8 lanes per table
        (512, 128, 128, 136, 6, "f32", True, True),     # sparse (ties at |m| = 0), debug outputs too
        (37, 40, 10, 33, 3, "f32", True, False),        # 4 lanes per table
        (19, 16, 7, 5, 1, "f32", False, False),         # 1 lane per table
        (25, 20, 12, 9, 2, "f32", True, False),         # 2 lanes per table
        (40, 64, 64, 20, 8, "f32", True, False),        # 8 comparisons
        (2100, 32, 8, 20, 5, "f32", True, False),       # multi-item kernel (rows of 32 bytes)
        (4096, 128, 128, 136, 6, "f32", False, False),  # wave-item kernel (one lane per table)
        (2500, 48, 128, 12, 7, "f16", True, True),      # wave-item kernel, f16 rows, debug outputs
        (4096, 64, 1024, 64, 8, "f16", True, False),    # route kernel + streamed gather (LUT 32 MiB)
    ],
)
def test_route_record_matches_the_oracle(b, i, o, t, c, lut_dtype, sparse, debug):
    x, anchors, thr = random_case(b, i, t, c, seed=b + i + t + c, sparse=sparse)
    check_record(forward_record(x, anchors, thr, o, lut_dtype, debug), x, anchors, thr)


@pytest.mark.parametrize("b,o", [(2, 16), (2100, 8), (4096, 128)])  # one-item, multi-item, wave-item kernels
def test_route_record_edge_margins(b, o):
    """Margins at the edges of the argmin's order: NaN (first NaN wins),
    ±inf, exact ties (first index wins), ±0 (|+0| = |-0|), subnormals."""
    tiny = np.float32(1.4e-45)
    vals = np.array([0.0, -0.0, tiny, -tiny, 1.0, -1.0, np.inf, -np.inf, np.nan, 2.0, 2.0, -2.0], dtype=np.float32)
    rng = np.random.default_rng(11)
    i = len(vals)
    x = np.tile(vals, (b, 1))
    for row in range(1, b):  # every row a different arrangement of the same values
        x[row] = vals[rng.permutation(i)]
    t, c = 48, 4
    anchors = rng.integers(0, i, size=(t, c, 2)).astype(np.int64)
    anchors[0] = [[0, 1], [1, 0], [2, 3], [4, 5]]   # +0 - -0, -0 - +0: both +0, a tie at |m| = 0
    anchors[1] = [[8, 0], [0, 8], [6, 7], [7, 6]]   # NaN margins (the first wins), then inf - -inf
    anchors[2] = [[9, 10], [10, 9], [3, 3], [2, 2]]  # 2 - 2 = 0 four times over: the first index wins
    anchors[3] = [[6, 6], [7, 7], [4, 4], [8, 8]]   # inf - inf = NaN, -inf - -inf = NaN, 0, NaN
    thr = np.zeros((t, c), dtype=np.float32)
    thr[4:] = (0.5 * rng.standard_normal((t - 4, c))).astype(np.float32)
    check_record(forward_record(x, anchors, thr, o), x, anchors, thr)
