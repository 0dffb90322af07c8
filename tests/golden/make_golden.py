"""Write the seeded-init golden fixtures for PairwiseLinear.

The reference's constructor draws anchors and the LUT from the global torch RNG
(layers/pairwise.py:55-68). Closed forms and known-answer tests cannot pin that
draw sequence, so this script imports the reference once, in the build
container only, and records what it produced. Only data is committed:
`init_fixtures.npz` (anchors as int16, small LUTs in full) and
`init_fixtures.json` (SHA-256 of each LUT's f32 bytes plus sampled entries).

Usage (needs the reference checkout; never runs on the GPU box):
    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_golden.py /root/reference
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile
from pathlib import Path

import numpy as np

# (in_features, out_features, tables, comparisons, seed): the reference tests'
# small layers (test_backend_parity.py:223-224, 237-238) and every layer of the
# benchmark configurations c1..c5.
CASES = [
    (8, 5, 3, 3, 1),
    (8, 5, 4, 3, 2),
    (256, 512, 16, 6, 0),
    (128, 128, 136, 6, 0),
    (784, 128, 136, 6, 0),
    (128, 128, 136, 6, 1),
    (128, 10, 136, 6, 2),
    (1024, 4096, 512, 8, 0),
]
FULL_LUT_MAX = 4096  # LUTs up to this many elements are stored in full
SAMPLES = 16


def case_key(case: tuple[int, int, int, int, int]) -> str:
    i, o, t, c, s = case
    return f"i{i}_o{o}_t{t}_c{c}_s{s}"


def sample_positions(numel: int) -> list[int]:
    rng = np.random.default_rng(12345)
    picks = rng.integers(0, numel, size=SAMPLES - 2).tolist()
    return sorted(set([0, numel - 1] + picks))


def main() -> None:
    ref_root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference").resolve()
    out_dir = Path(__file__).resolve().parent
    sys.dont_write_bytecode = True
    with tempfile.TemporaryDirectory() as tmp:
        # The reference maps package `tropnn` onto its repo root (pyproject.toml:56-57).
        os.symlink(ref_root, Path(tmp) / "tropnn")
        sys.path.insert(0, tmp)
        import torch
        from tropnn import PairwiseLinear  # noqa: E402  (reference, build container only)

        arrays: dict[str, np.ndarray] = {}
        meta: dict[str, dict] = {}
        for case in CASES:
            i, o, t, c, s = case
            layer = PairwiseLinear(i, o, tables=t, comparisons=c, seed=s, backend="torch")
            key = case_key(case)
            anchors = layer.anchors.numpy()
            lut = layer.lut.detach().contiguous().numpy()
            assert anchors.max() < 32768
            arrays[f"{key}__anchors"] = anchors.astype(np.int16)
            flat = lut.reshape(-1)
            if flat.size <= FULL_LUT_MAX:
                arrays[f"{key}__lut"] = lut
            pos = sample_positions(flat.size)
            meta[key] = {
                "in_features": i,
                "out_features": o,
                "tables": t,
                "comparisons": c,
                "seed": s,
                "lut_shape": list(lut.shape),
                "lut_sha256": hashlib.sha256(flat.tobytes()).hexdigest(),
                "lut_sample_pos": pos,
                "lut_sample_val": [float(flat[p]) for p in pos],
                "thresholds_all_zero": bool((layer.thresholds.detach() == 0).all()),
                "powers": layer.powers.tolist(),
                "output_scale": float(layer.output_scale),
                # the global RNG state after construction: the next draw
                "next_randn": float(torch.randn(()).item()),
            }
            del layer, lut, flat
        np.savez_compressed(out_dir / "init_fixtures.npz", **arrays)
        (out_dir / "init_fixtures.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")
        print(f"wrote {len(CASES)} cases to {out_dir}")


if __name__ == "__main__":
    main()
