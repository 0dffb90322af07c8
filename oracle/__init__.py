"""CPU oracle for the PairwiseLinear hot path. TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
or call anything here; `tropnn_amd` never does, and its HIP path fails loudly
when the HIP library is missing instead of falling back to this code.

Modules:
  pairwise_torch  torch restatement of the reference's `backend="torch"` path
                  (init, route, chunked gather-sum, min-margin / full STE,
                  autograd backward) -- the parity oracle for forward and
                  gradients.
  routing_np      numpy restatement of the comparator route (integer codes,
                  bit-exact) and of the min-margin selection.
  lut_cpu         ctypes wrapper over `lut_cpu.c`, a C restatement of the
                  reference's Zig CPU forward (kernels/src/lut.zig), used as
                  the Zig-equivalent CPU baseline.

How each function is pinned (known-answer tests, golden init fixtures,
closed forms and finite differences) is listed in tests/test_oracle_*.py.
Every function here is pinned; none is marked "parity unpinned".
"""
