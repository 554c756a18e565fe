"""CPU oracle for the bev-kernels hot paths (DCNv2 forward, MSDA forward).

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this directory; only
tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it, and only as the
checker (or the timed CPU baseline), never as a code path of the operators.

Modules:
  dcn     restatement of the reference's PyTorch goldens for DCNv2 (NCHW im2col and
          module forward, NHWC columns and forward), plus a scalar brute force.
  msda    restatement of the MSDA kernel semantics (direct loop over levels/points),
          the grid_sample closed form, and a scalar brute force.
  inputs  seeded generators of the BASELINE configurations.

Every function cites the reference file:line it follows. How each one is pinned (golden
vectors, closed forms, brute force, invariants) is listed in tests/test_oracle_*.py.
"""
