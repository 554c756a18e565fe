"""Writes the committed fixtures in tests/golden/ from the float64 oracle.

  dcn_c1.pt    BASELINE configs[0] (DCNv2 3x3, N=1, 64->64, 32x32, fp32 NCHW, seed 0):
               output [1, 64, 32, 32] (float32 of the float64 oracle) + input checksums
  msda_small.pt  a small 2-level MSDA problem (seed 11) with out-of-range samples:
               inputs + output (float64)

The reference repository ships no golden vectors for these operators, so the fixtures
freeze this repository's oracle (itself pinned by brute force and closed forms in
tests/test_oracle_*.py). Run: python tests/golden/make_golden.py
"""
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import dcn, inputs, msda  # noqa: E402


def checksum(t: torch.Tensor) -> float:
    return float(t.double().sum()) + float((t.double() ** 2).sum())


def main():
    d = inputs.dcn_inputs("dcn_c1")
    out = dcn.forward_nchw(d["x"].double(), d["offset"].double(), d["mask"].double(),
                           d["weight"].double(), d["bias"].double(), d["stride"], d["padding"],
                           d["dilation"])
    torch.save({
        "out": out.float(),
        "checksums": {k: checksum(d[k]) for k in ("x", "offset", "mask", "weight")},
    }, os.path.join(HERE, "dcn_c1.pt"))

    m = inputs.msda_random(2, [(6, 7), (3, 4)], 9, 2, 8, 3, seed=11, loc_lo=-0.3, loc_hi=1.3)
    m64 = {k: (v.double() if v.is_floating_point() else v) for k, v in m.items()}
    mo = msda.forward(**m64)
    torch.save(dict(m64, out=mo), os.path.join(HERE, "msda_small.pt"))
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
