"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

The reference (hy-nomas-rs) holds no numeric golden vectors for its MoE path,
so these fixtures are the oracle's outputs on seeded inputs, committed so that
  * test_golden.py can detect any later change of the oracle, and
  * the GPU tests can compare the HIP path against fixed numbers.
Inputs are not stored: they are regenerated from their seeds by the reference
generator (SplitMix64 + Box-Muller, pinned by known answers).

    python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "hy-nomas-rs_amd"), os.path.join(ROOT, "oracle"),
                os.path.dirname(HERE)]

import oracle as O  # noqa: E402
from golden_cases import CASES, build_case  # noqa: E402


def generator_kat():
    seeds = [0, 1, 1234567, 0x5EED0002]
    paths = ["", "a", "x", "blocks.0.moe.router", "blocks.0.moe.experts.7.down",
             "blocks.11.moe.dense.gate"]
    return {
        "splitmix64": {str(s): [f"{v:016x}" for v in O.splitmix64(s, 8)] for s in seeds},
        "path_seed": {f"{s}:{p}": f"{O.path_seed(s, p):016x}" for s in (0, 0x5EED0002)
                      for p in paths},
        "randn_f32_bits": {str(s): [f"{v:08x}" for v in
                                    O.randn_affine(s, 17).view(np.uint32).tolist()]
                           for s in seeds},
    }


def main():
    with open(os.path.join(HERE, "generator_kat.json"), "w") as f:
        json.dump(generator_kat(), f, indent=1, sort_keys=True)
    for name in CASES:
        c = build_case(name)
        out, idx, w, gap = O.forward_sparse(c["x"], c["p"], c["k"],
                                            shared_dense=c["shared_dense"], dense=c["dense"])
        counts = np.bincount(idx.ravel(), minlength=c["E"]).astype(np.int32)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), out=out, idx=idx, w=w, gap=gap,
                            counts=counts)
        print(f"{name}: rows={c['x'].shape[0]} near-ties={(gap < 1e-6).sum()}")


if __name__ == "__main__":
    main()
