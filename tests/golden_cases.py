"""Seeded small cases shared by the golden fixtures and the GPU tests.

Each case is regenerated from seeds with the reference generator; parameters
come back f32 in the oracle's stacked layout, already rounded to the case's
model dtype (as a checkpoint cast with to_dtype would be, weights.rs:129-133).
"""
import math

import numpy as np

import nomas_moe as nm
from nomas_moe import workloads as wl

PATH = "blocks.0.moe"

# name: rows, dim, experts, top_k, hidden, dtype, seed, bias, shared_dense, router std
CASES = {
    # the tiny f32 workload exactly as the benchmark defines it (zero biases)
    "tiny_f32": dict(workload="tiny"),
    # the same shape with biases everywhere and the additive dense branch
    "tiny_f32_bias_dense": dict(rows=208, dim=64, E=4, k=2, H=128, dtype="f32", seed=0x5EED0100,
                                bias=True, shared_dense=0.5, router_std=0.3),
    # bf16, a shape the MFMA kernels tile (D % 256 == 0, H % 128 == 0)
    "bf16_mfma": dict(rows=64, dim=256, E=8, k=2, H=128, dtype="bf16", seed=0x5EED0101,
                      bias=True, shared_dense=0.0, router_std=0.1),
    # f16, general path (D and H not tiled by the MFMA kernels), k = 3
    "f16_general": dict(rows=50, dim=72, E=6, k=3, H=100, dtype="f16", seed=0x5EED0102,
                        bias=True, shared_dense=0.0, router_std=0.2),
    # k = E: every expert selected
    "f32_k_eq_e": dict(rows=33, dim=32, E=4, k=4, H=48, dtype="f32", seed=0x5EED0103,
                       bias=True, shared_dense=0.0, router_std=0.3),
}


def _lin(t, s, key, out_f, in_f, bias):
    t[key + ".weight"] = nm.randn_affine(nm.path_seed(s, key), out_f * in_f, 0.0,
                                         1.0 / math.sqrt(in_f)).reshape(out_f, in_f)
    t[key + ".bias"] = (nm.randn_affine(nm.path_seed(s, key + ".bias"), out_f, 0.0, 0.1) if bias
                        else np.zeros(out_f, np.float32))


def case_tensors(name):
    """(checkpoint-keyed f32 tensors before rounding, x f32, meta dict)."""
    c = CASES[name]
    if "workload" in c:
        w = wl.WORKLOADS[c["workload"]]
        meta = dict(rows=w.rows, dim=w.dim, E=w.experts, k=w.top_k, H=w.hidden, dtype=w.dtype,
                    shared_dense=0.0)
        return wl.make_params(w), wl.make_x(w), meta
    s, D, H, E = c["seed"], c["dim"], c["H"], c["E"]
    t = {PATH + ".router.weight": nm.randn_affine(nm.path_seed(s, PATH + ".router"), E * D, 0.0,
                                                  c["router_std"]).reshape(E, D)}
    for e in range(E):
        base = f"{PATH}.experts.{e}"
        _lin(t, s, base + ".gate", H, D, c["bias"])
        _lin(t, s, base + ".up", H, D, c["bias"])
        _lin(t, s, base + ".down", D, H, c["bias"])
    if c["shared_dense"] > 0:
        _lin(t, s, PATH + ".dense.gate", H, D, c["bias"])
        _lin(t, s, PATH + ".dense.up", H, D, c["bias"])
        _lin(t, s, PATH + ".dense.down", D, H, c["bias"])
    x = nm.randn_affine(nm.path_seed(s, "x"), c["rows"] * D).reshape(c["rows"], D)
    meta = dict(rows=c["rows"], dim=D, E=E, k=c["k"], H=H, dtype=c["dtype"],
                shared_dense=c["shared_dense"])
    return t, x, meta


def build_case(name):
    """Oracle view of a case: rounded f32 inputs in the stacked layout."""
    t, x, meta = case_tensors(name)
    dt = meta["dtype"]
    rt = {key: nm.widen(nm.to_model_dtype(v, dt), dt) for key, v in t.items()}
    rx = nm.widen(nm.to_model_dtype(x, dt), dt)
    p, dense = wl.oracle_params(rt, meta["E"])
    return dict(x=rx, p=p, dense=dense, k=meta["k"], E=meta["E"],
                shared_dense=meta["shared_dense"], meta=meta, tensors=t, x_raw=x)
