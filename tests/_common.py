"""Shared helpers of the test suite: seeded cases, oracle comparison."""
from __future__ import annotations

import math

import numpy as np

import nomas_moe as nm
from nomas_moe import workloads as wl
import oracle as O

PATH = "blocks.0.moe"


def small_case(rows, dim, experts, top_k, hidden, seed, bias=True, dense=False,
               router_std=0.02, x_scale=1.0):
    """Seeded f32 parameters (checkpoint keys) and x for a small shape."""
    t = {}
    s = seed
    t[PATH + ".router.weight"] = nm.randn_affine(nm.path_seed(s, PATH + ".router"), experts * dim,
                                                 0.0, router_std).reshape(experts, dim)
    names = [f"{PATH}.experts.{e}" for e in range(experts)] + ([PATH + ".dense"] if dense else [])
    for base in names:
        for nmz, (o, i) in (("gate", (hidden, dim)), ("up", (hidden, dim)), ("down", (dim, hidden))):
            key = f"{base}.{nmz}"
            t[key + ".weight"] = nm.randn_affine(nm.path_seed(s, key), o * i, 0.0,
                                                 1.0 / math.sqrt(i)).reshape(o, i)
            t[key + ".bias"] = (nm.randn_affine(nm.path_seed(s, key + ".bias"), o, 0.0, 0.1)
                                if bias else np.zeros(o, np.float32))
    x = nm.randn_affine(nm.path_seed(s, "x"), rows * dim, 0.0, x_scale).reshape(rows, dim)
    return t, x


def rounded(t: dict, x: np.ndarray, dtype):
    """Round params and x to the model dtype; return (params f32-widened, x widened)."""
    rt = {k: nm.widen(nm.to_model_dtype(v, dtype), dtype) for k, v in t.items()}
    return rt, nm.widen(nm.to_model_dtype(x, dtype), dtype)


def rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| (the parity metric of the MoE outputs)."""
    ref = np.asarray(ref, np.float64)
    den = float(np.max(np.abs(ref))) if ref.size else 0.0
    if den == 0.0:
        return float(np.max(np.abs(np.asarray(got, np.float64)))) if ref.size else 0.0
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / den)


NEAR_TIE = 1e-6  # logit gap below which a routing difference is reported, not failed
