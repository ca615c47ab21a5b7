"""Helpers of the GPU tests: build layers, run forwards, compare with the oracle."""
from __future__ import annotations

import numpy as np
import torch

import nomas_moe as nm
import oracle as O

NEAR_TIE = 1e-6  # logit gap below which a routing difference is reported, not failed
TOL = {"f32": 1e-4, "bf16": 2e-2, "f16": 2e-2}  # max|gpu - oracle| / max|oracle|


def to_device(x_f32: np.ndarray, dtype) -> torch.Tensor:
    raw = nm.to_model_dtype(x_f32, dtype)
    t = torch.from_numpy(raw.view(np.int16) if raw.dtype == np.uint16 else raw)
    return t.view(nm.DataType.of(dtype).torch).cuda()


def layer_from_tensors(t, dtype, dim, hidden, E, k, s=0.0, path="blocks.0.moe"):
    cfg = nm.MoeConfig(E, k, s, 0)
    return nm.MoeLayer.from_source(nm.Weights.from_tensors(t, dtype), path, dim, hidden, cfg)


def rel_err(got, ref) -> float:
    ref = np.asarray(ref, np.float64)
    den = float(np.max(np.abs(ref))) if ref.size else 0.0
    diff = float(np.max(np.abs(np.asarray(got, np.float64) - ref))) if ref.size else 0.0
    return diff / den if den > 0 else diff


def check_routing(layer, rows, o_idx, o_w, o_gap, E):
    """Indices bit-exact and counts exact except on near ties; gates to 1e-5 relative.

    The 16-bit router sums each 32-term block of exact products in f32 before
    the f64 accumulation, so a logit carries about 1e-7 of its own scale in
    rounding; gates follow logit differences, and with logits of scale ~16
    (router std 0.5 at dim 1024) that reaches a few 1e-6.
    """
    idx, w, counts, gap = layer.routing(rows)
    near = o_gap < NEAR_TIE
    assert np.array_equal(idx[~near], o_idx[~near]), (
        f"expert indices differ on {(idx[~near] != o_idx[~near]).any(axis=1).sum()} rows")
    want_counts = np.bincount(o_idx.ravel(), minlength=E)
    if near.any():
        assert np.abs(counts - want_counts).sum() <= 2 * int(near.sum()) * o_idx.shape[1]
    else:
        assert np.array_equal(counts, want_counts)
    np.testing.assert_allclose(w[~near], o_w[~near], rtol=1e-5, atol=1e-7)
    return near


def compare(layer, x_dev, x_oracle, p, k, dtype, rows=None, shared_dense=0.0, dense=None):
    """Run the layer and compare outputs (on `rows`, default all) and routing with the oracle."""
    y = layer.forward(x_dev)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().reshape(x_oracle.shape)
    n = x_oracle.shape[0]
    o_idx, o_w, _, o_gap = O.route(x_oracle, p["wr"], k)
    near = check_routing(layer, n, o_idx, o_w, o_gap, p["wr"].shape[0])
    sel = np.arange(n) if rows is None else np.asarray(rows)
    sel = sel[~near[sel]]
    ref, _, _, _ = O.forward_sparse(x_oracle, p, k, rows=sel, shared_dense=shared_dense,
                                    dense=dense)
    err = rel_err(got[sel], ref)
    print(f"  rel err {err:.3e} on {sel.size} rows, near ties {int(near.sum())}, "
          f"mfma={layer.uses_mfma}", flush=True)
    assert err <= TOL[dtype], f"relative error {err:.3e} above {TOL[dtype]}"
    assert np.isfinite(got).all()
    return got, err
