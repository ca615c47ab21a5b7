"""The benchmark workloads at full size on the GPU.

Routing (expert indices and per-expert counts) is checked on every row
against the oracle's f64 routing; outputs on a seeded sample of rows (the
oracle's sparse f64 forward is exact per row, rows are independent), plus
size-independent properties: counts sum to rows * k, every row finite, and a
second forward is bitwise identical.
"""
import numpy as np
import pytest
import torch

import nomas_moe as nm
from nomas_moe import workloads as wl
import oracle as O
from _gpu import check_routing, rel_err, to_device, TOL

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["seg8b", "cfg8b", "fine64", "skewed16"])
def test_workload(name):
    w = wl.WORKLOADS[name]
    print(f"workload {name}: rows={w.rows} D={w.dim} E={w.experts} k={w.top_k} H={w.hidden}",
          flush=True)
    t = wl.make_params(w)
    x = wl.make_x(w)
    dt = w.dtype
    layer = nm.MoeLayer.from_source(nm.Weights.from_tensors(t, dt), wl.moe_path(), w.dim,
                                    w.hidden, nm.MoeConfig(w.experts, w.top_k))
    assert layer.uses_mfma
    xd = to_device(x, dt)
    y1 = layer.forward(xd)
    y2 = layer.forward(xd)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    got = y1.float().cpu().numpy()
    assert np.isfinite(got).all()
    del y1, y2, xd
    # oracle inputs: the same values rounded to the model dtype
    rx = nm.widen(nm.to_model_dtype(x, dt), dt)
    rt = {k: nm.widen(nm.to_model_dtype(v, dt), dt) for k, v in t.items()}
    del t
    p, _ = wl.oracle_params(rt, w.experts)
    del rt
    o_idx, o_w, _, o_gap = O.route(rx, p["wr"], w.top_k)
    near = check_routing(layer, w.rows, o_idx, o_w, o_gap, w.experts)
    _, _, counts, _ = layer.routing(w.rows)
    assert counts.sum() == w.rows * w.top_k
    print(f"  counts {counts.tolist()}  near ties {int(near.sum())}", flush=True)
    rng = np.random.default_rng(w.base_seed)
    sample = np.unique(np.concatenate([[0, w.rows - 1], rng.choice(w.rows, 46, replace=False)]))
    sample = sample[~near[sample]]
    ref, _, _, _ = O.forward_sparse(rx, p, w.top_k, rows=sample)
    err = rel_err(got[sample], ref)
    print(f"  rel err {err:.3e} on {sample.size} sampled rows", flush=True)
    assert err <= TOL[dt]
