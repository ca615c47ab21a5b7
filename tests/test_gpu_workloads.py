"""The benchmark workloads at full size on the GPU.

Routing (expert indices and per-expert counts) is checked on every row
against the oracle's f64 routing.  Outputs are checked on rows chosen by
construction so that every (expert, 256-row tile) of the grouped GEMMs is
covered at six offsets (both wave halves, several 16-row MFMA blocks, the
last live row of short tail tiles); a checked row covers every column tile
of its row tiles, including tiles split along K (rows are independent, so
the oracle evaluates exactly those rows).  Two bars
against the f64 oracle, and a tight bar against the oracle with the GPU
path's storage roundings.  Size-independent properties: counts sum to
rows * k, every row finite, a second forward bitwise identical.  The one-segment
shape also runs as an f16 and an f32 model.
"""
import dataclasses

import numpy as np
import pytest
import torch

import nomas_moe as nm
from nomas_moe import workloads as wl
import oracle as O
from _gpu import TOL, check_routing, check_tight, rel_err, tile_rows, to_device

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["seg8b", "cfg8b", "fine64", "skewed16"])
def test_workload(name):
    check_workload(wl.WORKLOADS[name])


@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_one_segment_in_other_model_dtypes(dt):
    # The one-segment 8B shape (4,680 rows, dim 3072, 8 experts, top-2, hidden
    # 8192) for f16 and f32 models: their own router and MFMA GEMM
    # instantiations (16x16x32 f16 MFMAs; for f32, f64 router MFMAs and four
    # 16x16x4 f32 MFMAs per 16-byte fragment) at full size.
    check_workload(dataclasses.replace(wl.WORKLOADS["seg8b"], dtype=dt))


def check_workload(w):
    name = w.name
    print(f"workload {name}: rows={w.rows} D={w.dim} E={w.experts} k={w.top_k} H={w.hidden} "
          f"{w.dtype}", flush=True)
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
    g_idx, _, counts, _ = layer.routing(w.rows)
    assert counts.sum() == w.rows * w.top_k
    print(f"  counts {counts.tolist()}  near ties {int(near.sum())}", flush=True)
    rows, ntiles = tile_rows(g_idx, w.experts)
    rows = rows[~near[rows]]
    tight = check_tight(got[rows], rx, p, w.top_k, dt, rows)
    print(f"  {rows.size} rows covering {ntiles} expert tiles: vs rounded oracle "
          f"max {tight[0]:.3e} worst row rms {tight[1]:.3e}", flush=True)
    sub = rows[::4]  # the f64 forward on every fourth of them
    ref, _, _, _ = O.forward_sparse(rx, p, w.top_k, rows=sub)
    err = rel_err(got[sub], ref)
    print(f"  rel err vs f64 oracle {err:.3e} on {sub.size} rows", flush=True)
    assert err <= TOL[dt]
