"""GPU parity: the HIP MoE forward against the CPU oracle on identical seeded inputs.

Bars (tolerances written here, per the path's contract):
  * expert indices and per-expert counts bit-exact, except rows whose f64
    logit gap between the k-th and (k+1)-th expert is below 1e-6 (reported);
  * outputs: max|gpu - oracle| / max|oracle| <= 1e-4 for f32, <= 2e-2 for
    bf16 / f16, the oracle computing in f64 from the same rounded inputs.
"""
import numpy as np
import pytest
import torch

import nomas_moe as nm
import oracle as O
from _common import NEAR_TIE, PATH, rel_err, rounded, small_case

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "bf16": 2e-2, "f16": 2e-2}


def run_case(rows, dim, experts, top_k, hidden, dtype, seed, bias=True, dense_coef=0.0,
             check_rows=None, router_std=0.02):
    print(f"case rows={rows} D={dim} E={experts} k={top_k} H={hidden} {dtype} seed={seed} "
          f"dense={dense_coef}", flush=True)
    dense = dense_coef > 0
    t, x = small_case(rows, dim, experts, top_k, hidden, seed, bias=bias, dense=dense,
                      router_std=router_std)
    cfg = nm.MoeConfig(experts, top_k, dense_coef, 1)
    layer = nm.MoeLayer.from_source(nm.Weights.from_tensors(t, dtype), PATH, dim, hidden, cfg)
    rt, rx = rounded(t, x, dtype)
    xd = torch.from_numpy(nm.to_model_dtype(x, dtype).view(
        np.float32 if dtype == "f32" else np.int16)).view(nm.DataType.of(dtype).torch).cuda()
    y = layer.forward(xd)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    idx, w, counts, gap = layer.routing(rows)
    p, dn = nm.workloads.oracle_params(rt, experts)
    o_idx, o_w, o_logits, o_gap = O.route(rx, p["wr"], top_k)
    near = o_gap < NEAR_TIE
    assert np.array_equal(idx[~near], o_idx[~near]), "expert indices differ"
    if not near.any():
        assert np.array_equal(counts, np.bincount(o_idx.ravel(), minlength=experts))
    np.testing.assert_allclose(w[~near], o_w[~near], rtol=1e-5, atol=1e-6)
    sel = np.arange(rows) if check_rows is None else np.asarray(check_rows)
    sel = sel[~near[sel]]
    ref, _, _, _ = O.forward_sparse(rx, p, top_k, rows=sel, shared_dense=dense_coef, dense=dn)
    err = rel_err(got[sel], ref)
    print(f"  rel err {err:.3e}  near-ties {int(near.sum())}  mfma={layer.uses_mfma}", flush=True)
    assert err <= TOL[dtype], f"rel err {err} > {TOL[dtype]}"
    return layer, err


def test_moe_output_shape_and_finiteness():
    """moe.rs:123-150 on the GPU: random weights, dim 32, hidden 64, 4 experts, top-2."""
    cfg = nm.MoeConfig(experts=4, top_k=2, shared_dense=0.0, seed=1)
    moe = nm.MoeLayer.from_source(nm.Weights.random(4, nm.DataType.F32), PATH, 32, 64, cfg)
    x = torch.from_numpy(nm.randn_affine(3, 1 * 5 * 32).reshape(1, 5, 32)).cuda()
    y = moe.forward(x)
    assert tuple(y.shape) == (1, 5, 32)
    assert torch.isfinite(y).all()
    # and the same random weights through the oracle
    p = {"wr": O.xavier(4, 32, O.path_seed(4, PATH + ".router"))}
    for nmz, key, o, i in (("wg", "gate", 64, 32), ("wu", "up", 64, 32), ("wd", "down", 32, 64)):
        p[nmz] = np.stack([O.xavier(o, i, O.path_seed(4, f"{PATH}.experts.{e}.{key}"))
                           for e in range(4)])
    ref, _, _, _ = O.forward_sparse(x.cpu().numpy().reshape(5, 32), p, 2)
    assert rel_err(y.cpu().numpy().reshape(5, 32), ref) <= 1e-4


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_small_general_path(dtype):
    # D=72, H=100: not tiled by the MFMA kernels -> general path for every dtype
    layer, _ = run_case(150, 72, 6, 2, 100, dtype, seed=11)
    assert not layer.uses_mfma


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_small_mfma_path(dtype):
    layer, _ = run_case(300, 256, 8, 2, 128, dtype, seed=12)
    assert layer.uses_mfma


def test_mfma_multi_tile_ragged():
    # several row tiles per expert, ragged last tiles, multiple column tiles
    run_case(1000, 512, 4, 2, 384, "bf16", seed=13)


def test_tiny_workload_f32():
    from nomas_moe.workloads import WORKLOADS
    w = WORKLOADS["tiny"]
    run_case(w.rows, w.dim, w.experts, w.top_k, w.hidden, "f32", seed=w.base_seed, bias=False)
