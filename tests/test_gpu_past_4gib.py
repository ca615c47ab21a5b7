"""Inputs past 4 GiB: the routed and K-blocked copies at 64-bit offsets.

x of 700,000 rows at dim 3072, bf16 (4.30 GB): the dispatch's K-blocked copy
of the routed rows (x_perm, 1.4M rows, 8.6 GB) and y_perm reach byte offsets
past 2^32, and so do the dense FFN's K-blocked copy of x and its output.  x is
drawn on the device; routing and outputs are checked against the oracle on 96
rows spread over the range, at both parity bars for the MoE.
"""
import math

import numpy as np
import pytest
import torch

import nomas_moe as nm
import oracle as O
from _common import small_case, rounded
from _gpu import NEAR_TIE, TOL, check_tight, layer_from_tensors, rel_err

pytestmark = pytest.mark.gpu

D, E, K, H = 3072, 8, 2, 256
ROWS = 700_000


def _device_x(rows, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(rows, D, device="cuda", generator=g, dtype=torch.bfloat16)


def test_moe_past_4_gib():
    print(f"moe past 4 GiB: rows={ROWS} x bytes={ROWS * D * 2}", flush=True)
    t, _ = small_case(8, D, E, K, H, 41)
    layer = layer_from_tensors(t, "bf16", D, H, E, K)
    rt, _ = rounded(t, np.zeros((1, D), np.float32), "bf16")
    p, _ = nm.workloads.oracle_params(rt, E)
    x = _device_x(ROWS, 7)
    y = layer.forward(x)
    torch.cuda.synchronize()
    sel = np.linspace(0, ROWS - 1, 96).astype(np.int64)
    sel_t = torch.from_numpy(sel).cuda()
    xs = x.index_select(0, sel_t).float().cpu().numpy()
    got = y.index_select(0, sel_t).float().cpu().numpy()
    del x, y
    idx, w, counts, _ = layer.routing(ROWS)
    assert counts.sum() == ROWS * K
    o_idx, o_w, _, o_gap = O.route(xs, p["wr"], K)
    ok = o_gap >= NEAR_TIE
    assert np.array_equal(idx[sel][ok], o_idx[ok])
    np.testing.assert_allclose(w[sel][ok], o_w[ok], rtol=1e-5, atol=1e-7)
    ref, _, _, _ = O.forward_sparse(xs, p, K, rows=np.nonzero(ok)[0])
    err = rel_err(got[ok], ref)
    tight = check_tight(got[ok], xs, p, K, "bf16", np.nonzero(ok)[0])
    print(f"  rel err {err:.3e} on {int(ok.sum())} rows; vs rounded oracle {tight[0]:.3e}",
          flush=True)
    assert err <= TOL["bf16"]


def test_ffn_past_4_gib():
    print(f"ffn past 4 GiB: rows={ROWS} x bytes={ROWS * D * 2}", flush=True)
    path = "blocks.0.mlp"
    t = {}
    for name, (o, i) in (("gate", (H, D)), ("up", (H, D)), ("down", (D, H))):
        key = f"{path}.{name}"
        t[key + ".weight"] = nm.randn_affine(nm.path_seed(43, key), o * i, 0.0,
                                             1.0 / math.sqrt(i)).reshape(o, i)
        t[key + ".bias"] = nm.randn_affine(nm.path_seed(43, key + ".bias"), o, 0.0, 0.1)
    ffn = nm.FeedForward.from_source(nm.Weights.from_tensors(t, "bf16"), path, D, H)
    x = _device_x(ROWS, 8)
    y = ffn.forward(x)
    torch.cuda.synchronize()
    sel = torch.from_numpy(np.linspace(0, ROWS - 1, 96).astype(np.int64)).cuda()
    xs = x.index_select(0, sel).float().cpu().numpy()
    got = y.index_select(0, sel).float().cpu().numpy()
    del x, y
    r = {k: nm.widen(nm.to_model_dtype(v, "bf16"), "bf16") for k, v in t.items()}
    f = {"wg": r[f"{path}.gate.weight"], "bg": r[f"{path}.gate.bias"],
         "wu": r[f"{path}.up.weight"], "bu": r[f"{path}.up.bias"],
         "wd": r[f"{path}.down.weight"], "bd": r[f"{path}.down.bias"]}
    err = rel_err(got, O.ffn(xs, f))
    print(f"  rel err {err:.3e} mfma={ffn.uses_mfma}", flush=True)
    assert ffn.uses_mfma
    assert err <= TOL["bf16"]
