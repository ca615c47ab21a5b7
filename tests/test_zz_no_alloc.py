"""The no-allocation forward (nomas_moe_forward_noalloc) against nomas_moe_forward.

Both entry points run the same kernels; the no-allocation one lays every device
buffer out in the library's static scratch array instead of the handle's own
workspace.  The same input must give the same expert indices, counts, gates
and bit-identical outputs, on two calls in a row (the second smaller), across
layers on the MFMA and the general path sharing the one array, with a K-split
GEMM tail (its arrival counters live in the array and must be back at zero
after each call), and a row count beyond the array is a clear error.  One
4,744-row segment of the 8B preset (one guidance branch: 4,680 video + 64
text rows) fits.  Reading the routing back after another handle's
no-allocation forward has reused the array is a state error, not stale data.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import nomas_moe as nm
from nomas_moe import _lib
from nomas_moe import workloads as wl
import oracle as O
from _common import rounded, small_case
from _gpu import TOL, rel_err, to_device

pytestmark = pytest.mark.gpu

PATH = "blocks.0.moe"


def _layer(dim, E, k, hidden, dtype, seed):
    t, _ = small_case(8, dim, E, k, hidden, seed)
    layer = nm.MoeLayer.from_source(nm.Weights.from_tensors(t, dtype), PATH, dim, hidden,
                                    nm.MoeConfig(E, k))
    return layer, t


def _noalloc(layer, x, out):
    stream = torch.cuda.current_stream().cuda_stream
    rows = x.numel() // layer.dim
    rc = _lib.lib().nomas_moe_forward_noalloc(layer._h, x.data_ptr(), out.data_ptr(), rows, stream)
    return rc, _lib.last_error()


def _check_pair(layer, t, x_f32, dtype, label):
    rows = x_f32.shape[0]
    print(f"{label}: rows={rows} D={layer.dim} E={layer.experts} k={layer.top_k} "
          f"H={layer.hidden} {dtype} mfma={layer.uses_mfma}", flush=True)
    xd = to_device(x_f32, dtype)
    y_ref = layer.forward(xd)
    torch.cuda.synchronize()
    r_idx, r_w, r_counts, r_gap = layer.routing(rows)
    y = torch.full_like(y_ref, float("nan"))
    rc, msg = _noalloc(layer, xd, y)
    assert rc == 0, msg
    torch.cuda.synchronize()
    idx, w, counts, gap = layer.routing(rows)  # read back from the scratch array
    assert np.array_equal(idx, r_idx)
    assert np.array_equal(counts, r_counts)
    assert np.array_equal(w, r_w) and np.array_equal(gap, r_gap)
    assert torch.equal(y, y_ref), (
        f"max |diff| {float((y.float() - y_ref.float()).abs().max()):.3e}")
    # and both within the parity bar of the oracle
    rt, rx = rounded(t, x_f32, dtype)
    p, _ = wl.oracle_params(rt, layer.experts)
    o_idx, _, _, o_gap = O.route(rx, p["wr"], layer.top_k)
    ok = o_gap >= 1e-6
    assert np.array_equal(idx[ok], o_idx[ok])
    ref, _, _, _ = O.forward_sparse(rx, p, layer.top_k, rows=np.nonzero(ok)[0])
    err = rel_err(y.float().cpu().numpy()[ok], ref)
    print(f"  bit-identical to nomas_moe_forward; rel err vs oracle {err:.3e}", flush=True)
    assert err <= TOL[dtype]


def test_noalloc_matches_forward_on_two_calls_and_two_layers():
    mf, tm = _layer(1024, 8, 2, 1024, "bf16", 71)     # MFMA path, K-split tail at 1500 rows
    gen, tg = _layer(64, 4, 2, 96, "f32", 72)         # general path (dim not a multiple of 256)
    assert mf.uses_mfma and not gen.uses_mfma
    _, x1 = small_case(1500, 1024, 8, 2, 1024, 73)
    _, x2 = small_case(700, 1024, 8, 2, 1024, 74)
    _, xg = small_case(300, 64, 4, 2, 96, 75)
    _check_pair(mf, tm, x1, "bf16", "mfma call 1")
    _check_pair(mf, tm, x2, "bf16", "mfma call 2 (smaller)")
    _check_pair(gen, tg, xg, "f32", "general-path layer on the same array")
    _check_pair(mf, tm, x1, "bf16", "mfma again after the general-path layer")


def test_noalloc_rejects_rows_beyond_the_array():
    layer, _ = _layer(1024, 8, 2, 1024, "bf16", 76)
    rows = 60000  # about 800 MB of buffers at dim 1024, hidden 1024, top-2
    x = torch.zeros(rows, 1024, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros_like(x)
    rc, msg = _noalloc(layer, x, y)
    print(f"rows={rows}: rc={rc} {msg}", flush=True)
    assert rc == 2
    assert "no-allocation forward holds" in msg and "use nomas_moe_forward" in msg
    limit = int(msg.split("at most ")[1].split(" rows")[0])
    assert 0 < limit < rows
    # the largest size it names runs, and matches the allocating forward
    _, xl = small_case(limit, 1024, 8, 2, 1024, 77)
    xd = to_device(xl, "bf16")
    y_ref = layer.forward(xd)
    yl = torch.empty_like(y_ref)
    rc, msg = _noalloc(layer, xd, yl)
    assert rc == 0, msg
    torch.cuda.synchronize()
    assert torch.equal(yl, y_ref)
    print(f"  limit {limit} rows runs and matches", flush=True)
    rc, _ = _noalloc(layer, x[:0], y[:0])
    assert rc == 0


def test_noalloc_runs_one_8b_segment():
    # dim 3072, 8 experts, top-2, hidden 8192, bf16: the reference's
    # per-branch forward_segment call
    w = wl.WORKLOADS["seg8b"]
    rows = 4744
    print(f"8B segment: rows={rows} D={w.dim} E={w.experts} k={w.top_k} H={w.hidden}", flush=True)
    t = wl.make_params(w)
    layer = nm.MoeLayer.from_source(nm.Weights.from_tensors(t, w.dtype), wl.moe_path(), w.dim,
                                    w.hidden, nm.MoeConfig(w.experts, w.top_k))
    assert layer.uses_mfma
    x = nm.randn_affine(nm.path_seed(w.base_seed, "x"), rows * w.dim, 0.0, 1.0).reshape(rows, w.dim)
    xd = to_device(x, w.dtype)
    y_ref = layer.forward(xd)
    torch.cuda.synchronize()
    r_idx, r_w, r_counts, _ = layer.routing(rows)
    y = torch.full_like(y_ref, float("nan"))
    rc, msg = _noalloc(layer, xd, y)
    assert rc == 0, msg
    torch.cuda.synchronize()
    idx, wt, counts, _ = layer.routing(rows)
    assert np.array_equal(idx, r_idx) and np.array_equal(wt, r_w)
    assert np.array_equal(counts, r_counts) and counts.sum() == rows * w.top_k
    assert torch.equal(y, y_ref)
    # a sample of rows against the f64 oracle as well
    rt, rx = rounded(t, x, w.dtype)
    del t
    p, _ = wl.oracle_params(rt, w.experts)
    del rt
    o_idx, _, _, o_gap = O.route(rx, p["wr"], w.top_k)
    ok = o_gap >= 1e-6
    assert np.array_equal(idx[ok], o_idx[ok])
    sub = np.nonzero(ok)[0][::150]
    ref, _, _, _ = O.forward_sparse(rx, p, w.top_k, rows=sub)
    err = rel_err(y.float().cpu().numpy()[sub], ref)
    print(f"  bit-identical to nomas_moe_forward; rel err vs oracle {err:.3e} on {sub.size} rows",
          flush=True)
    assert err <= TOL[w.dtype]


def test_routing_after_another_noalloc_forward_is_a_state_error():
    a, _ = _layer(1024, 8, 2, 1024, "bf16", 81)
    b, _ = _layer(64, 4, 2, 96, "f32", 82)
    _, xa = small_case(300, 1024, 8, 2, 1024, 83)
    _, xb = small_case(200, 64, 4, 2, 96, 84)
    xda, xdb = to_device(xa, "bf16"), to_device(xb, "f32")
    ya, yb = torch.empty_like(xda), torch.empty_like(xdb)
    rc, msg = _noalloc(a, xda, ya)
    assert rc == 0, msg
    torch.cuda.synchronize()
    a.routing(300)  # its own array contents: readable
    rc, msg = _noalloc(b, xdb, yb)
    assert rc == 0, msg
    torch.cuda.synchronize()
    with pytest.raises(nm.NomasError) as ei:
        a.routing(300)  # the array now holds b's forward
    assert ei.value.code == 7 and "overwritten" in str(ei.value), str(ei.value)
    print(f"  stale routing refused: {ei.value}", flush=True)
    b.routing(200)
    a.forward(xda)  # an allocating forward: its own workspace again
    torch.cuda.synchronize()
    a.routing(300)
