"""The forward inside a captured HIP graph.

A forward launches only kernels on the caller's stream once its workspace
exists (the K-split arrival counters are put back to zero by the kernels that
use them; nothing is cleared with a memset), so a caller can capture it.  Each
graph here is replayed several times, with other forwards of the same layer
(other inputs, other row counts) and host synchronisations between the
replays, and every replay must equal the eager forward bit for bit.
"""
import numpy as np
import pytest
import torch

import nomas_moe as nm
from nomas_moe import _lib
from _common import small_case
from _gpu import to_device

pytestmark = pytest.mark.gpu

PATH = "blocks.0.moe"


def _layer(dim, E, k, hidden, dtype, seed):
    t, _ = small_case(8, dim, E, k, hidden, seed)
    return nm.MoeLayer.from_source(nm.Weights.from_tensors(t, dtype), PATH, dim, hidden,
                                   nm.MoeConfig(E, k))


def _inputs(rows, dim, dtype, seed):
    return to_device(nm.randn_affine(seed, rows * dim).reshape(rows, dim), dtype)


def _noalloc(layer, x, out):
    rows = x.numel() // layer.dim
    rc = _lib.lib().nomas_moe_forward_noalloc(layer._h, x.data_ptr(), out.data_ptr(), rows,
                                              torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.last_error()


@pytest.mark.parametrize("entry", ["forward", "forward_noalloc"])
@pytest.mark.parametrize("dim,E,k,hidden,dtype,rows", [
    (256, 8, 2, 256, "bf16", 1500),   # MFMA path
    (256, 8, 2, 128, "f32", 700),     # MFMA path, f32
    (192, 4, 2, 96, "bf16", 400),     # general grouped GEMM
])
def test_graph_replays_match_eager(entry, dim, E, k, hidden, dtype, rows):
    layer = _layer(dim, E, k, hidden, dtype, 90 + rows % 7)
    run = (lambda x, y: layer.forward(x, out=y)) if entry == "forward" else \
        (lambda x, y: _noalloc(layer, x, y))
    x = _inputs(rows, dim, dtype, 1)
    other = _inputs(rows // 2 + 3, dim, dtype, 2)
    y = torch.empty_like(x)
    y_other = torch.empty_like(other)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        run(x, y)             # the workspace exists before the capture
        run(other, y_other)
    torch.cuda.synchronize()
    eager = y.clone()
    eager_other = y_other.clone()

    g = torch.cuda.CUDAGraph()
    y.zero_()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        run(x, y)
    torch.cuda.synchronize()
    for rep in range(4):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {rep} differs from the eager forward"
        # the program's own eager work between replays: another forward of
        # the same layer on other rows, which reuses the same buffers
        with torch.cuda.stream(s):
            run(other, y_other)
        torch.cuda.synchronize()
        assert torch.equal(y_other, eager_other)


def test_graph_of_one_8b_segment_without_allocation():
    # The reference's per-branch call at the 8B preset: 4,744 rows (4,680 video
    # + 64 text), dim 3072, 8 experts, top-2, hidden 8192, bf16, captured
    # through the no-allocation entry point (its buffers in the library's
    # static array), replayed with eager forwards of other row counts between
    from nomas_moe import workloads as wl
    w = wl.WORKLOADS["seg8b"]
    rows = 4744
    print(f"8B segment graph: rows={rows} D={w.dim} E={w.experts} k={w.top_k} H={w.hidden}",
          flush=True)
    layer = nm.MoeLayer.from_source(nm.Weights.from_tensors(wl.make_params(w), w.dtype),
                                    wl.moe_path(), w.dim, w.hidden, nm.MoeConfig(w.experts, w.top_k))
    x = _inputs(rows, w.dim, w.dtype, 3)
    other = _inputs(1000, w.dim, w.dtype, 4)
    y, y_other = torch.empty_like(x), torch.empty_like(other)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        _noalloc(layer, x, y)  # the array's address is looked up before the capture
        layer.forward(other, out=y_other)
    torch.cuda.synchronize()
    eager, eager_other = y.clone(), y_other.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _noalloc(layer, x, y)
    torch.cuda.synchronize()
    for rep in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {rep} differs from the eager forward"
        with torch.cuda.stream(s):
            _noalloc(layer, other, y_other)  # the same array, another row count
        torch.cuda.synchronize()
        assert torch.equal(y_other, eager_other)
    print("  3 replays equal the eager forward bit for bit", flush=True)


def _replay_check(run, y, eager, other_run, y_other, eager_other, s, reps=3):
    g = torch.cuda.CUDAGraph()
    y.zero_()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        run()
    torch.cuda.synchronize()
    for rep in range(reps):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {rep} differs from the eager forward"
        with torch.cuda.stream(s):
            other_run()
        torch.cuda.synchronize()
        assert torch.equal(y_other, eager_other)


@pytest.mark.parametrize("dim,hidden,dtype,rows", [
    (256, 256, "bf16", 1500),   # MFMA path
    (192, 96, "f32", 300),      # general path
])
def test_graph_of_dense_ffn(dim, hidden, dtype, rows):
    # the dense feed-forward (mlp.rs:39-48): tile table, K-blocked copy of x
    # and the two GEMMs, captured once its workspace exists
    from test_gpu_ffn import PATH as FPATH, ffn_case
    t, _ = ffn_case(8, dim, hidden, 71)
    ffn = nm.FeedForward.from_source(nm.Weights.from_tensors(t, dtype), FPATH, dim, hidden)
    x, other = _inputs(rows, dim, dtype, 5), _inputs(rows // 3 + 1, dim, dtype, 6)
    y, y_other = torch.empty_like(x), torch.empty_like(other)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        ffn.forward(x, out=y)
        ffn.forward(other, out=y_other)
    torch.cuda.synchronize()
    eager, eager_other = y.clone(), y_other.clone()
    _replay_check(lambda: ffn.forward(x, out=y), y, eager,
                  lambda: ffn.forward(other, out=y_other), y_other, eager_other, s)


def test_graph_of_block_forward():
    # the FFN half of a DiT block (block.rs:96-101): norm2 + modulate, the
    # routed forward and the gated residual in the combine, captured
    B, S, D, E, k, H = 2, 300, 256, 8, 2, 384
    layer = _layer(D, E, k, H, "bf16", 77)
    rng = np.random.default_rng(9)
    x = to_device((rng.standard_normal((B * S, D)) * 1.7).astype(np.float32), "bf16").reshape(B, S, D)
    sh, sc, g, nw = (torch.from_numpy((rng.standard_normal(n) * 0.5).astype(np.float32)).cuda()
                     for n in ((B, D), (B, D), (B, D), (D,)))
    other = _inputs(500, D, "bf16", 7)
    y, y_other = torch.empty_like(x), torch.empty_like(other)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        layer.forward_block(x, sh, sc, g, nw, out=y)
        layer.forward(other, out=y_other)
    torch.cuda.synchronize()
    eager, eager_other = y.clone(), y_other.clone()
    _replay_check(lambda: layer.forward_block(x, sh, sc, g, nw, out=y), y, eager,
                  lambda: layer.forward(other, out=y_other), y_other, eager_other, s)
