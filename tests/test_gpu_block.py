"""GPU parity of the DiT block seams around the FFN (block.rs:96-101).

  * norm2 + modulate (nomas_norm_modulate): h bit-exact against the oracle's
    orc_norm_modulate with correctly rounded square and root (pow_mode 1), which
    agrees with the reference's libm powf form (pow_mode 0) on every row here;
  * the gated residual (nomas_gated_residual): bit-exact;
  * MoeLayer.forward_block: routing of h bit-exact except near ties, out within
    the output tolerance of the oracle's block (f64 MoE, model-dtype seams), and
    bit-identical to norm_modulate -> forward -> gated_residual run separately.
"""
import numpy as np
import pytest
import torch

import nomas_moe as nm
import oracle as O
from _common import rounded, small_case
from _gpu import TOL, check_routing, layer_from_tensors, rel_err, to_device

pytestmark = pytest.mark.gpu


def seam_inputs(B, S, D, seed, dtype, affine=True, x_scale=1.7):
    """x (B*S, D) f32 plus f32 AdaLN parameters and norm gain, seeded."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((B * S, D)) * x_scale).astype(np.float32)
    sh = (rng.standard_normal((B, D)) * 0.5).astype(np.float32)
    sc = (rng.standard_normal((B, D)) * 0.5).astype(np.float32)
    g = (rng.standard_normal((B, D)) * 0.5).astype(np.float32)
    # norm2's random init is N(0, 1) (param_from_source with std 1, mod.rs:156-176)
    nw = rng.standard_normal(D).astype(np.float32) if affine else None
    return x, sh, sc, g, nw


def dev(a):
    return None if a is None else torch.from_numpy(a).cuda()


def bits(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy().view(np.int32)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("B,S,D,affine", [
    (2, 150, 256, True),    # last block partial; a block spanning two sequences
    (3, 7, 264, True),      # D not a multiple of 128; many sequences per block
    (1, 64, 3072, False),   # the 8B preset's width, no affine gain
    (1, 70, 6144, True),    # factors too wide for LDS: read from global memory
])
def test_norm_modulate_bitexact(dtype, B, S, D, affine):
    print(f"norm_modulate B={B} S={S} D={D} {dtype} affine={affine}", flush=True)
    x, sh, sc, _, nw = seam_inputs(B, S, D, 100 + D + S, dtype, affine)
    xd = to_device(x, dtype).reshape(B, S, D)
    h = nm.norm_modulate(xd, dev(sh), dev(sc), dev(nw), eps=1e-6)
    torch.cuda.synchronize()
    xm = O.round_dt(x, dtype)
    want1, inv1 = O.norm_modulate(xm, sh, sc, S, nw, 1e-6, dtype, pow_mode=1)
    got = h.reshape(B * S, D).float().cpu().numpy()
    assert np.array_equal(got.view(np.int32), want1.view(np.int32)), (
        f"{int((got != want1).sum())} elements differ")
    want0, inv0 = O.norm_modulate(xm, sh, sc, S, nw, 1e-6, dtype, pow_mode=0)
    same = inv0 == inv1
    print(f"  rows where powf and the rounded root agree: {int(same.sum())}/{same.size}",
          flush=True)
    assert np.array_equal(got[same].view(np.int32), want0[same].view(np.int32))


def test_norm_modulate_edge_rows_and_in_place():
    # a zero row (inv = eps^-1/2), a row of huge values (squares overflow f32
    # in the sum: inv = 0, h = shift), tiny values, then in place (h is x)
    B, S, D = 1, 70, 512
    x, sh, sc, _, nw = seam_inputs(B, S, D, 7, "bf16")
    x[0] = 0.0
    x[1] = 3e38
    x[2] *= 1e-20
    xd = to_device(x, "bf16").reshape(B, S, D)
    h = nm.norm_modulate(xd, dev(sh), dev(sc), dev(nw))
    want, _ = O.norm_modulate(O.round_dt(x, "bf16"), sh, sc, S, nw, 1e-6, "bf16", pow_mode=1)
    assert np.array_equal(bits(h).reshape(B * S, D), want.view(np.int32))
    nm.norm_modulate(xd, dev(sh), dev(sc), dev(nw), out=xd)
    assert torch.equal(xd, h)


def test_norm_modulate_zero_rows_and_errors():
    x = torch.empty((1, 0, 256), dtype=torch.bfloat16, device="cuda")
    z = torch.zeros((1, 256), device="cuda")
    assert nm.norm_modulate(x, z, z).shape == (1, 0, 256)
    L = nm._lib.lib()
    xd = torch.zeros((10, 256), dtype=torch.bfloat16, device="cuda")
    # rows not a whole number of sequences, a width that is not a multiple of 8
    assert L.nomas_norm_modulate(1, xd.data_ptr(), xd.data_ptr(), 10, 256, 3, None, 1e-6,
                                 z.data_ptr(), z.data_ptr(), None) == 2
    assert L.nomas_norm_modulate(1, xd.data_ptr(), xd.data_ptr(), 10, 252, 10, None, 1e-6,
                                 z.data_ptr(), z.data_ptr(), None) == 2
    assert L.nomas_gated_residual(1, xd.data_ptr(), xd.data_ptr(), None, xd.data_ptr(), 10, 256,
                                  10, None) == 2
    assert b"gate" in L.nomas_moe_last_error()


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_gated_residual_bitexact(dtype):
    B, S, D = 3, 41, 200
    rng = np.random.default_rng(5)
    x = O.round_dt(rng.standard_normal((B * S, D)).astype(np.float32), dtype)
    y = O.round_dt(rng.standard_normal((B * S, D)).astype(np.float32), dtype)
    g = rng.standard_normal((B, D)).astype(np.float32)
    xd, yd = to_device(x, dtype).reshape(B, S, D), to_device(y, dtype).reshape(B, S, D)
    out = nm.gated_residual(xd, yd, dev(g))
    want = O.gated_residual(x, y, g, S, dtype)
    assert np.array_equal(bits(out).reshape(B * S, D), want.view(np.int32))
    nm.gated_residual(xd, yd, dev(g), out=yd)  # in place over y
    assert torch.equal(yd, out)


def block_case(B, S, D, E, k, H, dtype, seed, s=0.0, affine=True):
    t, _ = small_case(B * S, D, E, k, H, seed, dense=s > 0)
    x, sh, sc, g, nw = seam_inputs(B, S, D, seed, dtype, affine)
    layer = layer_from_tensors(t, dtype, D, H, E, k, s)
    rt, xm = rounded(t, x, dtype)
    p, dn = nm.workloads.oracle_params(rt, E)
    return layer, x, xm, sh, sc, g, nw, p, dn


@pytest.mark.parametrize("dtype,H", [("bf16", 384), ("f16", 384), ("f32", 200)])
def test_forward_block(dtype, H):
    B, S, D, E, k = 2, 300, 256, 8, 2
    print(f"forward_block B={B} S={S} D={D} E={E} k={k} H={H} {dtype}", flush=True)
    layer, x, xm, sh, sc, g, nw, p, _ = block_case(B, S, D, E, k, H, dtype, seed=61)
    xd = to_device(x, dtype).reshape(B, S, D)
    out = layer.forward_block(xd, dev(sh), dev(sc), dev(g), dev(nw))
    torch.cuda.synchronize()
    # routing is h's: h bit-exact with pow_mode 1
    h1, _ = O.norm_modulate(xm, sh, sc, S, nw, 1e-6, dtype, pow_mode=1)
    o_idx, o_w, _, o_gap = O.route(h1, p["wr"], k)
    near = check_routing(layer, B * S, o_idx, o_w, o_gap, E)
    # the block's output against the reference's arithmetic (pow_mode 0)
    ref, _, _, _ = O.block_ffn(xm, p, k, sh, sc, g, S, nw, 1e-6, dtype, pow_mode=0)
    got = out.reshape(B * S, D).float().cpu().numpy()
    err = rel_err(got[~near], ref[~near])
    print(f"  rel err {err:.3e}, near ties {int(near.sum())}, mfma={layer.uses_mfma}", flush=True)
    assert np.isfinite(got).all() and err <= TOL[dtype]
    # the same kernels run one by one give the same bits
    h = nm.norm_modulate(xd, dev(sh), dev(sc), dev(nw))
    y = layer.forward(h)
    assert torch.equal(nm.gated_residual(xd, y, dev(g)), out)


def test_forward_block_shared_dense_and_in_place():
    B, S, D, E, k, H = 3, 100, 256, 4, 1, 256
    layer, x, xm, sh, sc, g, nw, p, dn = block_case(B, S, D, E, k, H, "bf16", seed=62, s=0.5,
                                                     affine=False)
    xd = to_device(x, "bf16").reshape(B, S, D)
    out = layer.forward_block(xd, dev(sh), dev(sc), dev(g), None)
    ref, _, idx, gap = O.block_ffn(xm, p, k, sh, sc, g, S, None, 1e-6, "bf16", pow_mode=0,
                                   shared_dense=0.5, dense=dn)
    near = gap < 1e-6
    got = out.reshape(B * S, D).float().cpu().numpy()
    assert rel_err(got[~near], ref[~near]) <= TOL["bf16"]
    x2 = xd.clone()
    layer.forward_block(x2, dev(sh), dev(sc), dev(g), None, out=x2)  # in place
    assert torch.equal(x2, out)


def test_forward_block_headline_shape_properties():
    # three sequences of 4744 rows (the 8B preset's 4680 video + 64 text tokens
    # per guidance branch), dim 3072, E8 top-2: gate 0 returns x exactly, and
    # the block equals the composed kernels bit for bit
    B, S, D, E, k, H = 3, 4744, 3072, 8, 2, 1024
    layer, x, xm, sh, sc, g, nw, p, _ = block_case(B, S, D, E, k, H, "bf16", seed=63)
    xd = to_device(x, "bf16").reshape(B, S, D)
    zero = torch.zeros((B, D), device="cuda")
    assert torch.equal(layer.forward_block(xd, dev(sh), dev(sc), zero, dev(nw)), xd)
    out = layer.forward_block(xd, dev(sh), dev(sc), dev(g), dev(nw))
    h = nm.norm_modulate(xd, dev(sh), dev(sc), dev(nw))
    assert torch.equal(nm.gated_residual(xd, layer.forward(h), dev(g)), out)
    want, _ = O.norm_modulate(xm, sh, sc, S, nw, 1e-6, "bf16", pow_mode=1)
    assert np.array_equal(bits(h).reshape(B * S, D), want.view(np.int32))


def test_dense_ffn_block_composition():
    # BlockFfn::Dense: h -> FeedForward -> gated residual (block.rs:96-101)
    B, S, D, H = 2, 130, 256, 256
    t, _ = small_case(B * S, D, 1, 1, H, 64)
    f = {k.replace("blocks.0.moe.experts.0", "blocks.0.mlp"): v for k, v in t.items()
         if ".experts.0." in k}
    ffn = nm.FeedForward.from_source(nm.Weights.from_tensors(f, "bf16"), "blocks.0.mlp", D, H)
    x, sh, sc, g, nw = seam_inputs(B, S, D, 64, "bf16")
    xd = to_device(x, "bf16").reshape(B, S, D)
    h = nm.norm_modulate(xd, dev(sh), dev(sc), dev(nw))
    out = nm.gated_residual(xd, ffn.forward(h), dev(g))
    xm = O.round_dt(x, "bf16")
    h0, _ = O.norm_modulate(xm, sh, sc, S, nw, 1e-6, "bf16", pow_mode=0)
    r = {k: nm.widen(nm.to_model_dtype(v, "bf16"), "bf16") for k, v in f.items()}
    ff = {"wg": r["blocks.0.mlp.gate.weight"], "bg": r["blocks.0.mlp.gate.bias"],
          "wu": r["blocks.0.mlp.up.weight"], "bu": r["blocks.0.mlp.up.bias"],
          "wd": r["blocks.0.mlp.down.weight"], "bd": r["blocks.0.mlp.down.bias"]}
    y = O.round_dt(O.ffn(h0, ff).astype(np.float32), "bf16")
    ref = O.gated_residual(xm, y, g, S, "bf16")
    assert rel_err(out.reshape(B * S, D).float().cpu().numpy(), ref) <= TOL["bf16"]


def test_block_and_plain_forwards_interleaved_with_regrowth():
    # plain forward (small), fused block (larger: the workspace regrows and adds
    # room for h), plain again (smaller), block again: each call against its
    # own reference; the handle keeps working across layouts
    B, D, E, k, H, dtype = 2, 256, 8, 2, 128, "bf16"
    layer, x, xm, sh, sc, g, nw, p, _ = block_case(B, 400, D, E, k, H, dtype, seed=66)
    xd = to_device(x, dtype)
    for S, mode in ((50, "plain"), (400, "block"), (20, "plain"), (300, "block")):
        print(f"interleaved {mode} S={S}", flush=True)
        if mode == "plain":
            rows = B * S
            y = layer.forward(xd[:rows]).float().cpu().numpy()
            ref, _, _, _ = O.forward_sparse(xm[:rows], p, k)
            o_idx, o_w, _, o_gap = O.route(xm[:rows], p["wr"], k)
        else:
            xs = np.concatenate([x[b * 400:b * 400 + S] for b in range(B)])
            xms = np.concatenate([xm[b * 400:b * 400 + S] for b in range(B)])
            rows = B * S
            y = layer.forward_block(to_device(xs, dtype).reshape(B, S, D), dev(sh), dev(sc),
                                    dev(g), dev(nw)).reshape(rows, D).float().cpu().numpy()
            ref, _, _, _ = O.block_ffn(xms, p, k, sh, sc, g, S, nw, 1e-6, dtype, pow_mode=0)
            h1, _ = O.norm_modulate(xms, sh, sc, S, nw, 1e-6, dtype, pow_mode=1)
            o_idx, o_w, _, o_gap = O.route(h1, p["wr"], k)
        near = check_routing(layer, rows, o_idx, o_w, o_gap, E)
        assert np.isfinite(y).all() and rel_err(y[~near], ref[~near]) <= TOL[dtype]


def test_two_handles_alternating_on_one_stream():
    # two layers of different shapes used in turn: each has its own workspace
    l1, x1, xm1, *_, p1, _ = block_case(1, 300, 256, 8, 2, 128, "bf16", seed=67)
    l2, x2, xm2, *_, p2, _ = block_case(1, 500, 512, 4, 1, 256, "bf16", seed=68)
    x1d, x2d = to_device(x1, "bf16"), to_device(x2, "bf16")
    outs = []
    for _ in range(2):
        outs.append((l1.forward(x1d).float().cpu().numpy(), l2.forward(x2d).float().cpu().numpy()))
    for (a, b) in outs:
        assert rel_err(a, O.forward_sparse(xm1, p1, 2)[0]) <= TOL["bf16"]
        assert rel_err(b, O.forward_sparse(xm2, p2, 1)[0]) <= TOL["bf16"]
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
