"""GPU parity over a fixed, seeded sample of random configurations.

Each case draws dim, hidden, experts, top-k, rows, dtype, router scale and
the shared dense branch from fixed lists (MFMA-tiled and general shapes, one
to 256 experts, up to top-20), builds the layer from seeded checkpoint
tensors and compares routing and outputs with the oracle to the usual bars
(tests/_gpu.py: compare).  Configurations the library rejects at
construction (the dispatch kernel's LDS limit) are skipped.
"""
import random

import numpy as np
import pytest
import torch

import nomas_moe as nm
import oracle as O
from _common import rounded, small_case
from _gpu import TOL, check_routing, compare, layer_from_tensors, rel_err, to_device

pytestmark = pytest.mark.gpu


def _cases(seed=20261202, n=40):
    rng = random.Random(seed)
    out = []
    for c in range(n):
        D = rng.choice([64, 72, 256, 512, 768, 1024])
        H = rng.choice([96, 128, 256, 384, 640])
        E = rng.choice([1, 2, 3, 5, 8, 13, 16, 17, 31, 33, 64, 70, 100, 256])
        k = rng.randint(1, min(E, rng.choice([2, 4, 10, 20])))
        s = rng.choice([0.0, 0.0, 0.5])
        rows = rng.choice([1, 7, 64, 65, 300, 1000, 2500])
        while rows > 1 and rows * (k + 1) * D * H * 6 > 5e9:  # oracle work per case
            rows //= 2
        dt = rng.choice(["bf16", "f16", "f32"])
        std = rng.choice([0.02, 0.5])
        out.append((rows, D, E, k, H, dt, s, std, 3000 + c))
    return out


@pytest.mark.parametrize("rows,D,E,k,H,dt,s,std,seed", _cases())
def test_random_configuration(rows, D, E, k, H, dt, s, std, seed):
    print(f"sweep rows={rows} D={D} E={E} k={k} H={H} {dt} dense={s} std={std} seed={seed}",
          flush=True)
    t, x = small_case(rows, D, E, k, H, seed, dense=s > 0, router_std=std)
    try:
        layer = layer_from_tensors(t, dt, D, H, E, k, s)
    except nm.NomasError as e:
        pytest.skip(f"rejected by the library: {e}")
    rt, rx = rounded(t, x, dt)
    p, dn = nm.workloads.oracle_params(rt, E)
    compare(layer, to_device(x, dt), rx, p, k, dt, shared_dense=s, dense=dn)


def _block_cases(seed=20261203, n=12):
    rng = random.Random(seed)
    out = []
    for c in range(n):
        B = rng.choice([1, 2, 3])
        S = rng.choice([1, 17, 64, 300])
        D = rng.choice([64, 256, 264, 512])
        H = rng.choice([96, 128, 256])
        E = rng.choice([1, 4, 8, 17, 40])
        k = rng.randint(1, min(E, 4))
        s = rng.choice([0.0, 0.5])
        dt = rng.choice(["bf16", "f16", "f32"])
        affine = rng.choice([True, False])
        out.append((B, S, D, E, k, H, dt, s, affine, 4000 + c))
    return out


@pytest.mark.parametrize("B,S,D,E,k,H,dt,s,affine,seed", _block_cases())
def test_random_block_configuration(B, S, D, E, k, H, dt, s, affine, seed):
    """forward_block (norm2 + modulate, MoE, gated residual) on seeded random shapes."""
    from test_gpu_block import block_case, dev
    print(f"block sweep B={B} S={S} D={D} E={E} k={k} H={H} {dt} dense={s} affine={affine} "
          f"seed={seed}", flush=True)
    try:
        layer, x, xm, sh, sc, g, nw, p, dn = block_case(B, S, D, E, k, H, dt, seed, s, affine)
    except nm.NomasError as e:
        pytest.skip(f"rejected by the library: {e}")
    out = layer.forward_block(to_device(x, dt).reshape(B, S, D), dev(sh), dev(sc), dev(g), dev(nw))
    torch.cuda.synchronize()
    h1, _ = O.norm_modulate(xm, sh, sc, S, nw, 1e-6, dt, pow_mode=1)
    o_idx, o_w, _, o_gap = O.route(h1, p["wr"], k)
    near = check_routing(layer, B * S, o_idx, o_w, o_gap, E)
    ref, _, _, _ = O.block_ffn(xm, p, k, sh, sc, g, S, nw, 1e-6, dt, pow_mode=0,
                               shared_dense=s, dense=dn)
    got = out.reshape(B * S, D).float().cpu().numpy()
    err = rel_err(got[~near], ref[~near])
    print(f"  rel err {err:.3e}, near ties {int(near.sum())}, mfma={layer.uses_mfma}", flush=True)
    assert np.isfinite(got).all() and err <= TOL[dt]


@pytest.mark.parametrize("B,S,D,E,k,H,dt,s,affine,seed", [
    (2, 64, 512, 16, 8, 128, "bf16", 0.0, True, 4100),   # one group of 8 slots
    (1, 300, 256, 40, 10, 256, "f16", 0.5, False, 4101),  # 8 + 3 (dense slot)
    (3, 17, 512, 64, 8, 128, "f32", 0.5, True, 4102),    # 8 + 1 (dense slot)
    (1, 64, 264, 17, 9, 96, "bf16", 0.0, True, 4103),    # 8 + 1, general GEMM path
])
def test_block_many_slots(B, S, D, E, k, H, dt, s, affine, seed):
    """forward_block with 8 or more slots per row: the gated-residual combine
    sums its slots in groups of up to 8."""
    test_random_block_configuration(B, S, D, E, k, H, dt, s, affine, seed)


def _ffn_cases(seed=20261204, n=8):
    rng = random.Random(seed)
    return [(rng.choice([1, 33, 256, 700, 2000]), rng.choice([64, 72, 256, 512]),
             rng.choice([96, 128, 256, 384]), rng.choice(["bf16", "f16", "f32"]),
             rng.choice([True, False]), 5000 + c) for c in range(n)]


@pytest.mark.parametrize("rows,D,H,dt,bias,seed", _ffn_cases())
def test_random_ffn_configuration(rows, D, H, dt, bias, seed):
    """The dense SwiGLU FFN (mlp.rs:42-46) on seeded random shapes."""
    from test_gpu_ffn import run
    run(rows, D, H, dt, seed, bias=bias)
