"""GPU parity of the dense SwiGLU feed-forward (FeedForward::SwiGlu, mlp.rs:9-59).

The same bar as the MoE outputs: max|gpu - oracle| / max|oracle| <= 1e-4 for
f32 and <= 2e-2 for bf16 / f16, the oracle (orc_ffn_f64) computing in f64 from
the same rounded inputs.
"""
import math

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file

import nomas_moe as nm
import oracle as O
from _common import rel_err
from _gpu import TOL, to_device

pytestmark = pytest.mark.gpu

PATH = "blocks.0.mlp"


def ffn_case(rows, dim, hidden, seed, bias=True):
    """Seeded f32 parameters (checkpoint keys) and x."""
    t = {}
    for name, (o, i) in (("gate", (hidden, dim)), ("up", (hidden, dim)), ("down", (dim, hidden))):
        key = f"{PATH}.{name}"
        t[key + ".weight"] = nm.randn_affine(nm.path_seed(seed, key), o * i, 0.0,
                                             1.0 / math.sqrt(i)).reshape(o, i)
        if bias:
            t[key + ".bias"] = nm.randn_affine(nm.path_seed(seed, key + ".bias"), o, 0.0, 0.1)
    x = nm.randn_affine(nm.path_seed(seed, "x"), rows * dim).reshape(rows, dim)
    return t, x


def oracle_f(t, dtype):
    """The parameters rounded to the model dtype, widened, in the oracle's names."""
    r = {k: nm.widen(nm.to_model_dtype(v, dtype), dtype) for k, v in t.items()}
    return {"wg": r[f"{PATH}.gate.weight"], "bg": r.get(f"{PATH}.gate.bias"),
            "wu": r[f"{PATH}.up.weight"], "bu": r.get(f"{PATH}.up.bias"),
            "wd": r[f"{PATH}.down.weight"], "bd": r.get(f"{PATH}.down.bias")}


def run(rows, dim, hidden, dtype, seed, bias=True):
    print(f"ffn rows={rows} D={dim} H={hidden} {dtype} seed={seed} bias={bias}", flush=True)
    t, x = ffn_case(rows, dim, hidden, seed, bias)
    ffn = nm.FeedForward.from_source(nm.Weights.from_tensors(t, dtype), PATH, dim, hidden)
    y = ffn.forward(to_device(x, dtype))
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    ref = O.ffn(nm.widen(nm.to_model_dtype(x, dtype), dtype), oracle_f(t, dtype))
    err = rel_err(got, ref)
    print(f"  rel err {err:.3e} mfma={ffn.uses_mfma}", flush=True)
    assert np.isfinite(got).all()
    assert err <= TOL[dtype], f"relative error {err:.3e} above {TOL[dtype]}"
    return ffn, x, got


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_mfma_path(dtype):
    ffn, _, _ = run(300, 256, 384, dtype, seed=41)
    assert ffn.uses_mfma


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_general_path(dtype):
    # shapes the MFMA kernels do not tile take the general path
    ffn, _, _ = run(130, 72, 100, dtype, seed=42)
    assert not ffn.uses_mfma


@pytest.mark.parametrize("rows", [1, 255, 256, 257, 1000])
def test_row_counts_around_tile_edges(rows):
    run(rows, 256, 256, "bf16", seed=43 + rows)


def test_no_bias_and_zero_rows():
    ffn, _, _ = run(64, 256, 128, "bf16", seed=44, bias=False)
    y = ffn.forward(torch.empty((0, 256), dtype=torch.bfloat16, device="cuda"))
    assert tuple(y.shape) == (0, 256)


def test_random_init_matches_reference_keys_and_n_params():
    # Weights::Random: xavier weights keyed by path_seed(seed, "{path}.{gate,up,down}"),
    # zero biases (mod.rs:80-95); n_params = mlp.rs:50-58
    D, H = 256, 128
    ffn = nm.FeedForward.from_source(nm.Weights.random(7, "f32"), PATH, D, H)
    assert ffn.n_params() == 2 * (H * D + H) + (D * H + D)
    f = {"wg": O.xavier(H, D, O.path_seed(7, PATH + ".gate")),
         "wu": O.xavier(H, D, O.path_seed(7, PATH + ".up")),
         "wd": O.xavier(D, H, O.path_seed(7, PATH + ".down"))}
    x = nm.randn_affine(3, 10 * D).reshape(10, D)
    y = ffn.forward(torch.from_numpy(x).cuda())
    assert rel_err(y.cpu().numpy(), O.ffn(x, f)) <= TOL["f32"]


def test_host_tensors_and_leading_dims():
    ffn, x, got = run(96, 256, 256, "bf16", seed=45)
    raw = nm.to_model_dtype(x, "bf16")
    xh = torch.from_numpy(raw.view(np.int16)).view(torch.bfloat16).reshape(2, 48, 256)
    yh = ffn.forward(xh)  # host tensor: copied in and out; leading dims folded
    assert tuple(yh.shape) == (2, 48, 256) and not yh.is_cuda
    assert torch.equal(yh.reshape(96, 256).float(), torch.from_numpy(got))


def test_host_tensors_in_pieces():
    # 9,000 host rows: two pieces of 4,544 and 4,456 rows whose copies overlap the other's forward;
    # against the oracle and a device forward of all rows (a K-split tile may round differently)
    t, x = ffn_case(9000, 256, 256, 46)
    ffn = nm.FeedForward.from_source(nm.Weights.from_tensors(t, "bf16"), PATH, 256, 256)
    raw = nm.to_model_dtype(x, "bf16")
    xh = torch.from_numpy(raw.view(np.int16)).view(torch.bfloat16)
    yd = ffn.forward(xh.cuda()).float().cpu().numpy()
    yh = ffn.forward(xh)
    assert not yh.is_cuda
    got = yh.float().numpy()
    ref = O.ffn(nm.widen(raw, "bf16"), oracle_f(t, "bf16"))
    assert rel_err(got, ref) <= TOL["bf16"]
    assert rel_err(got, yd) <= 1e-2  # at most a bf16 ulp where rounding differs


def test_safetensors_checkpoint_equals_in_memory_tensors(tmp_path):
    t, x = ffn_case(80, 256, 256, seed=46)
    f = str(tmp_path / "ffn.safetensors")
    save_file(t, f)
    a = nm.FeedForward.from_source(nm.Weights.loaded([f], "bf16"), PATH, 256, 256)
    b = nm.FeedForward.from_source(nm.Weights.from_tensors(t, "bf16"), PATH, 256, 256)
    xd = to_device(x, "bf16")
    assert torch.equal(a.forward(xd), b.forward(xd))


def test_dense_ffn_equals_one_expert_moe():
    # the MoE with one expert and top-1 runs the same expert with gate 1/(1+1e-9)
    D, H = 256, 256
    t, x = ffn_case(200, D, H, seed=47)
    ffn = nm.FeedForward.from_source(nm.Weights.from_tensors(t, "bf16"), PATH, D, H)
    mt = {"m.router.weight": np.zeros((1, D), np.float32)}
    for k, v in t.items():
        mt[k.replace(PATH, "m.experts.0")] = v
    moe = nm.MoeLayer.from_source(nm.Weights.from_tensors(mt, "bf16"), "m", D, H,
                                  nm.MoeConfig(1, 1))
    xd = to_device(x, "bf16")
    a = ffn.forward(xd).float().cpu().numpy()
    b = moe.forward(xd).float().cpu().numpy()
    assert rel_err(a, b) <= 1e-2


def test_stage_profiling():
    ffn, _, _ = run(512, 256, 256, "bf16", seed=48)
    ffn.set_profiling(True)
    ffn.forward(to_device(nm.randn_affine(1, 512 * 256).reshape(512, 256), "bf16"))
    st = ffn.stage_times()
    ffn.set_profiling(False)
    assert set(st) == set(nm.FeedForward.STAGES)
    assert st["gemm_gate_up"] > 0 and st["gemm_down"] > 0
    assert st["router"] == 0 and st["combine"] == 0  # no such stages: no kernel, zero time


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_preset_8b_dense_ffn_full_size(dtype):
    # What the shipped 8B preset runs (moe: None, config.rs:297-330): the
    # dense SwiGLU FFN at dim 3072, hidden 3072 * 4.0 = 12288 (block.rs:38),
    # on one 4,744-row segment (4,680 video + 64 text rows), Weights::Random
    # (xavier weights, zero biases: mod.rs:80-95).  Rows at six offsets of
    # every 256-row GEMM tile (both wave halves, the last tile's tail) are
    # checked against the oracle in f64.
    D, H, rows, seed = 3072, 12288, 4744, 0x5EED0000
    print(f"8B dense FFN rows={rows} D={D} H={H} {dtype}", flush=True)
    ffn = nm.FeedForward.from_source(nm.Weights.random(seed, dtype), PATH, D, H)
    assert ffn.uses_mfma
    x = nm.randn_affine(nm.path_seed(seed, "x"), rows * D).reshape(rows, D)
    y = ffn.forward(to_device(x, dtype))
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    assert np.isfinite(got).all()
    sel = np.unique(np.minimum(
        (np.arange(0, rows, 256)[:, None] + np.array([0, 53, 127, 128, 199, 255])[None, :]).ravel(),
        rows - 1))
    f = {k: nm.widen(nm.to_model_dtype(O.xavier(o, i, O.path_seed(seed, f"{PATH}.{n}")), dtype), dtype)
         for k, n, o, i in (("wg", "gate", H, D), ("wu", "up", H, D), ("wd", "down", D, H))}
    xr = nm.widen(nm.to_model_dtype(x[sel], dtype), dtype)
    err = rel_err(got[sel], O.ffn(xr, f))
    print(f"  rel err {err:.3e} on {sel.size} rows", flush=True)
    assert err <= TOL[dtype], f"relative error {err:.3e} above {TOL[dtype]}"
