"""GPU parity: the HIP MoE forward against the CPU oracle on identical seeded inputs.

Bars (the path's contract):
  * expert indices and per-expert counts bit-exact, except rows whose f64
    logit gap between the k-th and (k+1)-th expert is below 1e-6 (reported);
  * outputs: max|gpu - oracle| / max|oracle| <= 1e-4 for f32 and <= 2e-2 for
    bf16 / f16, the oracle computing in f64 from the same rounded inputs.
"""
import math
import os

import numpy as np
import pytest
import torch

import nomas_moe as nm
import oracle as O
from _common import PATH, rounded, small_case
from _gpu import TOL, compare, layer_from_tensors, rel_err, to_device
from golden_cases import CASES, case_tensors

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def run_case(rows, dim, E, k, H, dtype, seed, bias=True, s=0.0, router_std=0.02, check_rows=None):
    print(f"case rows={rows} D={dim} E={E} k={k} H={H} {dtype} seed={seed} dense={s}", flush=True)
    t, x = small_case(rows, dim, E, k, H, seed, bias=bias, dense=s > 0, router_std=router_std)
    layer = layer_from_tensors(t, dtype, dim, H, E, k, s)
    rt, rx = rounded(t, x, dtype)
    p, dn = nm.workloads.oracle_params(rt, E)
    compare(layer, to_device(x, dtype), rx, p, k, dtype, rows=check_rows, shared_dense=s, dense=dn)
    return layer


def test_moe_output_shape_and_finiteness():
    """moe.rs:123-150 on the GPU: random weights, dim 32, hidden 64, 4 experts, top-2."""
    cfg = nm.MoeConfig(experts=4, top_k=2, shared_dense=0.0, seed=1)
    moe = nm.MoeLayer.from_source(nm.Weights.random(4, nm.DataType.F32), PATH, 32, 64, cfg)
    x = torch.from_numpy(nm.randn_affine(3, 1 * 5 * 32).reshape(1, 5, 32)).cuda()
    y = moe.forward(x)
    assert tuple(y.shape) == (1, 5, 32)
    assert torch.isfinite(y).all()
    # the same random weights (xavier by path seed, zero bias) through the oracle
    p = {"wr": O.xavier(4, 32, O.path_seed(4, PATH + ".router"))}
    for name, key, o, i in (("wg", "gate", 64, 32), ("wu", "up", 64, 32), ("wd", "down", 32, 64)):
        p[name] = np.stack([O.xavier(o, i, O.path_seed(4, f"{PATH}.experts.{e}.{key}"))
                            for e in range(4)])
    ref, _, _, _ = O.forward_sparse(x.cpu().numpy().reshape(5, 32), p, 2)
    assert rel_err(y.cpu().numpy().reshape(5, 32), ref) <= 1e-4


@pytest.mark.parametrize("name", sorted(CASES))
def test_golden_fixture(name):
    """The HIP path against the committed oracle outputs (tests/golden/)."""
    t, x, m = case_tensors(name)
    print(f"golden {name}: {m}", flush=True)
    g = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    layer = layer_from_tensors(t, m["dtype"], m["dim"], m["H"], m["E"], m["k"], m["shared_dense"])
    y = layer.forward(to_device(x, m["dtype"]))
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    idx, w, counts, gap = layer.routing(m["rows"])
    near = g["gap"] < 1e-6
    assert np.array_equal(idx[~near], g["idx"][~near])
    if not near.any():
        assert np.array_equal(counts, g["counts"])
    err = rel_err(got[~near], g["out"][~near])
    print(f"  rel err {err:.3e} mfma={layer.uses_mfma}", flush=True)
    assert err <= TOL[m["dtype"]]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_general_path(dtype):
    # D=72, H=100 are not tiled by the MFMA kernels: the general path for every dtype
    assert not run_case(150, 72, 6, 2, 100, dtype, seed=11).uses_mfma


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_mfma_path(dtype):
    assert run_case(300, 256, 8, 2, 128, dtype, seed=12).uses_mfma


def test_mfma_f32_ragged_split_tiles():
    # f32 on the matrix cores (16x16x4 MFMAs): ragged expert tiles, several
    # column tiles, a K long enough for the K-split tail, the quarter-tile
    # staging of the down GEMM's output
    run_case(900, 512, 4, 3, 384, "f32", seed=14)


def test_mfma_multi_tile_ragged():
    # several row tiles per expert, ragged last tiles, several column tiles, k = 3
    run_case(1000, 512, 4, 3, 384, "bf16", seed=13)


@pytest.mark.parametrize("rows", [1, 63, 64, 65, 257, 700])
def test_row_counts_around_chunk_and_tile_edges(rows):
    run_case(rows, 256, 8, 2, 128, "bf16", seed=100 + rows)


def test_zero_rows():
    t, x = small_case(4, 256, 8, 2, 128, 21)
    layer = layer_from_tensors(t, "bf16", 256, 128, 8, 2)
    y = layer.forward(to_device(x[:0], "bf16"))
    assert tuple(y.shape) == (0, 256)
    idx, w, counts, gap = layer.routing(0)
    assert counts.sum() == 0


def test_empty_and_overloaded_experts():
    # router rows 4..7 strongly negative on a constant feature: those experts never
    # win; rows concentrate on few experts (ragged, empty experts in the tile list)
    E, D, H, k = 8, 256, 128, 2
    t, x = small_case(900, D, E, k, H, 22)
    x[:, 0] = 4.0
    wr = t[PATH + ".router.weight"]
    wr[:, 0] = [3.0, 1.5, 0.0, -1.0, -40.0, -40.0, -40.0, -40.0]
    layer = layer_from_tensors(t, "bf16", D, H, E, k)
    rt, rx = rounded(t, x, "bf16")
    p, _ = nm.workloads.oracle_params(rt, E)
    compare(layer, to_device(x, "bf16"), rx, p, k, "bf16")
    _, _, counts, _ = layer.routing(900)
    assert (counts[4:] == 0).all() and counts.sum() == 900 * k


@pytest.mark.parametrize("E", [8, 40, 96])
def test_exact_ties_go_to_the_lowest_index(E):
    # duplicated router rows give bit-identical logits; the reference's
    # first-max-wins argmax (moe.rs:78-80) takes the lower expert.  Ties are
    # exact here, so no row is exempt: indices must equal the oracle's on every
    # row (E = 8 and 40 use the four-lanes-per-row selection, 96 the
    # wave-parallel one; 40 and 96 span several 16-expert logit blocks).
    D, H, k = 256, 128, 3
    t, x = small_case(400, D, E, k, H, 29 + E, router_std=0.2)
    wr = t[PATH + ".router.weight"]
    wr[E - 1] = wr[1]        # across logit blocks for E > 16
    wr[2] = wr[1]
    wr[E // 2] = wr[0]
    layer = layer_from_tensors(t, "bf16", D, H, E, k)
    rt, rx = rounded(t, x, "bf16")
    p, _ = nm.workloads.oracle_params(rt, E)
    layer.forward(to_device(x, "bf16"))
    torch.cuda.synchronize()
    idx, _, counts, gap = layer.routing(400)
    o_idx, _, o_logits, _ = O.route(rx, p["wr"], k)
    assert np.array_equal(o_logits[:, 1], o_logits[:, 2]) and np.array_equal(o_logits[:, 1], o_logits[:, E - 1])
    assert np.array_equal(idx, o_idx)
    assert np.array_equal(counts, np.bincount(o_idx.ravel(), minlength=E))
    # a selected duplicate implies its lower twins were selected first
    sel = np.zeros((400, E), bool)
    np.put_along_axis(sel, idx.astype(np.int64), True, axis=1)
    assert not (sel[:, 2] & ~sel[:, 1]).any() and not (sel[:, E - 1] & ~sel[:, 1]).any()


@pytest.mark.parametrize("E,k", [(8, 2), (40, 3), (64, 8)])
def test_near_ties_inside_the_selection_keys(E, k):
    # Twin router rows that differ only in one coordinate, by 2^-17, on a
    # column of x set to +-1: the twins' f64 logits differ by 2^-17 (7.6e-6),
    # far above the kernel's logit error (about 1e-8) and the 1e-6 near-tie
    # exemption, but inside the resolution of the selection's 32-bit keys
    # (17 significant bits: 1.5e-5 at these logit magnitudes of 2-4).  So
    # the f64 logits, not the expert index, must decide between twins, and
    # the indices must equal the oracle's on every row.
    D, H, rows = 256, 128, 400
    t, x = small_case(rows, D, E, k, H, 71 + E, router_std=0.2)
    wr = t[PATH + ".router.weight"]
    m0 = 5
    x[:, m0] = np.where(np.arange(rows) % 2 == 0, 1.0, -1.0)
    pairs = [(1, 2), (0, E - 1), (E // 2, E // 2 + 1)]
    for a, b in pairs:
        wr[b] = wr[a]
        wr[a, m0] = 0.0
        wr[b, m0] = 2.0 ** -17
    layer = layer_from_tensors(t, "bf16", D, H, E, k)
    rt, rx = rounded(t, x, "bf16")
    p, _ = nm.workloads.oracle_params(rt, E)
    layer.forward(to_device(x, "bf16"))
    torch.cuda.synchronize()
    idx, _, counts, _ = layer.routing(rows)
    o_idx, _, o_logits, o_gap = O.route(rx, p["wr"], k)
    for a, b in pairs:
        assert np.allclose(np.abs(o_logits[:, b] - o_logits[:, a]), 2.0 ** -17, rtol=1e-6, atol=0)
    sel = np.zeros((rows, E), bool)
    np.put_along_axis(sel, o_idx.astype(np.int64), True, axis=1)
    split = np.zeros(rows, bool)  # rows where the oracle chose exactly one twin
    for a, b in pairs:
        split |= sel[:, a] != sel[:, b]
    assert split.sum() >= 10, "too few rows with a twin on each side of the k-th place"
    assert (o_gap[split] >= 1e-6).all()  # none of them exempt
    assert np.array_equal(idx, o_idx)
    assert np.array_equal(counts, np.bincount(o_idx.ravel(), minlength=E))


@pytest.mark.parametrize("E,k,dtype", [(16, 2, "bf16"), (24, 3, "bf16"), (32, 4, "f16"),
                                       (48, 6, "bf16"), (64, 8, "f16"), (65, 8, "bf16")])
def test_router_pass_widths(E, k, dtype):
    # one pass over x covers 16, 32 or 64 experts (E <= 16, <= 32, more), with
    # partly filled 16-expert blocks; the selection takes 8 lanes per row up to
    # 64 experts (2 candidates per lane up to 16 experts, 8 beyond), the whole
    # wave per row past 64
    run_case(330, 256, E, k, 128, dtype, seed=40 + E, router_std=0.2)


@pytest.mark.parametrize("rows", [4999, 8192, 8193])
@pytest.mark.parametrize("E,k", [(16, 2), (32, 4), (64, 8)])
def test_router_block_plans(rows, E, k):
    # The 16-bit router's rows per block and ring depth follow the row count
    # and the experts: up to 8,192 rows and 32 experts, 32-row blocks with a
    # deep ring (1 or 2 groups of 16 experts), otherwise 64-row blocks (up to
    # 4 groups).  The dispatch adds the two 32-row histograms of each 64-row
    # chunk (the last chunk of 4,999 rows has one).  Routing on every row,
    # outputs on a spread of rows.
    D, H = 256, 128
    t, x = small_case(rows, D, E, k, H, 500 + E + rows, router_std=0.2)
    layer = layer_from_tensors(t, "bf16", D, H, E, k)
    rt, rx = rounded(t, x, "bf16")
    p, _ = nm.workloads.oracle_params(rt, E)
    sel = np.unique(np.r_[np.arange(0, rows, 97), rows - 1])
    compare(layer, to_device(x, "bf16"), rx, p, k, "bf16", rows=sel)


def test_more_than_64_slots_per_row():
    # top-70 of 80: the combine reads slots past 64 from memory, not from lanes
    run_case(100, 256, 80, 70, 128, "bf16", seed=39, router_std=0.2)


def test_routed_buffers_past_2_gib():
    # 180,000 rows, top-2 of 8 at dim 3072: x_perm and y_perm hold 360,000
    # routed rows (2.2 GB each), so their byte offsets pass 2^31.  Routing is
    # checked on every row, the outputs on 96 rows spread over the range.
    E, D, H, k, T = 8, 3072, 256, 2, 180_000
    t, x = small_case(T, D, E, k, H, 31)
    layer = layer_from_tensors(t, "bf16", D, H, E, k)
    rt, rx = rounded(t, x, "bf16")
    p, _ = nm.workloads.oracle_params(rt, E)
    rows = np.linspace(0, T - 1, 96).astype(np.int64)
    compare(layer, to_device(x, "bf16"), rx, p, k, "bf16", rows=rows)


def test_k_equals_experts_mfma():
    run_case(200, 256, 4, 4, 256, "bf16", seed=23)


def test_top1_single_expert_dense_ffn():
    # E = 1, k = 1: the block degenerates to the dense SwiGLU FFN (mlp.rs:42-46)
    run_case(333, 256, 1, 1, 256, "bf16", seed=24)
    run_case(50, 64, 1, 1, 96, "f32", seed=25)


def test_max_experts():
    # 256 experts: the router keeps 64 rows x 256 f64 logits in LDS (128 KB)
    run_case(300, 256, 256, 8, 128, "bf16", seed=26, router_std=0.2)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_shared_dense_branch(dtype):
    D, H = (256, 128) if dtype == "bf16" else (64, 80)
    run_case(180, D, 6, 2, H, dtype, seed=27, s=0.6)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_nontemporal_output_whole_row_combine(dtype):
    """y_perm past the 256 MiB last-level cache (11,008 rows x top-4 x 3072 x 2 bytes = 270.5 MB):
    the down GEMM and the combine store nontemporally, and the combine covers a whole 3072-wide
    row per pass.  Checked on every 43rd row and the last."""
    rows = 11008
    sel = np.unique(np.r_[np.arange(0, rows, 43), rows - 1])
    run_case(rows, 3072, 8, 4, 128, dtype, seed=29, check_rows=sel)


def test_workspace_regrowth_and_determinism():
    E, D, H, k = 8, 256, 256, 2
    t, x = small_case(1500, D, E, k, H, 28)
    layer = layer_from_tensors(t, "bf16", D, H, E, k)
    rt, rx = rounded(t, x, "bf16")
    p, _ = nm.workloads.oracle_params(rt, E)
    xd = to_device(x, "bf16")
    outs = {}
    for n in (100, 1500, 37, 1500):
        got, _ = compare(layer, xd[:n], rx[:n], p, k, "bf16")
        outs.setdefault(n, []).append(got)
    # no atomics in the data path: repeated forwards are bitwise identical
    assert np.array_equal(outs[1500][0], outs[1500][1])
