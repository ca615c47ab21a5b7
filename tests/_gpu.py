"""Helpers of the GPU tests: build layers, run forwards, compare with the oracle."""
from __future__ import annotations

import numpy as np
import torch

import nomas_moe as nm
import oracle as O

NEAR_TIE = 1e-6  # logit gap below which a routing difference is reported, not failed
TOL = {"f32": 1e-4, "bf16": 2e-2, "f16": 2e-2}  # max|gpu - oracle| / max|oracle|
# Against the oracle with the GPU path's storage roundings (h, y_perm and the
# output in the model dtype, the combine an f32 FMA chain): (max|gpu - ref| /
# max|ref|, ||gpu - ref|| / ||ref||).  What remains is the kernels' own f32
# accumulation order and the rare model-dtype rounding it flips.
TIGHT = {"f32": (1e-5, 5e-6), "bf16": (1e-2, 5e-3), "f16": (1e-2, 5e-3)}

# Row offsets inside each 256-row expert tile that the full-size tests check:
# both wave halves of the token rows (0-127, 128-255), several 16-row MFMA
# blocks, and the tile's last live row (its padded tail when the tile is short).
TILE_OFFSETS = (0, 53, 127, 128, 199, 255)
BM = 256


def tile_rows(idx: np.ndarray, E: int, offsets=TILE_OFFSETS, bm: int = BM):
    """Rows that cover every (expert, 256-row tile) of the grouped GEMMs.

    An expert's rows sit in x_perm in ascending row order (the dispatch's
    stable permutation), so its r-th row lands in tile r // bm at offset
    r % bm.  For each tile and each wanted offset (clamped to the tile's last
    live row) the row at that rank is taken, unless a row already taken for
    another expert lands on that same (expert, tile, offset).  A checked row
    covers every column tile of both GEMMs for its row tiles (the output row
    needs all of h), including tiles split along K.  Returns (rows, tiles),
    tiles = the number of (expert, tile) pairs covered."""
    T, k = idx.shape
    ranks = {}
    for e in range(E):
        ranks[e] = np.nonzero((idx == e).any(axis=1))[0]  # ascending rows = positions
    covered = set()
    chosen = []
    pos = {}  # (row, expert) -> rank
    for e in range(E):
        for r_i, row in enumerate(ranks[e]):
            pos[(int(row), e)] = r_i
    ntiles = 0
    for e in range(E):
        n = ranks[e].size
        for t0 in range(0, n, bm):
            ntiles += 1
            last = min(t0 + bm, n) - 1
            for off in offsets:
                r_i = min(t0 + off, last)
                key = (e, t0 // bm, r_i - t0)
                if key in covered:
                    continue
                row = int(ranks[e][r_i])
                chosen.append(row)
                for ee in idx[row]:
                    ee = int(ee)
                    rr = pos[(row, ee)]
                    covered.add((ee, rr // bm, rr - (rr // bm) * bm))
    return np.unique(np.asarray(chosen, np.int64)), ntiles


def rms_rel(got, ref) -> float:
    """||got - ref||_2 / ||ref||_2."""
    ref = np.asarray(ref, np.float64)
    den = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    num = float(np.sqrt(np.mean((np.asarray(got, np.float64) - ref) ** 2))) if ref.size else 0.0
    return num / den if den > 0 else num


def to_device(x_f32: np.ndarray, dtype) -> torch.Tensor:
    raw = nm.to_model_dtype(x_f32, dtype)
    t = torch.from_numpy(raw.view(np.int16) if raw.dtype == np.uint16 else raw)
    return t.view(nm.DataType.of(dtype).torch).cuda()


def layer_from_tensors(t, dtype, dim, hidden, E, k, s=0.0, path="blocks.0.moe"):
    cfg = nm.MoeConfig(E, k, s, 0)
    return nm.MoeLayer.from_source(nm.Weights.from_tensors(t, dtype), path, dim, hidden, cfg)


def rel_err(got, ref) -> float:
    ref = np.asarray(ref, np.float64)
    den = float(np.max(np.abs(ref))) if ref.size else 0.0
    diff = float(np.max(np.abs(np.asarray(got, np.float64) - ref))) if ref.size else 0.0
    return diff / den if den > 0 else diff


def check_routing(layer, rows, o_idx, o_w, o_gap, E):
    """Indices bit-exact and counts exact except on near ties; gates to 1e-5 relative.

    The 16-bit router sums each 32-term block of exact products in f32 before
    the f64 accumulation, so a logit carries about 1e-7 of its own scale in
    rounding; gates follow logit differences, and with logits of scale ~16
    (router std 0.5 at dim 1024) that reaches a few 1e-6.
    """
    idx, w, counts, gap = layer.routing(rows)
    near = o_gap < NEAR_TIE
    assert np.array_equal(idx[~near], o_idx[~near]), (
        f"expert indices differ on {(idx[~near] != o_idx[~near]).any(axis=1).sum()} rows")
    want_counts = np.bincount(o_idx.ravel(), minlength=E)
    if near.any():
        assert np.abs(counts - want_counts).sum() <= 2 * int(near.sum()) * o_idx.shape[1]
    else:
        assert np.array_equal(counts, want_counts)
    np.testing.assert_allclose(w[~near], o_w[~near], rtol=1e-5, atol=1e-7)
    return near


def compare(layer, x_dev, x_oracle, p, k, dtype, rows=None, shared_dense=0.0, dense=None):
    """Run the layer and compare outputs (on `rows`, default all) and routing with the oracle."""
    y = layer.forward(x_dev)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().reshape(x_oracle.shape)
    n = x_oracle.shape[0]
    o_idx, o_w, _, o_gap = O.route(x_oracle, p["wr"], k)
    near = check_routing(layer, n, o_idx, o_w, o_gap, p["wr"].shape[0])
    sel = np.arange(n) if rows is None else np.asarray(rows)
    sel = sel[~near[sel]]
    ref, _, _, _ = O.forward_sparse(x_oracle, p, k, rows=sel, shared_dense=shared_dense,
                                    dense=dense)
    err = rel_err(got[sel], ref)
    tight = check_tight(got[sel], x_oracle, p, k, dtype, sel, shared_dense, dense)
    print(f"  rel err {err:.3e} on {sel.size} rows, near ties {int(near.sum())}, "
          f"mfma={layer.uses_mfma}; vs rounded oracle max {tight[0]:.3e} "
          f"worst row rms {tight[1]:.3e}",
          flush=True)
    assert err <= TOL[dtype], f"relative error {err:.3e} above {TOL[dtype]}"
    assert np.isfinite(got).all()
    return got, err


def row_rms_rel(got, ref) -> float:
    """The worst row's ||got_r - ref_r|| / ||ref_r|| (a fault confined to one
    tile shows in its rows without being diluted by the others)."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    num = np.sqrt(np.mean((got - ref) ** 2, axis=1))
    den = np.sqrt(np.mean(ref * ref, axis=1))
    ok = den > 0
    worst = float(np.max(num[ok] / den[ok])) if ok.any() else 0.0
    return max(worst, float(np.max(num[~ok])) if (~ok).any() else 0.0)


def tight_metrics(got_rows, ref_rows):
    """(max|got - ref| / max|ref|, the worst row's relative rms)."""
    return rel_err(got_rows, ref_rows), row_rms_rel(got_rows, ref_rows)


def check_tight(got_rows, x_oracle, p, k, dtype, rows, shared_dense=0.0, dense=None):
    """The tight bar: the GPU rows against the oracle with the GPU path's
    storage roundings (orc_forward_sparse_rounded).  Returns (max, worst-row rms)."""
    ref = O.forward_sparse_rounded(x_oracle, p, k, dtype, rows=rows, shared_dense=shared_dense,
                                   dense=dense)
    m, r = tight_metrics(got_rows, ref)
    tm, tr = TIGHT[dtype]
    assert m <= tm and r <= tr, (
        f"vs the rounded oracle: max {m:.3e} (bar {tm}), worst row rms {r:.3e} (bar {tr})")
    return m, r
