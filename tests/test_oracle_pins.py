"""Pins of the CPU oracle (oracle/moe_oracle.c) -- CPU only.

The reference (hy-nomas-rs) ships no numeric golden vectors for its MoE path,
so every oracle function is pinned here by something independent of it:
  * published known answers (SplitMix64 outputs, the FNV-1a test suite);
  * textbook invariants (Box-Muller radius and angle, softmax sums);
  * independent library implementations of the same mathematics (numpy /
    torch float64 matmul, softmax, silu, stable argsort) on small inputs;
  * special cases that reduce to closed forms (k = E, one dominant expert,
    zero input, permutation of rows, the additive dense branch).
test_each_planted_mistake_is_caught plants each plausible mistake in the
oracle (on the CPU, through orc_mutation) and requires that at least one pin
fails -- the pins have teeth.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O

# --------------------------------------------------------------------------
# known answers
# --------------------------------------------------------------------------

# SplitMix64 (Steele, Lea & Flood; Vigna's reference splitmix64.c) from state 0
SPLITMIX_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
# FNV-1a 64-bit test vectors (FNV reference suite): offset basis cbf29ce484222325
FNV1A_64 = {"": 0xCBF29CE484222325, "a": 0xAF63DC4C8601EC8C, "foobar": 0x85944171F73967E8}


def pin_splitmix64():
    assert O.splitmix64(0, 3) == SPLITMIX_SEED0


def pin_fnv1a():
    # path_seed(0, p) is plain FNV-1a (mod.rs:47-55 with a zero base seed)
    for s, h in FNV1A_64.items():
        assert O.path_seed(0, s) == h, s
    # a non-zero seed only changes the offset basis: empty path -> basis ^ seed
    assert O.path_seed(0x5EED0002, "") == FNV1A_64[""] ^ 0x5EED0002


def _uniform_draws(seed, n):
    return [(v >> 11) * (1.0 / 9007199254740992.0) for v in O.splitmix64(seed, n)]


def pin_box_muller():
    # z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), r = sqrt(-2 ln u1): the radius
    # and the angle of each pair are fixed by the two uniform draws.
    seed, pairs = 1234, 200
    u = _uniform_draws(seed, 2 * pairs)
    z = O.randn_affine(seed, 2 * pairs).astype(np.float64)
    for j in range(pairs):
        u1, u2 = u[2 * j], u[2 * j + 1]
        z0, z1 = z[2 * j], z[2 * j + 1]
        r2 = -2.0 * math.log(u1)
        assert abs(z0 * z0 + z1 * z1 - r2) <= 1e-6 * max(1.0, r2), j
        ang = math.atan2(z1, z0) % (2 * math.pi)
        want = (2 * math.pi * u2) % (2 * math.pi)
        d = abs(ang - want)
        assert min(d, 2 * math.pi - d) <= 1e-5 * (1 + 1 / max(math.sqrt(r2), 1e-3)), j


def pin_affine_and_moments():
    z = O.randn_affine(77, 200_000).astype(np.float64)
    assert abs(z.mean()) < 5 / math.sqrt(z.size)
    assert abs(z.std() - 1.0) < 5 / math.sqrt(2 * z.size)
    a = O.randn_affine(77, 1000, mean=3.0, std=0.5)
    np.testing.assert_allclose(a, (z[:1000] * 0.5 + 3.0).astype(np.float32), rtol=0, atol=5e-7)


def pin_uniform():
    # deterministic_uniform (tensor_utils.rs:140-155): one 53-bit draw per
    # element, mapped affinely onto [lo, hi); range and the U(lo, hi) moments
    # hold independently of how the draw is formed
    lo, hi, n = -0.5, 1.5, 100_000
    u = O.uniform(31, n, lo, hi).astype(np.float64)
    assert u.min() >= lo and u.max() < hi
    assert abs(u.mean() - (lo + hi) / 2) < 5 * (hi - lo) / math.sqrt(12 * n)
    assert abs(u.var() - (hi - lo) ** 2 / 12) < 0.01 * (hi - lo) ** 2 / 12
    want = np.array([lo + d * (hi - lo) for d in _uniform_draws(31, 64)], np.float32)
    np.testing.assert_array_equal(u[:64].astype(np.float32), want)


def pin_xavier_std():
    w = O.xavier(256, 192, 9).astype(np.float64)
    want = math.sqrt(2.0 / (256 + 192))
    assert abs(w.std() - want) < 0.02 * want
    np.testing.assert_array_equal(w.ravel().astype(np.float32),
                                  O.randn_affine(9, 256 * 192, 0.0, want))


def pin_bf16_rounding():
    x = np.concatenate([O.randn_affine(5, 4000, 0.0, 10.0),
                        np.array([1.00390625, 1.01171875, -2.5e-30, 3.0e38, 0.0], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.round_bf16(x), want)


# --------------------------------------------------------------------------
# routing (moe.rs:67-95)
# --------------------------------------------------------------------------

def _np_route(x, wr, k):
    """Independent restatement: numpy f64 logits, stable descending sort
    (lowest index first on ties), softmax renormalised over the top k."""
    logits = x.astype(np.float64) @ wr.astype(np.float64).T
    order = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    idx = np.sort(order, axis=1)
    top = np.take_along_axis(p, idx, axis=1)
    w = top / (top.sum(axis=1, keepdims=True) + 1e-9)
    return idx.astype(np.int32), w, logits


def pin_route_bruteforce():
    rng = np.random.default_rng(3)
    for (T, D, E, k) in [(64, 16, 6, 2), (40, 24, 8, 3), (16, 8, 4, 4), (30, 12, 5, 1)]:
        x = rng.standard_normal((T, D)).astype(np.float32)
        wr = rng.standard_normal((E, D)).astype(np.float32)
        idx, w, logits, gap = O.route(x, wr, k)
        ridx, rw, rl = _np_route(x, wr, k)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_allclose(w, rw, rtol=1e-12, atol=1e-15)
        np.testing.assert_allclose(logits, rl, rtol=1e-12, atol=1e-12)


def pin_route_ties_lowest_index():
    # experts 1 and 3 identical: every tie must go to expert 1
    rng = np.random.default_rng(4)
    wr = rng.standard_normal((5, 8)).astype(np.float32)
    wr[3] = wr[1]
    x = np.tile(wr[1], (6, 1)) * np.float32(4.0)  # makes experts 1 and 3 the two largest
    idx, w, _, gap = O.route(x, wr, 1)
    assert (idx[:, 0] == 1).all()
    idx2, w2, _, _ = O.route(x, wr, 2)
    assert (idx2 == [1, 3]).all()
    np.testing.assert_allclose(w2, 0.5, rtol=1e-8)


def pin_route_one_hot_rows():
    # x = e_j selects column j of the router weight as the logits
    rng = np.random.default_rng(5)
    wr = rng.standard_normal((6, 10)).astype(np.float32)
    x = np.eye(10, dtype=np.float32)
    _, _, logits, _ = O.route(x, wr, 2)
    np.testing.assert_array_equal(logits, wr.T.astype(np.float64))


def pin_route_weights_sum_to_one():
    # the reference's own routing test (moe.rs:152-188): uniform(0.1, 0.9)
    # probabilities of shape (1, 3, 5) from seed 5, top-2, weights sum to 1.
    # With x = log(p) and an identity router the softmax returns p / sum(p).
    p = O.uniform(5, 15, 0.1, 0.9).reshape(3, 5).astype(np.float64)
    x = np.log(p).astype(np.float32)
    idx, w, _, _ = O.route(x, np.eye(5, dtype=np.float32), 2)
    assert np.all(np.abs(w.sum(axis=1) - 1.0) < 1e-5)
    want = np.sort(np.argsort(-p, axis=1, kind="stable")[:, :2], axis=1)
    np.testing.assert_array_equal(idx, want)


# --------------------------------------------------------------------------
# forward (moe.rs:65-109, mlp.rs:42-46)
# --------------------------------------------------------------------------

def _params(seed, E, D, H, bias=True, scale=1.0):
    rng = np.random.default_rng(seed)
    f = lambda *s: (rng.standard_normal(s) * scale).astype(np.float32)  # noqa: E731
    p = {"wr": f(E, D) * np.float32(0.3),
         "wg": f(E, H, D) / np.float32(math.sqrt(D)), "wu": f(E, H, D) / np.float32(math.sqrt(D)),
         "wd": f(E, D, H) / np.float32(math.sqrt(H))}
    if bias:
        p.update(bg=f(E, H) * np.float32(0.1), bu=f(E, H) * np.float32(0.1), bd=f(E, D) * np.float32(0.1))
    else:
        p.update(bg=None, bu=None, bd=None)
    return p


def _torch_ffn(x, wg, bg, wu, bu, wd, bd):
    """down(silu(gate x) * up x) with torch float64 (mlp.rs:42-46)."""
    t = lambda a: None if a is None else torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    xt = t(x)
    g = xt @ t(wg).T + (0 if bg is None else t(bg))
    u = xt @ t(wu).T + (0 if bu is None else t(bu))
    y = (torch.nn.functional.silu(g) * u) @ t(wd).T + (0 if bd is None else t(bd))
    return y.numpy()


def _torch_moe(x, p, k):
    idx, w, _ = _np_route(x, p["wr"], k)
    out = np.zeros((x.shape[0], x.shape[1]))
    for r in range(x.shape[0]):
        for j in range(k):
            e = idx[r, j]
            y = _torch_ffn(x[r:r + 1], p["wg"][e], None if p["bg"] is None else p["bg"][e],
                           p["wu"][e], None if p["bu"] is None else p["bu"][e],
                           p["wd"][e], None if p["bd"] is None else p["bd"][e])
            out[r] += w[r, j] * y[0]
    return out


def pin_forward_bruteforce():
    for (T, D, E, k, H) in [(24, 20, 5, 2, 28), (10, 16, 4, 3, 12)]:
        p = _params(11, E, D, H)
        x = np.random.default_rng(12).standard_normal((T, D)).astype(np.float32)
        got, idx, w, _ = O.forward_sparse(x, p, k)
        want = _torch_moe(x, p, k)
        np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)


def _fmaf(a, b, c):
    """f32 fused multiply-add: a*b + c with one rounding (the f32 product is
    exact in x86 long double, and the sum is rounded to 64 bits first, which
    changes the f32 result only on an exact double-rounding midpoint)."""
    ld = np.longdouble
    return (np.asarray(a, ld) * np.asarray(b, ld) + np.asarray(c, ld)).astype(np.float32)


def _rounded_moe(x, p, k, dt):
    """The GPU path's storage roundings, from numpy f64 GEMMs: h and y stored in
    dt (via f32), the combine an f32 FMA per slot in ascending expert order,
    the output rounded to dt."""
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dt]

    def st(v):
        return torch.from_numpy(np.asarray(v, np.float64).astype(np.float32)).to(tdt).float().numpy()

    idx, w, _ = _np_route(x, p["wr"], k)
    x64 = x.astype(np.float64)
    out = np.zeros(x.shape, np.float32)
    for r in range(x.shape[0]):
        acc = np.zeros(x.shape[1], np.float32)
        for j in range(k):
            e = idx[r, j]
            g = p["wg"][e].astype(np.float64) @ x64[r] + p["bg"][e]
            u = p["wu"][e].astype(np.float64) @ x64[r] + p["bu"][e]
            a = st(g / (1.0 + np.exp(-g)) * u)
            y = st(p["wd"][e].astype(np.float64) @ a.astype(np.float64) + p["bd"][e])
            acc = _fmaf(y, np.float32(w[r, j]), acc)
        out[r] = st(acc)
    return out


def pin_forward_rounded_bruteforce():
    # orc_forward_sparse_rounded: the same roundings, written independently
    for (T, D, E, k, H) in [(24, 20, 5, 2, 28), (10, 16, 4, 3, 12)]:
        p = _params(13, E, D, H)
        x = np.random.default_rng(14).standard_normal((T, D)).astype(np.float32)
        for dt in ("f32", "bf16", "f16"):
            got = O.forward_sparse_rounded(x, p, k, dt)
            np.testing.assert_array_equal(got.astype(np.float32), _rounded_moe(x, p, k, dt))
            assert np.array_equal(got, O.round_dt(got.astype(np.float32), dt))
        # with f32 storage it is the f64 forward to within f32 rounding
        ref, _, _, _ = O.forward_sparse(x, p, k)
        f32 = O.forward_sparse_rounded(x, p, k, "f32")
        assert np.max(np.abs(f32 - ref)) <= 1e-6 * np.max(np.abs(ref))


def pin_route_model_dtype_structure():
    # orc_route_model_dtype: its candle-specific rounding is unpinned, but its
    # structure is not: in f32 it chooses the f64 routing's experts (the
    # random logits here have no near ties), exact ties go to the lowest
    # index, and the gates sum to one in the model dtype
    rng = np.random.default_rng(21)
    for (T, D, E, k) in [(300, 64, 8, 2), (200, 48, 16, 5)]:
        x = rng.standard_normal((T, D)).astype(np.float32)
        wr = (rng.standard_normal((E, D)) * 0.3).astype(np.float32)
        i64, _, _, gap = O.route(x, wr, k)
        i32, w32 = O.route_model_dtype(x, wr, k, "f32")
        ok = gap > 1e-4
        np.testing.assert_array_equal(i32[ok], i64[ok])
        np.testing.assert_allclose(w32.sum(axis=1), 1.0, atol=1e-5)
        xb, wb = O.round_bf16(x), O.round_bf16(wr)
        wb[3] = wb[1]  # experts 1 and 3 always tie exactly
        ib, gb = O.route_model_dtype(xb, wb, k, "bf16")
        assert not ((ib == 3).any(axis=1) & ~(ib == 1).any(axis=1)).any()
        assert np.array_equal(gb, O.round_bf16(gb))
        np.testing.assert_allclose(gb.astype(np.float64).sum(axis=1), 1.0, atol=2e-2)


def pin_dense_equals_sparse():
    # the reference's dense evaluation (moe.rs:97-102) equals the sparse one
    p = _params(13, 6, 32, 48)
    x = np.random.default_rng(14).standard_normal((40, 32)).astype(np.float32)
    dense = O.forward_dense_f32(x, p, 2)
    sparse, _, _, _ = O.forward_sparse(x, p, 2)
    assert np.max(np.abs(dense - sparse)) <= 1e-5 * np.max(np.abs(sparse))


def pin_k_equals_experts():
    # k = E: out = sum_e softmax(logits)_e * FFN_e(x), no selection at all
    E, D, H = 4, 12, 20
    p = _params(15, E, D, H)
    x = np.random.default_rng(16).standard_normal((9, D)).astype(np.float32)
    got, idx, _, _ = O.forward_sparse(x, p, E)
    logits = x.astype(np.float64) @ p["wr"].astype(np.float64).T
    sm = torch.softmax(torch.from_numpy(logits), dim=1).numpy()
    want = sum(sm[:, e:e + 1] / (1 + 1e-9) * _torch_ffn(x, p["wg"][e], p["bg"][e], p["wu"][e],
                                                         p["bu"][e], p["wd"][e], p["bd"][e])
               for e in range(E))
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)


def pin_single_dominant_expert():
    # one router row far above the others: top-1 picks it with weight 1
    E, D, H = 5, 10, 14
    p = _params(17, E, D, H)
    x = np.abs(np.random.default_rng(18).standard_normal((7, D))).astype(np.float32) + 0.5
    p["wr"][2] = 50.0
    got, idx, w, _ = O.forward_sparse(x, p, 1)
    assert (idx[:, 0] == 2).all()
    want = _torch_ffn(x, p["wg"][2], p["bg"][2], p["wu"][2], p["bu"][2], p["wd"][2], p["bd"][2])
    np.testing.assert_allclose(got, want / (1 + 1e-9), rtol=1e-10, atol=1e-12)


def pin_zero_input_zero_output():
    # zero input with zero biases gives an exactly zero output (mlp.rs:89-105 analogue)
    p = _params(19, 4, 8, 16, bias=False)
    got, _, _, _ = O.forward_sparse(np.zeros((3, 8), np.float32), p, 2)
    assert np.all(got == 0.0)


def pin_row_permutation():
    p = _params(20, 4, 16, 24)
    x = np.random.default_rng(21).standard_normal((12, 16)).astype(np.float32)
    perm = np.random.default_rng(22).permutation(12)
    a, _, _, _ = O.forward_sparse(x, p, 2)
    b, _, _, _ = O.forward_sparse(x[perm], p, 2)
    np.testing.assert_array_equal(a[perm], b)


def pin_shared_dense_branch():
    # moe.rs:103-106: out += s * dense(x), added after the experts
    E, D, H = 4, 12, 16
    p = _params(23, E, D, H)
    dn = {k: v[0] for k, v in _params(24, 1, D, H).items() if k != "wr"}
    x = np.random.default_rng(25).standard_normal((6, D)).astype(np.float32)
    base, _, _, _ = O.forward_sparse(x, p, 2)
    got, _, _, _ = O.forward_sparse(x, p, 2, shared_dense=0.75, dense=dn)
    want = base + 0.75 * _torch_ffn(x, dn["wg"], dn["bg"], dn["wu"], dn["bu"], dn["wd"], dn["bd"])
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)


def pin_ffn_bruteforce():
    # FeedForward::SwiGlu (mlp.rs:39-48) against an independent torch f64 evaluation
    D, H = 20, 28
    f = {k: v[0] for k, v in _params(31, 1, D, H).items() if k != "wr"}
    x = np.random.default_rng(32).standard_normal((9, D)).astype(np.float32)
    want = _torch_ffn(x, f["wg"], f["bg"], f["wu"], f["bu"], f["wd"], f["bd"])
    np.testing.assert_allclose(O.ffn(x, f), want, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(O.ffn(x, f, rows=[7, 2]), want[[7, 2]], rtol=1e-10, atol=1e-12)


def pin_ffn_equals_single_expert():
    # one expert, top-1: every row routed with gate p / (p + 1e-9), p = 1
    D, H = 12, 16
    p = _params(33, 1, D, H)
    f = {k: v[0] for k, v in p.items() if k != "wr"}
    x = np.random.default_rng(34).standard_normal((5, D)).astype(np.float32)
    moe, idx, w, _ = O.forward_sparse(x, p, 1)
    assert (idx == 0).all()
    np.testing.assert_allclose(w, 1.0 / (1.0 + 1e-9), rtol=0, atol=1e-15)
    np.testing.assert_allclose(O.ffn(x, f), moe * (1.0 + 1e-9), rtol=1e-12, atol=1e-14)


# --------------------------------------------------------------------------
# block seams: norm2 + modulate (norm.rs:55-65, modulate.rs:69-79) and the
# gated residual (block.rs:101)
# --------------------------------------------------------------------------

def pin_f16_rounding():
    # numpy's float16 cast is round-to-nearest-even with subnormals and overflow
    rng = np.random.default_rng(8)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(2.0) ** rng.integers(
            -30, 18, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.9, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                  np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(O.round_f16(x), want)
    assert np.isnan(O.round_f16(np.array([np.nan], np.float32))).all()


def pin_modulate_formula():
    # the reference's modulate_formula test (modulate.rs:85-99): x = ones(1,3,4),
    # shift [1,0,0,0], scale [0,1,0,0] -> token 0 [2,2,1,1], token 1 col 0 = 2.
    # eps = 0 makes the norm of a row of ones exactly 1.
    h, inv = O.norm_modulate(np.ones((3, 4), np.float32), np.array([[1, 0, 0, 0]], np.float32),
                             np.array([[0, 1, 0, 0]], np.float32), seq=3, eps=0.0)
    assert (inv == 1.0).all()
    np.testing.assert_array_equal(h, np.tile(np.array([2, 2, 1, 1], np.float32), (3, 1)))


def pin_rms_norm_unit_variance():
    # norm.rs:80-92: RmsNorm::no_affine(16, 1e-6) on deterministic_randn([2,5,16], 7)
    # gives rows of mean square 1 within 1e-3 (modulate with zero shift/scale is
    # the identity)
    x = O.randn_affine(7, 2 * 5 * 16).reshape(10, 16)
    z = np.zeros((2, 16), np.float32)
    h, _ = O.norm_modulate(x, z, z, seq=5, eps=1e-6)
    ms = (h.astype(np.float64) ** 2).mean(axis=1)
    assert np.abs(ms - 1.0).max() < 1e-3, ms


def pin_zero_row_stays_finite():
    # norm.rs:94-106: a zero row normalises to zeros (inv = eps^-1/2)
    z = np.zeros((1, 8), np.float32)
    sh = np.arange(8, dtype=np.float32)[None] * np.float32(0.25)
    h, inv = O.norm_modulate(z, sh, np.ones((1, 8), np.float32), seq=1, eps=1e-6)
    assert np.isfinite(h).all() and np.isfinite(inv).all()
    np.testing.assert_array_equal(h, sh)  # 0 * (1 + 1) + shift
    assert abs(inv[0] - 1000.0) <= 1e-3


def _seam_case(seed, rows, D, seq):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, D)).astype(np.float32) * np.float32(1.7)
    nb = rows // seq
    return (x, rng.standard_normal(D).astype(np.float32),
            (rng.standard_normal((nb, D)) * 0.5).astype(np.float32),
            (rng.standard_normal((nb, D)) * 0.5).astype(np.float32))


def pin_norm_modulate_f32_vs_float64():
    # f32 model: every step is an f32 op, so h is the exact f64 formula within a
    # few f32 ulps (the sequential f32 sum of D squares is the largest term)
    x, w, sh, sc = _seam_case(9, 12, 256, 4)
    h, inv = O.norm_modulate(x, sh, sc, seq=4, norm_w=w, eps=1e-6, dt="f32")
    xd = x.astype(np.float64)
    inv_ref = 1.0 / np.sqrt((xd ** 2).mean(axis=1) + 1e-6)
    np.testing.assert_allclose(inv, inv_ref, rtol=2e-6)
    b = np.arange(12) // 4
    ref = xd * inv_ref[:, None] * w * (1.0 + sc[b]) + sh[b]
    np.testing.assert_allclose(h, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def pin_norm_modulate_bf16_vs_torch():
    # the same op sequence as torch bf16 tensor ops (torch's own reductions and
    # roundings): elements agree bit for bit except where torch's differently
    # ordered sum moves inv across a bf16 rounding edge (one ulp apart)
    for dt, tdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        x, w, sh, sc = _seam_case(10, 64, 512, 16)
        xt = torch.from_numpy(x).to(tdt)
        xm = xt.float().numpy()
        h, _ = O.norm_modulate(xm, sh, sc, seq=16, norm_w=w, eps=1e-6, dt=dt)
        f = xt.float()
        inv = (f.pow(2).mean(-1, keepdim=True) + 1e-6).pow(-0.5)
        n = (f * inv * torch.from_numpy(w)).to(tdt).float()
        b = torch.arange(64) // 16
        opl = torch.from_numpy(sc)[b] + 1.0
        m = (n * opl + torch.from_numpy(sh)[b]).to(tdt).float()
        eq = (h == m.numpy()).mean()
        # an ulp of n carried through (1 + scale), plus an ulp of h
        u = 2.0 ** -7 if dt == "bf16" else 2.0 ** -10
        bound = (u * ((n * opl).abs() + m.abs())).numpy()
        assert eq >= 0.995 and (np.abs(h - m.numpy()) <= bound).all(), (dt, eq)


def pin_pow_modes_agree():
    # libm powf against correctly rounded square / root: the same bits except
    # where powf's result lands within its error bound of a midpoint
    x, w, sh, sc = _seam_case(11, 200, 384, 50)
    for dt in ("f32", "bf16"):
        xm = O.round_dt(x, dt)
        h0, i0 = O.norm_modulate(xm, sh, sc, 50, w, 1e-6, dt, pow_mode=0)
        h1, i1 = O.norm_modulate(xm, sh, sc, 50, w, 1e-6, dt, pow_mode=1)
        assert (i0 == i1).mean() >= 0.99
        assert (np.abs(i0.view(np.int32) - i1.view(np.int32)) <= 1).all()


def pin_gated_residual_closed_forms():
    rng = np.random.default_rng(12)
    for dt, tdt in (("f32", torch.float32), ("bf16", torch.bfloat16), ("f16", torch.float16)):
        x = O.round_dt(rng.standard_normal((6, 32)).astype(np.float32), dt)
        y = O.round_dt(rng.standard_normal((6, 32)).astype(np.float32), dt)
        zero, one = np.zeros((2, 32), np.float32), np.ones((2, 32), np.float32)
        np.testing.assert_array_equal(O.gated_residual(x, y, zero, 3, dt), x)
        # gate 1: the model dtype's own addition
        want = (torch.from_numpy(x).to(tdt) + torch.from_numpy(y).to(tdt)).float().numpy()
        np.testing.assert_array_equal(O.gated_residual(x, y, one, 3, dt), want)
        # gate 2: doubling is exact, so x + 2y rounds once
        want2 = (torch.from_numpy(x).to(tdt) + 2 * torch.from_numpy(y).to(tdt)).float().numpy()
        np.testing.assert_array_equal(O.gated_residual(x, y, 2 * one, 3, dt), want2)


PINS = [pin_splitmix64, pin_fnv1a, pin_box_muller, pin_affine_and_moments, pin_uniform,
        pin_xavier_std,
        pin_bf16_rounding, pin_route_bruteforce, pin_route_ties_lowest_index,
        pin_route_one_hot_rows, pin_route_weights_sum_to_one, pin_forward_bruteforce,
        pin_forward_rounded_bruteforce, pin_route_model_dtype_structure,
        pin_dense_equals_sparse, pin_k_equals_experts, pin_single_dominant_expert,
        pin_zero_input_zero_output, pin_row_permutation, pin_shared_dense_branch,
        pin_ffn_bruteforce, pin_ffn_equals_single_expert,
        pin_f16_rounding, pin_modulate_formula, pin_rms_norm_unit_variance,
        pin_zero_row_stays_finite, pin_norm_modulate_f32_vs_float64,
        pin_norm_modulate_bf16_vs_torch, pin_pow_modes_agree, pin_gated_residual_closed_forms]


@pytest.mark.parametrize("pin", PINS, ids=[p.__name__ for p in PINS])
def test_pin(pin):
    O.set_mutation(0)
    pin()


@pytest.mark.parametrize("name", sorted(O.MUTATIONS))
def test_each_planted_mistake_is_caught(name):
    failed = []
    try:
        O.set_mutation(O.MUTATIONS[name])
        for pin in PINS:
            try:
                pin()
            except AssertionError:
                failed.append(pin.__name__)
    finally:
        O.set_mutation(0)
    assert failed, f"no pin detects the planted mistake {name!r}"
