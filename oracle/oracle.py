"""ctypes view of the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by the tests, the smoke check and the
CPU-baseline leg of ``bench.py``, never by the product package.  The C source
(``moe_oracle.c``) restates hy-nomas-rs's generator (tensor_utils.rs:65-162,
modules/mod.rs:47-55), ``MoeLayer::forward`` (modules/moe.rs:65-109,
modules/mlp.rs:42-46) and the FFN seams of ``DiTBlock::forward``
(modules/block.rs:96,101, modules/norm.rs:55-65, modules/modulate.rs:69-79);
this module only marshals numpy arrays.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# NOMAS_ORACLE_LIB selects another build (the sanitizer build, liboracle_san.so)
_LIB_PATH = os.environ.get("NOMAS_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")


def build() -> None:
    """Compile liboracle.so with gcc (make)."""
    subprocess.run(["make", "-B", "-C", _HERE], check=True, stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = C.CDLL(_LIB_PATH)
    L.orc_splitmix64_next.restype = C.c_uint64
    L.orc_splitmix64_next.argtypes = [C.POINTER(C.c_uint64)]
    L.orc_path_seed.restype = C.c_uint64
    L.orc_path_seed.argtypes = [C.c_uint64, C.c_char_p]
    L.orc_randn_affine.restype = None
    L.orc_randn_affine.argtypes = [C.c_uint64, C.c_double, C.c_double, C.c_int64, _f32p]
    L.orc_uniform.restype = None
    L.orc_uniform.argtypes = [C.c_uint64, C.c_double, C.c_double, C.c_int64, _f32p]
    L.orc_xavier.restype = None
    L.orc_xavier.argtypes = [C.c_int64, C.c_int64, C.c_uint64, _f32p]
    L.orc_round_bf16.restype = None
    L.orc_round_bf16.argtypes = [_f32p, C.c_int64]
    L.orc_route_f64.restype = None
    L.orc_route_f64.argtypes = [C.c_int64] * 4 + [_f32p, _f32p, C.c_void_p, C.c_void_p,
                                                 C.c_void_p, C.c_void_p]
    L.orc_forward_sparse_f64.restype = None
    L.orc_forward_sparse_f64.argtypes = (
        [C.c_int64] * 4 + [C.c_void_p] * 8 + [C.c_double] + [C.c_void_p] * 6
        + [C.c_void_p, C.c_int64, _f64p, C.c_void_p, C.c_void_p, C.c_void_p])
    L.orc_forward_sparse_rounded.restype = None
    L.orc_forward_sparse_rounded.argtypes = (
        [C.c_int64] * 4 + [C.c_void_p] * 8 + [C.c_double] + [C.c_void_p] * 6
        + [C.c_void_p, C.c_int64, _f64p, C.c_int])
    L.orc_route_model_dtype.restype = None
    L.orc_route_model_dtype.argtypes = [C.c_int64] * 4 + [_f32p, _f32p, C.c_int, C.c_void_p,
                                                          C.c_void_p]
    L.orc_ffn_f64.restype = None
    L.orc_ffn_f64.argtypes = [C.c_int64] * 2 + [C.c_void_p] * 7 + [C.c_void_p, C.c_int64, _f64p]
    L.orc_forward_dense_f32.restype = C.c_int
    L.orc_forward_dense_f32.argtypes = (
        [C.c_int64] * 5 + [C.c_void_p] * 8 + [C.c_double] + [C.c_void_p] * 6
        + [_f32p, C.c_void_p])
    L.orc_round_f16.restype = None
    L.orc_round_f16.argtypes = [_f32p, C.c_int64]
    L.orc_norm_modulate.restype = None
    L.orc_norm_modulate.argtypes = ([C.c_int64] * 3 + [_f32p, C.c_void_p, C.c_double, _f32p, _f32p]
                                    + [C.c_int, C.c_int, _f32p, _f32p])
    L.orc_gated_residual.restype = None
    L.orc_gated_residual.argtypes = [C.c_int64] * 3 + [_f32p] * 3 + [C.c_int, _f32p]
    L.orc_num_threads.restype = C.c_int
    L.orc_set_num_threads.restype = None
    L.orc_set_num_threads.argtypes = [C.c_int]
    _lib = L
    return L


def set_mutation(m: int) -> None:
    C.c_int.in_dll(lib(), "orc_mutation").value = int(m)


MUTATIONS = {
    "boxmuller_swap": 1,
    "tie_high_index": 2,
    "no_renorm": 3,
    "swap_gate_up": 4,
    "drop_down_bias": 5,
    "down_transposed": 6,
    "fnv_prime": 7,
    "splitmix_shift": 8,
    "modulate_no_one": 9,
    "var_d_minus_1": 10,
    "norm_no_round": 11,
    "ungated_residual": 12,
    "h_unrounded": 13,
    "combine_unfused": 14,
}

# Faults of the GPU path simulated in the oracle (not oracle mistakes): the
# parity tests offer their output as if it were the GPU's, to show which bar
# rejects it.
KERNEL_FAULTS = {
    "gate_up_loses_fragment": 15,
}


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def splitmix64(seed: int, n: int) -> list[int]:
    st = C.c_uint64(seed)
    return [lib().orc_splitmix64_next(C.byref(st)) for _ in range(n)]


def path_seed(seed: int, path: str) -> int:
    return lib().orc_path_seed(seed, path.encode())


def randn_affine(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_randn_affine(seed, mean, std, n, out)
    return out


def uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_uniform(seed, lo, hi, n, out)
    return out


def xavier(out_f: int, in_f: int, seed: int) -> np.ndarray:
    out = np.empty(out_f * in_f, np.float32)
    lib().orc_xavier(out_f, in_f, seed, out)
    return out.reshape(out_f, in_f)


def round_bf16(a: np.ndarray) -> np.ndarray:
    out = np.array(a, dtype=np.float32, copy=True, order="C")
    lib().orc_round_bf16(out, out.size)
    return out


def round_f16(a: np.ndarray) -> np.ndarray:
    out = np.array(a, dtype=np.float32, copy=True, order="C")
    lib().orc_round_f16(out, out.size)
    return out


DT_CODE = {"f32": 0, "bf16": 1, "f16": 2}


def round_dt(a: np.ndarray, dt: str) -> np.ndarray:
    """Round f32 values to the model dtype, widened back to f32."""
    return {"f32": lambda v: np.array(v, np.float32), "bf16": round_bf16, "f16": round_f16}[dt](a)


def norm_modulate(x, shift, scale, seq, norm_w=None, eps=1e-6, dt="f32", pow_mode=0):
    """h = modulate(norm2(x), shift, scale) (norm.rs:55-65, modulate.rs:69-79).

    x: (rows, D) values of the model dtype (as f32); shift / scale (rows/seq, D).
    Returns (h (rows, D) f32 holding model-dtype values, inv_rms (rows,)).
    pow_mode 0: libm powf as the reference; 1: correctly rounded square and root.
    """
    x = _f32(x)
    rows, D = x.shape
    h = np.empty_like(x)
    inv = np.empty(rows, np.float32)
    nw = _f32(norm_w)
    lib().orc_norm_modulate(rows, D, int(seq), x, _ptr(nw), float(eps), _f32(shift),
                            _f32(scale), DT_CODE[dt], int(pow_mode), h, inv)
    return h, inv


def gated_residual(x, y, gate, seq, dt="f32"):
    """out = x + y * gate (block.rs:101), each op rounded to the model dtype."""
    x, y = _f32(x), _f32(y)
    out = np.empty_like(x)
    lib().orc_gated_residual(x.shape[0], x.shape[1], int(seq), x, y, _f32(gate), DT_CODE[dt], out)
    return out


def block_ffn(x, p, k, shift, scale, gate, seq, norm_w=None, eps=1e-6, dt="f32", pow_mode=0,
              shared_dense=0.0, dense=None):
    """The FFN half of DiTBlock::forward around the MoE (block.rs:96-101):
    returns (out (rows, D) f32 in the model dtype, h, idx, gap), the MoE in f64
    (forward_sparse) with its output rounded to the model dtype."""
    h, _ = norm_modulate(x, shift, scale, seq, norm_w, eps, dt, pow_mode)
    y, idx, _, gap = forward_sparse(h, p, k, shared_dense=shared_dense, dense=dense)
    y_dt = round_dt(y.astype(np.float32), dt)
    return gated_residual(x, y_dt, gate, seq, dt), h, idx, gap


def route(x, wr, k):
    """f64 routing of every row: (idx[T,k] ascending expert, w[T,k], logits[T,E], gap[T])."""
    x, wr = _f32(x), _f32(wr)
    T, D = x.shape
    E = wr.shape[0]
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float64)
    logits = np.empty((T, E), np.float64)
    gap = np.empty(T, np.float64)
    lib().orc_route_f64(T, D, E, k, x, wr, _ptr(idx), _ptr(w), _ptr(logits), _ptr(gap))
    return idx, w, logits, gap


def route_model_dtype(x, wr, k, dt):
    """Routing op by op in the model dtype as candle evaluates moe.rs:67-95
    (PARITY UNPINNED: a restatement of candle's per-op rounding that no
    reference output checks).  x, wr hold values of dt.  Returns (idx[T,k]
    ascending, w[T,k] f32)."""
    x, wr = _f32(x), _f32(wr)
    T, D = x.shape
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    lib().orc_route_model_dtype(T, D, wr.shape[0], k, x, wr, DT_CODE[dt], _ptr(idx), _ptr(w))
    return idx, w


def forward_sparse(x, p, k, rows=None, shared_dense=0.0, dense=None):
    """f64 MoE forward of the given rows (all rows when None).

    ``p`` holds f32 arrays in the reference layout: wr (E,D), wg/wu (E,H,D),
    bg/bu (E,H), wd (E,D,H), bd (E,D).  ``dense`` optionally holds the shared
    dense FFN as wg (H,D), bg, wu, bu, wd (D,H), bd.
    Returns (out[n,D] f64, idx[n,k], w[n,k], gap[n]).
    """
    x = _f32(x)
    T, D = x.shape
    E, H = p["wg"].shape[0], p["wg"].shape[1]
    arrs = [_f32(p.get(n)) for n in ("wr", "wg", "bg", "wu", "bu", "wd", "bd")]
    dn = [None] * 6 if dense is None else [_f32(dense.get(n)) for n in
                                           ("wg", "bg", "wu", "bu", "wd", "bd")]
    if rows is None:
        rows_a, n = None, T
    else:
        rows_a = np.ascontiguousarray(rows, dtype=np.int64)
        n = rows_a.size
    out = np.empty((n, D), np.float64)
    idx = np.empty((n, k), np.int32)
    w = np.empty((n, k), np.float64)
    gap = np.empty(n, np.float64)
    lib().orc_forward_sparse_f64(D, E, k, H, _ptr(x), *[_ptr(a) for a in arrs],
                                 float(shared_dense), *[_ptr(a) for a in dn],
                                 _ptr(rows_a), n, out, _ptr(idx), _ptr(w), _ptr(gap))
    return out, idx, w, gap


def forward_sparse_rounded(x, p, k, dt, rows=None, shared_dense=0.0, dense=None):
    """forward_sparse with the GPU path's storage roundings (dt "f32" / "bf16" /
    "f16"): the SwiGLU intermediate and each expert's output held in the model
    dtype, the combine an f32 fused multiply-add per slot in ascending expert
    order, the output rounded to dt.  Returns out[n,D] f64 (values of dt)."""
    x = _f32(x)
    T, D = x.shape
    E, H = p["wg"].shape[0], p["wg"].shape[1]
    arrs = [_f32(p.get(n)) for n in ("wr", "wg", "bg", "wu", "bu", "wd", "bd")]
    dn = [None] * 6 if dense is None else [_f32(dense.get(n)) for n in
                                           ("wg", "bg", "wu", "bu", "wd", "bd")]
    if rows is None:
        rows_a, n = None, T
    else:
        rows_a = np.ascontiguousarray(rows, dtype=np.int64)
        n = rows_a.size
    out = np.empty((n, D), np.float64)
    lib().orc_forward_sparse_rounded(D, E, k, H, _ptr(x), *[_ptr(a) for a in arrs],
                                     float(shared_dense), *[_ptr(a) for a in dn],
                                     _ptr(rows_a), n, out, DT_CODE[dt])
    return out


def ffn(x, f, rows=None):
    """f64 dense SwiGLU feed-forward (mlp.rs:39-48) of the given rows (all when None).

    ``f`` holds f32 arrays in the reference layout: wg, wu (H,D), bg, bu (H,),
    wd (D,H), bd (D,); missing biases are zero.  Returns out[n,D] f64.
    """
    x = _f32(x)
    T, D = x.shape
    H = f["wg"].shape[0]
    arrs = [_f32(f.get(n)) for n in ("wg", "bg", "wu", "bu", "wd", "bd")]
    if rows is None:
        rows_a, n = None, T
    else:
        rows_a = np.ascontiguousarray(rows, dtype=np.int64)
        n = rows_a.size
    out = np.empty((n, D), np.float64)
    lib().orc_ffn_f64(D, H, _ptr(x), *[_ptr(a) for a in arrs], _ptr(rows_a), n, out)
    return out


def forward_dense_f32(x, p, k, shared_dense=0.0, dense=None, return_weights=False):
    """The reference algorithm in f32: every expert on every row (CPU baseline)."""
    x = _f32(x)
    T, D = x.shape
    E, H = p["wg"].shape[0], p["wg"].shape[1]
    arrs = [_f32(p.get(n)) for n in ("wr", "wg", "bg", "wu", "bu", "wd", "bd")]
    dn = [None] * 6 if dense is None else [_f32(dense.get(n)) for n in
                                           ("wg", "bg", "wu", "bu", "wd", "bd")]
    out = np.empty((T, D), np.float32)
    wd = np.empty((T, E), np.float32) if return_weights else None
    rc = lib().orc_forward_dense_f32(T, D, E, k, H, _ptr(x), *[_ptr(a) for a in arrs],
                                     float(shared_dense), *[_ptr(a) for a in dn], out, _ptr(wd))
    if rc != 0:
        raise MemoryError("oracle dense forward could not allocate its scratch")
    return (out, wd) if return_weights else out


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(n)
