"""MI355X top-k MoE feed-forward block with hy-nomas-rs's module interface.

Mirrors the reference's Rust API (nomas-core/src/modules/moe.rs,
nomas-core/src/config.rs:202-213, nomas-core/src/modules/mod.rs:20-56):

    cfg = MoeConfig(experts=4, top_k=2, shared_dense=0.0, seed=1)
    moe = MoeLayer.from_source(Weights.random(4, DataType.F32), "blocks.0.moe", 32, 64, cfg)
    y = moe.forward(x)          # x: (..., D) torch tensor on the GPU or the host
    moe.n_params()

Every computation runs in libnomas_moe.so (hand-written gfx950 kernels behind
a C ABI); this module only marshals arguments.  Errors raise NomasError
subclasses that mirror the reference's error variants (error.rs:7-46).
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import Mapping, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import nomas_moe_config

__all__ = [
    "DataType", "MoeConfig", "Weights", "MoeLayer", "FeedForward", "NomasError", "InvalidConfig",
    "WeightKey", "IoError", "path_seed", "randn_affine", "to_model_dtype", "norm_modulate",
    "gated_residual",
]


class DataType(enum.IntEnum):
    """config.rs:30-39."""
    F32 = 0
    Bf16 = 1
    F16 = 2

    @property
    def torch(self) -> torch.dtype:
        return {0: torch.float32, 1: torch.bfloat16, 2: torch.float16}[int(self)]

    @classmethod
    def of(cls, dt) -> "DataType":
        if isinstance(dt, DataType):
            return dt
        if isinstance(dt, torch.dtype):
            return {torch.float32: cls.F32, torch.bfloat16: cls.Bf16, torch.float16: cls.F16}[dt]
        return {"f32": cls.F32, "bf16": cls.Bf16, "f16": cls.F16}[str(dt).lower()]


def _check_out(out: torch.Tensor, like: torch.Tensor, what: str = "out") -> torch.Tensor:
    """A caller-supplied output must be exactly what the kernels write: x's
    shape and dtype, contiguous, and on the same side (the same GPU for a
    device x, the host for a host x).  Checked before any call into the
    library, so a bad buffer is an error instead of an out-of-bounds write."""
    if not isinstance(out, torch.Tensor):
        raise NomasError(2, f"{what} must be a torch.Tensor, got {type(out).__name__}")
    if tuple(out.shape) != tuple(like.shape):
        raise NomasError(2, f"{what}: expected shape {tuple(like.shape)}, got {tuple(out.shape)}")
    if out.dtype != like.dtype:
        raise NomasError(2, f"{what}: expected dtype {like.dtype}, got {out.dtype}")
    if not out.is_contiguous():
        raise NomasError(2, f"{what} must be contiguous")
    if out.device != like.device:
        raise NomasError(2, f"{what} is on {out.device}, the input on {like.device}")
    return out


def _new_output(xc):
    """An output like xc: on the GPU for a GPU input; pinned for a host input,
    so that the result is copied straight back (torch caches pinned blocks)."""
    if not xc.is_cuda and torch.cuda.is_available():
        return torch.empty(xc.shape, dtype=xc.dtype, pin_memory=True)
    return torch.empty_like(xc)


class NomasError(RuntimeError):
    """A failed call into the library; ``code`` is the nomas_status value."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class InvalidConfig(NomasError):
    """Error::InvalidConfig (error.rs:24-26)."""


class WeightKey(NomasError):
    """Error::WeightKey (error.rs:20-22)."""


class IoError(NomasError):
    """A checkpoint that cannot be read or parsed: the reference's
    Error::Msg("loading {path}: {e}") (weights.rs:112-115), same message form."""


_ERRORS = {1: InvalidConfig, 3: WeightKey, 4: IoError}


def _check(rc: int) -> None:
    if rc != 0:
        raise _ERRORS.get(rc, NomasError)(rc, _lib.last_error())


@dataclass
class MoeConfig:
    """MoeConfig (config.rs:202-213)."""
    experts: int
    top_k: int
    shared_dense: float = 0.0
    seed: int = 0

    def _c(self) -> nomas_moe_config:
        return nomas_moe_config(int(self.experts), int(self.top_k), float(self.shared_dense),
                                int(self.seed) & 0xFFFFFFFFFFFFFFFF)

    def validate(self) -> None:
        """The MoE clause of NomasConfig::validate (config.rs:394-399)."""
        c = self._c()
        _check(_lib.lib().nomas_moe_config_validate(C.byref(c)))


def path_seed(seed: int, path: str) -> int:
    """Weights::path_seed (mod.rs:47-55)."""
    return int(_lib.lib().nomas_path_seed(seed & 0xFFFFFFFFFFFFFFFF, path.encode()))


def randn_affine(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """deterministic_randn_affine (tensor_utils.rs:123-138), flattened, f32."""
    out = np.empty(int(n), np.float32)
    _lib.lib().nomas_randn_affine(seed & 0xFFFFFFFFFFFFFFFF, float(mean), float(std), int(n),
                                  out.ctypes.data)
    return out


def to_model_dtype(a: np.ndarray, dtype) -> np.ndarray:
    """f32 array -> raw storage of the model dtype (round to nearest even):
    float32 for F32, uint16 bit patterns for Bf16 / F16."""
    dt = DataType.of(dtype)
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dt == DataType.F32:
        return a
    out = np.empty(a.shape, np.uint16)
    fn = _lib.lib().nomas_f32_to_bf16 if dt == DataType.Bf16 else _lib.lib().nomas_f32_to_f16
    fn(a.ctypes.data, out.ctypes.data, a.size)
    return out


def widen(a: np.ndarray, dtype) -> np.ndarray:
    """Raw model-dtype storage -> f32 values (exact)."""
    dt = DataType.of(dtype)
    if dt == DataType.F32:
        return np.asarray(a, np.float32)
    if dt == DataType.Bf16:
        return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float32)


def _seam_params(x: torch.Tensor, named) -> list:
    """(B, D) AdaLN parameters (and an optional (D,) gain) as contiguous f32 on x's device."""
    B, _, D = x.shape
    out = []
    for name, t, shape in named:
        if t is None:
            out.append(None)
            continue
        if tuple(t.shape) != shape(B, D):
            raise NomasError(2, f"{name}: expected {shape(B, D)}, got {tuple(t.shape)}")
        out.append(t.to(device=x.device, dtype=torch.float32).contiguous())
    return out


def _seam_input(x: torch.Tensor) -> torch.Tensor:
    if x.dim() != 3:
        raise NomasError(2, f"expected (B, L, D) activations, got shape {tuple(x.shape)}")
    if not x.is_cuda:
        raise NomasError(2, "the block seams take device tensors")
    DataType.of(x.dtype)
    return x.contiguous()


def _ptr(t):
    return None if t is None else t.data_ptr()


def norm_modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                  norm_w: torch.Tensor | None = None, eps: float = 1e-6,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """h = modulate(norm2(x), shift, scale) (block.rs:96; norm.rs:55-65,
    modulate.rs:69-79).  x: (B, L, D) device tensor in f32 / bf16 / f16;
    shift / scale: (B, D); norm_w: (D,) or None (RmsNorm::no_affine)."""
    xc = _seam_input(x)
    B, S, D = xc.shape
    sh, sc, nw = _seam_params(xc, (("shift", shift, lambda b, d: (b, d)),
                                   ("scale", scale, lambda b, d: (b, d)),
                                   ("norm_w", norm_w, lambda b, d: (d,))))
    if out is None:
        out = torch.empty_like(xc)
    else:
        _check_out(out, xc)
    stream = torch.cuda.current_stream(xc.device).cuda_stream
    _check(_lib.lib().nomas_norm_modulate(int(DataType.of(xc.dtype)), xc.data_ptr(),
                                          out.data_ptr(), B * S, D, max(S, 1), _ptr(nw),
                                          float(eps), sh.data_ptr(), sc.data_ptr(), stream))
    return out


def gated_residual(x: torch.Tensor, y: torch.Tensor, gate: torch.Tensor,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """out = x + y * gate (block.rs:101).  x, y: (B, L, D) device tensors of one
    dtype; gate: (B, D)."""
    xc = _seam_input(x)
    if tuple(y.shape) != tuple(xc.shape) or y.dtype != xc.dtype or y.device != xc.device:
        raise NomasError(2, "y must match x in shape, dtype and device")
    yc = y.contiguous()
    B, S, D = xc.shape
    (g,) = _seam_params(xc, (("gate", gate, lambda b, d: (b, d)),))
    if out is None:
        out = torch.empty_like(xc)
    else:
        _check_out(out, xc)
    stream = torch.cuda.current_stream(xc.device).cuda_stream
    _check(_lib.lib().nomas_gated_residual(int(DataType.of(xc.dtype)), xc.data_ptr(),
                                           yc.data_ptr(), g.data_ptr(), out.data_ptr(), B * S, D,
                                           max(S, 1), stream))
    return out


class Weights:
    """Where a module's parameters come from (mod.rs:20-45).

    * ``Weights.random(seed, dtype)`` -- deterministic xavier init keyed by the
      parameter path, zero biases (Weights::Random).
    * ``Weights.loaded(files, dtype)`` -- safetensors checkpoint files
      (Weights::Loaded over weights::load_dit's VarBuilder).
    * ``Weights.tensors(mapping, dtype)`` -- in-memory f32 arrays keyed like
      the checkpoint (VarBuilder::from_tensors).
    """

    def __init__(self, kind: str, dtype, device: int = 0, seed: int = 0,
                 files: Sequence[str] = (), tensors: Mapping[str, np.ndarray] | None = None):
        self.kind = kind
        self.dtype = DataType.of(dtype)
        self.device = int(device)
        self.seed = int(seed)
        self.files = list(files)
        self.tensors = dict(tensors or {})

    @classmethod
    def random(cls, seed: int, dtype=DataType.F32, device: int = 0) -> "Weights":
        return cls("random", dtype, device, seed=seed)

    @classmethod
    def loaded(cls, files: Sequence[str] | str, dtype=DataType.F32, device: int = 0) -> "Weights":
        if isinstance(files, str):
            files = [files]
        return cls("loaded", dtype, device, files=files)

    @classmethod
    def tensors_(cls, tensors: Mapping[str, np.ndarray], dtype=DataType.F32,
                 device: int = 0) -> "Weights":
        return cls("tensors", dtype, device, tensors=tensors)

    # the reference names this VarBuilder::from_tensors; keep a short alias
    from_tensors = tensors_


class MoeLayer:
    """Router + expert bank (moe.rs:16-22) on one MI355X."""

    def __init__(self, handle: C.c_void_p, cfg: MoeConfig, dtype: DataType, device: int):
        self._h = handle
        self.cfg = cfg
        self.dtype = dtype
        self.device = device
        d, hdn, e, k, dt = C.c_int64(), C.c_int64(), C.c_int64(), C.c_int64(), C.c_int()
        _check(_lib.lib().nomas_moe_dims(self._h, C.byref(d), C.byref(hdn), C.byref(e),
                                         C.byref(k), C.byref(dt)))
        self.dim, self.hidden, self.experts, self.top_k = d.value, hdn.value, e.value, k.value

    # -- construction: MoeLayer::from_source (moe.rs:26-62) ------------------
    @classmethod
    def from_source(cls, src: Weights, path: str, dim: int, hidden: int,
                    cfg: MoeConfig) -> "MoeLayer":
        L = _lib.lib()
        c = cfg._c()
        h = C.c_void_p()
        if src.kind == "random":
            rc = L.nomas_moe_from_random(C.byref(c), path.encode(), dim, hidden, int(src.dtype),
                                         src.seed & 0xFFFFFFFFFFFFFFFF, src.device, C.byref(h))
        elif src.kind == "loaded":
            arr = (C.c_char_p * len(src.files))(*[f.encode() for f in src.files])
            rc = L.nomas_moe_from_safetensors(C.byref(c), arr, len(src.files), path.encode(), dim,
                                              hidden, int(src.dtype), src.device, C.byref(h))
        elif src.kind == "tensors":
            rc = cls._from_tensors(src, path, dim, hidden, cfg, c, h)
        else:
            raise ValueError(f"unknown weight source {src.kind!r}")
        _check(rc)
        return cls(h, cfg, src.dtype, src.device)

    @staticmethod
    def _from_tensors(src, path, dim, hidden, cfg, c, h) -> int:
        t = src.tensors
        E = int(cfg.experts)

        def stack(fmt, shape, bias):
            arrs = []
            for e in range(E):
                key = fmt.format(e=e)
                if key not in t:
                    if bias:
                        arrs.append(np.zeros(shape, np.float32))
                        continue
                    raise WeightKey(3, f"missing tensor {key}")
                a = np.asarray(t[key], np.float32)
                if a.shape != shape:
                    raise WeightKey(3, f"{key}: expected shape {shape}, got {a.shape}")
                arrs.append(a)
            return to_model_dtype(np.stack(arrs), src.dtype)

        def one(key, shape, required=True):
            if key not in t:
                if required:
                    raise WeightKey(3, f"missing tensor {key}")
                return None
            a = np.asarray(t[key], np.float32)
            if a.shape != shape:
                raise WeightKey(3, f"{key}: expected shape {shape}, got {a.shape}")
            return to_model_dtype(a, src.dtype)

        D, H = int(dim), int(hidden)
        ex = path + ".experts.{e}"
        keep = [
            one(f"{path}.router.weight", (E, D)),
            stack(ex + ".gate.weight", (H, D), False), stack(ex + ".gate.bias", (H,), True),
            stack(ex + ".up.weight", (H, D), False), stack(ex + ".up.bias", (H,), True),
            stack(ex + ".down.weight", (D, H), False), stack(ex + ".down.bias", (D,), True),
        ]
        if cfg.shared_dense > 0:
            dp = path + ".dense"
            keep += [one(dp + ".gate.weight", (H, D)), one(dp + ".gate.bias", (H,), False),
                     one(dp + ".up.weight", (H, D)), one(dp + ".up.bias", (H,), False),
                     one(dp + ".down.weight", (D, H)), one(dp + ".down.bias", (D,), False)]
        else:
            keep += [None] * 6
        ptrs = [None if a is None else a.ctypes.data for a in keep]
        return _lib.lib().nomas_moe_from_host(C.byref(c), D, H, int(src.dtype), src.device,
                                              *ptrs, C.byref(h))

    # -- MoeLayer::forward (moe.rs:65-109) -----------------------------------
    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """x: (..., D) in the model dtype, on the layer's GPU or on the host."""
        if x.dim() < 1 or x.shape[-1] != self.dim:
            raise NomasError(2, f"expected last dim {self.dim}, got shape {tuple(x.shape)}")
        if x.dtype != self.dtype.torch:
            raise NomasError(2, f"expected dtype {self.dtype.torch}, got {x.dtype}")
        xc = x.contiguous()
        rows = xc.numel() // self.dim
        if out is None:
            out = _new_output(xc)
        else:
            _check_out(out, xc)
        L = _lib.lib()
        if xc.is_cuda:
            stream = torch.cuda.current_stream(xc.device).cuda_stream
            _check(L.nomas_moe_forward(self._h, xc.data_ptr(), out.data_ptr(), rows, stream))
        else:
            _check(L.nomas_moe_forward_host(self._h, xc.data_ptr(), out.data_ptr(), rows))
        return out

    __call__ = forward

    # -- the FFN half of DiTBlock::forward (block.rs:96-101) ------------------
    def forward_block(self, x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                      gate: torch.Tensor, norm_w: torch.Tensor | None = None, eps: float = 1e-6,
                      out: torch.Tensor | None = None) -> torch.Tensor:
        """x + moe(modulate(norm2(x), shift, scale)) * gate: the FFN half of
        DiTBlock::forward (block.rs:96-101) around this MoE.  x: (B, L, D) in
        the model dtype on the layer's GPU; shift / scale / gate: (B, D);
        norm_w: (D,) or None (no affine gain).  out may be x (in place)."""
        xc = _seam_input(x)
        if xc.shape[-1] != self.dim or xc.dtype != self.dtype.torch:
            raise NomasError(2, f"expected (B, L, {self.dim}) {self.dtype.torch}, got "
                                f"{tuple(x.shape)} {x.dtype}")
        B, S, D = xc.shape
        sh, sc, g, nw = _seam_params(xc, (("shift", shift, lambda b, d: (b, d)),
                                          ("scale", scale, lambda b, d: (b, d)),
                                          ("gate", gate, lambda b, d: (b, d)),
                                          ("norm_w", norm_w, lambda b, d: (d,))))
        if out is None:
            out = torch.empty_like(xc)
        else:
            # in place on a strided x would compute on a copy and write the
            # contiguous result over x's strided storage: the check rejects it
            _check_out(out, xc)
        stream = torch.cuda.current_stream(xc.device).cuda_stream
        _check(_lib.lib().nomas_moe_forward_block(
            self._h, xc.data_ptr(), out.data_ptr(), B * S, max(S, 1), _ptr(nw), float(eps),
            sh.data_ptr(), sc.data_ptr(), g.data_ptr(), stream))
        return out

    def n_params(self) -> int:
        """moe.rs:112-114."""
        return int(_lib.lib().nomas_moe_n_params(self._h))

    def routing(self, rows: int):
        """Routing of the last forward: (idx[rows,k] ascending, w[rows,k], counts[E], gap[rows])."""
        k, E = self.top_k, self.experts
        idx = np.empty((rows, k), np.int32)
        w = np.empty((rows, k), np.float32)
        counts = np.empty(E, np.int32)
        gap = np.empty(rows, np.float32)
        _check(_lib.lib().nomas_moe_routing(self._h, idx.ctypes.data, w.ctypes.data,
                                            counts.ctypes.data, gap.ctypes.data))
        return idx, w, counts, gap

    def set_profiling(self, on: bool) -> None:
        _check(_lib.lib().nomas_moe_set_profiling(self._h, 1 if on else 0))

    STAGES = ("router", "scan", "dispatch", "gemm_gate_up", "gemm_down", "combine")

    def stage_times(self) -> dict:
        """Average per-stage milliseconds of the forwards profiled since the last call."""
        ms = (C.c_float * 6)()
        _check(_lib.lib().nomas_moe_stage_times(self._h, ms))
        return dict(zip(self.STAGES, [float(v) for v in ms]))

    @property
    def uses_mfma(self) -> bool:
        return bool(_lib.lib().nomas_moe_uses_mfma(self._h))

    def close(self) -> None:
        if self._h:
            _lib.lib().nomas_moe_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class FeedForward:
    """Dense SwiGLU feed-forward (FeedForward::SwiGlu, mlp.rs:9-59) on one MI355X:
    y = down(silu(gate(x)) * up(x)), on the expert GEMM kernels without routing."""

    STAGES = ("router", "tile_table", "kblock_copy", "gemm_gate_up", "gemm_down", "combine")

    def __init__(self, handle: C.c_void_p, dim: int, hidden: int, dtype: DataType, device: int):
        self._h = handle
        self.dim, self.hidden = int(dim), int(hidden)
        self.dtype = dtype
        self.device = device

    # -- FeedForward::from_source (mlp.rs:18-37), Activation::Silu -------------
    @classmethod
    def from_source(cls, src: Weights, path: str, dim: int, hidden: int) -> "FeedForward":
        L = _lib.lib()
        h = C.c_void_p()
        if src.kind == "random":
            rc = L.nomas_ffn_from_random(path.encode(), dim, hidden, int(src.dtype),
                                         src.seed & 0xFFFFFFFFFFFFFFFF, src.device, C.byref(h))
        elif src.kind == "loaded":
            arr = (C.c_char_p * len(src.files))(*[f.encode() for f in src.files])
            rc = L.nomas_ffn_from_safetensors(arr, len(src.files), path.encode(), dim, hidden,
                                              int(src.dtype), src.device, C.byref(h))
        elif src.kind == "tensors":
            t = src.tensors
            D, H = int(dim), int(hidden)

            def one(key, shape, required):
                if key not in t:
                    if required:
                        raise WeightKey(3, f"missing tensor {key}")
                    return None
                a = np.asarray(t[key], np.float32)
                if a.shape != shape:
                    raise WeightKey(3, f"{key}: expected shape {shape}, got {a.shape}")
                return to_model_dtype(a, src.dtype)

            keep = [one(f"{path}.gate.weight", (H, D), True), one(f"{path}.gate.bias", (H,), False),
                    one(f"{path}.up.weight", (H, D), True), one(f"{path}.up.bias", (H,), False),
                    one(f"{path}.down.weight", (D, H), True), one(f"{path}.down.bias", (D,), False)]
            ptrs = [None if a is None else a.ctypes.data for a in keep]
            rc = L.nomas_ffn_from_host(D, H, int(src.dtype), src.device, *ptrs, C.byref(h))
        else:
            raise ValueError(f"unknown weight source {src.kind!r}")
        _check(rc)
        return cls(h, dim, hidden, src.dtype, src.device)

    # -- FeedForward::forward (mlp.rs:39-48) -----------------------------------
    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """x: (..., D) in the model dtype, on the layer's GPU or on the host."""
        if x.dim() < 1 or x.shape[-1] != self.dim:
            raise NomasError(2, f"expected last dim {self.dim}, got shape {tuple(x.shape)}")
        if x.dtype != self.dtype.torch:
            raise NomasError(2, f"expected dtype {self.dtype.torch}, got {x.dtype}")
        xc = x.contiguous()
        rows = xc.numel() // self.dim
        if out is None:
            out = _new_output(xc)
        else:
            _check_out(out, xc)
        L = _lib.lib()
        if xc.is_cuda:
            stream = torch.cuda.current_stream(xc.device).cuda_stream
            _check(L.nomas_ffn_forward(self._h, xc.data_ptr(), out.data_ptr(), rows, stream))
        else:
            _check(L.nomas_ffn_forward_host(self._h, xc.data_ptr(), out.data_ptr(), rows))
        return out

    __call__ = forward

    def n_params(self) -> int:
        """mlp.rs:50-58."""
        return int(_lib.lib().nomas_ffn_n_params(self._h))

    def set_profiling(self, on: bool) -> None:
        _check(_lib.lib().nomas_ffn_set_profiling(self._h, 1 if on else 0))

    def stage_times(self) -> dict:
        """Average per-stage milliseconds of the forwards profiled since the last call."""
        ms = (C.c_float * 6)()
        _check(_lib.lib().nomas_ffn_stage_times(self._h, ms))
        return dict(zip(self.STAGES, [float(v) for v in ms]))

    @property
    def uses_mfma(self) -> bool:
        return bool(_lib.lib().nomas_ffn_uses_mfma(self._h))

    def close(self) -> None:
        if self._h:
            _lib.lib().nomas_ffn_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
