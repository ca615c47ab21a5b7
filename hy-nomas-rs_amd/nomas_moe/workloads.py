"""Seeded synthetic workloads for the MoE feed-forward block.

Five shapes of the hy-nomas-rs MoE FFN (dim D, experts E, top-k, SwiGLU hidden
H).  All tensors are drawn with the reference generator
(deterministic_randn_affine, tensor_utils.rs:123-138) from per-tensor seeds
path_seed(base, key) (mod.rs:47-55), with base = 0x5EED0000 + index and the
reference's checkpoint keys (weights.rs:78-93) as paths:

* x ~ N(0, 1), key "x"; router W ~ N(0, 0.02); gate/up W ~ N(0, 1/sqrt(D));
  down W ~ N(0, 1/sqrt(H)); biases zero (or N(0, 0.1) with ``bias=True``).
* "fine64" gives the router a per-expert logit bias b_e ~ N(0, 0.5): column 0
  of x is set to 1, router column 0 holds b_e and the other router columns are
  N(0, 1/sqrt(D-1)), so logits ~ N(0, 1) + b_e with a bias-free router.
* "skewed16" uses the same construction with fixed biases: expert 0 gets +8
  (selected by essentially every row, ~50% of all assignments) and experts
  1..15 share the second slot with Zipf(s=1.2) frequencies.  The 15 biases were
  fitted once by a seeded Monte-Carlo fixed-point iteration on
  argmax(N(0,1) + b) and are stored here as constants.
Parameters are returned in f32 (reference (out, in) layout); the caller rounds
to the model dtype.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import path_seed, randn_affine

SKEW_BIASES = [8.0, 0.0, -0.592, -0.89, -1.09, -1.239, -1.345, -1.439, -1.52, -1.584, -1.646,
               -1.687, -1.747, -1.789, -1.839, -1.859]


@dataclass(frozen=True)
class Workload:
    name: str
    index: int
    rows: int
    dim: int
    experts: int
    top_k: int
    hidden: int
    dtype: str
    router: str = "normal"  # normal | fine64 | skewed16
    note: str = ""
    sequences: int = 1  # the batch of the DiT block the rows come from (rows / seq)

    @property
    def base_seed(self) -> int:
        return 0x5EED0000 + self.index

    @property
    def assignments(self) -> int:
        return self.rows * self.top_k

    def gemm_flops(self, rows: int | None = None) -> float:
        a = (self.rows if rows is None else rows) * self.top_k
        return 6.0 * a * self.dim * self.hidden


WORKLOADS = {
    w.name: w for w in [
        Workload("tiny", 0, 208, 64, 4, 2, 128, "f32",
                 note="192 video + 16 text rows, f32"),
        Workload("seg8b", 1, 4680, 3072, 8, 2, 8192, "bf16",
                 note="8B preset, one segment: 3 latent frames x 1560 rows"),
        Workload("cfg8b", 2, 14232, 3072, 8, 2, 8192, "bf16",
                 note="8B preset, three guidance branches stacked: 3 x (4680 video + 64 text)",
                 sequences=3),
        Workload("fine64", 3, 16384, 3072, 64, 8, 1536, "bf16", router="fine64",
                 note="fine-grained: 64 experts, top-8, per-expert logit bias N(0, 0.5)"),
        Workload("skewed16", 4, 32768, 3072, 16, 2, 4096, "bf16", router="skewed16",
                 note="skewed: one expert ~50% of assignments, the rest Zipf(1.2)"),
    ]
}


def moe_path(block: int = 0) -> str:
    return f"blocks.{block}.moe"


def make_x(w: Workload, rows: int | None = None) -> np.ndarray:
    """Hidden states (rows, D) in f32; a prefix of the full workload when rows < w.rows."""
    n = w.rows if rows is None else rows
    x = randn_affine(path_seed(w.base_seed, "x"), n * w.dim).reshape(n, w.dim)
    if w.router != "normal":
        x[:, 0] = 1.0
    return x


def make_router(w: Workload) -> np.ndarray:
    """The router weight (E, D) in f32 (key {path}.router.weight)."""
    D, E, s = w.dim, w.experts, w.base_seed
    p = moe_path()
    if w.router == "normal":
        return randn_affine(path_seed(s, p + ".router"), E * D, 0.0, 0.02).reshape(E, D)
    wr = np.empty((E, D), np.float32)
    wr[:, 1:] = randn_affine(path_seed(s, p + ".router"), E * (D - 1), 0.0,
                             1.0 / math.sqrt(D - 1)).reshape(E, D - 1)
    if w.router == "fine64":
        wr[:, 0] = randn_affine(path_seed(s, p + ".router.logit_bias"), E, 0.0, 0.5)
    else:
        wr[:, 0] = np.asarray(SKEW_BIASES[:E], np.float32)
    return wr


def make_params(w: Workload, bias: bool = False, dense: bool = False) -> dict:
    """f32 parameters keyed like the checkpoint (weights.rs:78-93)."""
    D, H, E, s = w.dim, w.hidden, w.experts, w.base_seed
    p = moe_path()
    t = {p + ".router.weight": make_router(w)}

    def lin(path, out_f, in_f, std):
        t[path + ".weight"] = randn_affine(path_seed(s, path), out_f * in_f, 0.0,
                                           std).reshape(out_f, in_f)
        t[path + ".bias"] = (randn_affine(path_seed(s, path + ".bias"), out_f, 0.0, 0.1) if bias
                             else np.zeros(out_f, np.float32))

    names = [f"{p}.experts.{e}" for e in range(E)] + ([p + ".dense"] if dense else [])
    for base in names:
        lin(base + ".gate", H, D, 1.0 / math.sqrt(D))
        lin(base + ".up", H, D, 1.0 / math.sqrt(D))
        lin(base + ".down", D, H, 1.0 / math.sqrt(H))
    return t


def oracle_params(t: dict, E: int, block: int = 0):
    """Reorganise checkpoint-keyed arrays into the stacked layout of the CPU oracle."""
    p = moe_path(block)
    out = {"wr": t[p + ".router.weight"]}
    for name, key in (("wg", "gate.weight"), ("bg", "gate.bias"), ("wu", "up.weight"),
                      ("bu", "up.bias"), ("wd", "down.weight"), ("bd", "down.bias")):
        out[name] = np.stack([t[f"{p}.experts.{e}.{key}"] for e in range(E)])
    dense = None
    if p + ".dense.gate.weight" in t:
        dense = {name: t[f"{p}.dense.{key}"] for name, key in
                 (("wg", "gate.weight"), ("bg", "gate.bias"), ("wu", "up.weight"),
                  ("bu", "up.bias"), ("wd", "down.weight"), ("bd", "down.bias"))}
    return out, dense
