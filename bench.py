#!/usr/bin/env python3
"""MoE-FFN throughput on one MI355X: tokens/s of the top-k MoE feed-forward block.

Default workload: dim 3072, 8 experts, top-2, SwiGLU hidden 8192, bf16, 14,232
rows (three guidance branches of the 8B preset stacked: 3 x (4680 video + 64
text)).  Inputs are synthetic and seeded (nomas_moe.workloads); weights are
random-init of that architecture.  One step = one full forward (router,
scan, dispatch, gate/up GEMM, down GEMM, combine) with x already resident in
HBM.  Prints one JSON line.

  python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]
                  [--ffn [--ffn-hidden H] | --block | --vendor-gemm | --hbm-yardstick |
                   --host-tensors]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hy-nomas-rs_amd"))

METRIC = "MoE-FFN tokens/s at dim3072 E8 top2 bf16; % of bf16 MFMA and HBM peak"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E


def algorithmic(w, b):
    """Algorithmic flops / bytes per launch of each stage (fixed definitions)."""
    T, D, E, k, H = w.rows, w.dim, w.experts, w.top_k, w.hidden
    A = T * k
    return {
        "gemm_gate_up_flops": 4.0 * A * D * H,
        "gemm_down_flops": 2.0 * A * D * H,
        "router_bytes": T * D * b + E * D * b + 8 * T * k,
        "dispatch_bytes": T * D * b + A * D * b + 8 * A,
        "combine_bytes": A * D * b + 8 * A + T * D * b,
    }


def traffic_from_profile(workload):
    """HBM bytes per launch of the gate/up GEMM, from the committed rocprofv3
    counter summary (FETCH_SIZE + WRITE_SIZE, calibrated against a copy of
    known size), or None when no summary for this workload exists."""
    path = os.path.join(ROOT, "profiles", f"gemm_gate_up_{workload}_hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def copy_probe(mb):
    """A plain device copy of known size (f16 -> f32 conversion: reads 2 bytes
    and writes 4 bytes per element), used to calibrate the FETCH_SIZE and
    WRITE_SIZE counters."""
    import torch
    n = mb * (1 << 20) // 2
    src = torch.ones(n, dtype=torch.float16, device="cuda")
    dst = torch.empty(n, dtype=torch.float32, device="cuda")
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_elements": n, "read_bytes": 2 * n, "write_bytes": 4 * n}))
    return 0


def cpu_baseline(w, params, x, target_s=12.0):
    """The reference algorithm (every expert on every row, f32) on host cores,
    timed on a bounded prefix of the workload's rows."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    from nomas_moe import workloads as wl

    p, _ = wl.oracle_params(params, w.experts)
    probe = 4
    t0 = time.perf_counter()
    O.forward_dense_f32(x[:probe], p, w.top_k)
    dt = time.perf_counter() - t0
    rows = int(max(probe, min(w.rows, probe * target_s / max(dt, 1e-3))))
    t0 = time.perf_counter()
    O.forward_dense_f32(x[:rows], p, w.top_k)
    dt = time.perf_counter() - t0
    return {
        "value": rows / dt,
        "unit": "tokens/s",
        "cores": O.num_threads(),
        "kind": "port",
        "sample": f"first {rows} of {w.rows} rows, faithful dense f32 (all {w.experts} experts "
                  f"per row, as the reference evaluates), {dt:.1f} s",
    }


def bench_ffn(args, w) -> int:
    """The dense SwiGLU feed-forward (FeedForward::SwiGlu) at the workload's shape."""
    import numpy as np
    import torch
    import nomas_moe as nm

    dt = nm.DataType.of(w.dtype)
    ffn = nm.FeedForward.from_source(nm.Weights.random(0x5EED0000, dt), "blocks.0.mlp", w.dim,
                                     w.hidden)
    raw = nm.to_model_dtype(nm.randn_affine(0x5EED0001, w.rows * w.dim).reshape(w.rows, w.dim), dt)
    xd = torch.from_numpy(raw.view(np.int16) if raw.dtype == np.uint16 else raw)
    xd = xd.view(dt.torch).cuda()
    y = torch.empty_like(xd)
    for _ in range(args.warmup):
        ffn.forward(xd, out=y)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    def timed_steps():
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            ffn.forward(xd, out=y)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps

    ms = timed_steps()  # the forwards alone; then again with the stage events
    ffn.set_profiling(True)
    timed_steps()
    st = ffn.stage_times()
    ffn.set_profiling(False)
    flops = 6.0 * w.rows * w.dim * w.hidden
    gemm_ms = st["gemm_gate_up"] + st["gemm_down"]
    print(json.dumps({
        "metric": f"dense SwiGLU FFN tokens/s at dim{w.dim} hidden{w.hidden} {w.dtype}",
        "value": w.rows / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "dtype": w.dtype,
        "data": "synthetic (seeded N(0,1) rows, random-init weights)",
        "config": {"workload": f"dense FFN, {w.rows} rows", "rows": w.rows, "dim": w.dim,
                   "hidden": w.hidden},
        "stages_ms": st, "gemm_tflops": flops / (gemm_ms * 1e-3) / 1e12,
        "gemm_frac": flops / (gemm_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "uses_mfma": ffn.uses_mfma}))
    return 0


def bench_host_tensors(args, w) -> int:
    """The host-tensor forward (nomas_moe_forward_host, the candle-CPU-tensor call): x in and y out
    in host memory, PCIe copies included, with pageable and with pinned buffers, against the
    device-resident forward.  Wall-clock per forward over the timed steps (each host-tensor call
    returns with y in host memory)."""
    import numpy as np
    import torch
    import nomas_moe as nm
    from nomas_moe import workloads as wl

    dt = nm.DataType.of(w.dtype)
    layer = nm.MoeLayer.from_source(nm.Weights.from_tensors(wl.make_params(w), dt), wl.moe_path(),
                                    w.dim, w.hidden, nm.MoeConfig(w.experts, w.top_k, 0.0, 0))
    raw = nm.to_model_dtype(wl.make_x(w), dt)
    xh = torch.from_numpy(raw.view(np.int16) if raw.dtype == np.uint16 else raw).view(dt.torch)
    cases = {"pageable": (xh, torch.empty_like(xh)),
             "pinned": (xh.pin_memory(), torch.empty_like(xh).pin_memory())}
    xd = xh.cuda()
    cases["device"] = (xd, torch.empty_like(xd))
    ms = {}
    for name, (x, y) in cases.items():
        for _ in range(args.warmup):
            layer.forward(x, out=y)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            layer.forward(x, out=y)
        torch.cuda.synchronize()
        ms[name] = (time.perf_counter() - t0) / args.steps * 1e3
    mb = w.rows * w.dim * raw.itemsize / 1e6
    print(json.dumps({
        "metric": f"host-tensor MoE-FFN tokens/s at dim{w.dim} E{w.experts} top{w.top_k} {w.dtype}, "
                  "PCIe copies included",
        "value": w.rows / (ms["pageable"] * 1e-3), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms["pageable"],
        "higher_is_better": True, "dtype": w.dtype, "data": "synthetic (seeded N(0,1) rows, "
        "random-init weights of this shape)",
        "config": {"workload": f"{w.name}: {w.note}", "rows": w.rows,
                   "x_and_y_mb_each_way": round(mb, 1)},
        "ms_per_forward": ms,
        "tokens_per_s": {k: w.rows / (v * 1e-3) for k, v in ms.items()}}))
    return 0


def bench_block(args, w) -> int:
    """The FFN half of the DiT block around the MoE (block.rs:96-101) --
    norm2 + modulate, the MoE, the gated residual -- against the plain MoE
    forward on the same rows."""
    import numpy as np
    import torch
    import nomas_moe as nm
    from nomas_moe import workloads as wl

    dt = nm.DataType.of(w.dtype)
    B, S, D = w.sequences, w.rows // w.sequences, w.dim
    params = wl.make_params(w)
    cfg = nm.MoeConfig(w.experts, w.top_k, 0.0, 0)
    layer = nm.MoeLayer.from_source(nm.Weights.from_tensors(params, dt), wl.moe_path(), D,
                                    w.hidden, cfg)
    raw = nm.to_model_dtype(wl.make_x(w), dt)
    xd = torch.from_numpy(raw.view(np.int16) if raw.dtype == np.uint16 else raw)
    xd = xd.view(dt.torch).cuda().reshape(B, S, D)
    rnd = lambda seed, n, std: torch.from_numpy(nm.randn_affine(seed, n, 0.0, std)).cuda()
    shift, scale, gate = (rnd(w.base_seed + i, B * D, 0.5).reshape(B, D) for i in (1, 2, 3))
    norm_w = rnd(w.base_seed + 4, D, 1.0)
    out = torch.empty_like(xd)
    stream = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(args.steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps

    ms_block = timed(lambda: layer.forward_block(xd, shift, scale, gate, norm_w, out=out))
    ms_plain = timed(lambda: layer.forward(xd, out=out))
    ms_seam = timed(lambda: nm.norm_modulate(xd, shift, scale, norm_w, out=out))
    b = 2 if w.dtype != "f32" else 4
    print(json.dumps({
        "metric": f"DiT block FFN half (norm2 + modulate, MoE, gated residual) tokens/s at "
                  f"dim{D} E{w.experts} top{w.top_k} {w.dtype}",
        "value": w.rows / (ms_block * 1e-3), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_block,
        "higher_is_better": True, "dtype": w.dtype,
        "data": "synthetic (seeded N(0,1) rows, random-init weights, N(0,0.25) AdaLN parameters)",
        "config": {"workload": f"{w.name}: {w.note}", "sequences": B, "seq_len": S, "dim": D,
                   "experts": w.experts, "top_k": w.top_k, "hidden": w.hidden},
        "plain_moe_ms": ms_plain, "seam_overhead_ms": ms_block - ms_plain,
        "norm_modulate_ms": ms_seam,
        # norm_modulate alone: reads x twice (once through the sum of squares,
        # once for h) and writes h
        "norm_modulate_hbm_gbps": 3.0 * w.rows * D * b / (ms_seam * 1e-3) / 1e9,
    }))
    return 0


def bench_vendor_gemm(args, w) -> int:
    """The vendor GEMM library (hipBLASLt through torch.matmul) on dense GEMMs
    with the flops of the workload's grouped ones: all A = rows * top_k routed
    rows against one weight (gate/up: A x D times D x 2H; down: A x H times
    H x D), operands drawn like the workload's (rows N(0, 1), weights
    N(0, 1/sqrt(fan_in)), h = silu(g) * u of the gate/up product).  At the
    chip's power limit the arithmetic rate depends on the operand bits, so the
    data is matched, not just the shapes.  A same-box yardstick for the grouped
    GEMMs, not part of the MoE path."""
    import torch

    T, D, H, k = w.rows, w.dim, w.hidden, w.top_k
    A = T * k
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[w.dtype]
    g = torch.Generator(device="cuda")
    g.manual_seed(w.base_seed)
    x = torch.randn(A, D, generator=g, device="cuda").to(dt)
    w1 = (torch.randn(2 * H, D, generator=g, device="cuda") / D ** 0.5).to(dt)
    w2 = (torch.randn(D, H, generator=g, device="cuda") / H ** 0.5).to(dt)
    gu = x @ w1.t()
    h = (torch.nn.functional.silu(gu[:, :H].float()) * gu[:, H:].float()).to(dt)
    del gu
    stream = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(args.steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps

    out1 = torch.empty(A, 2 * H, dtype=dt, device="cuda")
    out2 = torch.empty(A, D, dtype=dt, device="cuda")
    ms1 = timed(lambda: torch.matmul(x, w1.t(), out=out1))
    ms2 = timed(lambda: torch.matmul(h, w2.t(), out=out2))

    def alternating():
        # the two GEMMs in the forward's order (gate/up, down, gate/up, ...),
        # each bracketed by its own events: at the power limit a kernel's
        # rate depends on what ran before it
        for _ in range(args.warmup):
            torch.matmul(x, w1.t(), out=out1)
            torch.matmul(h, w2.t(), out=out2)
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3 * args.steps)]
        for i in range(args.steps):
            ev[3 * i].record(stream)
            torch.matmul(x, w1.t(), out=out1)
            ev[3 * i + 1].record(stream)
            torch.matmul(h, w2.t(), out=out2)
            ev[3 * i + 2].record(stream)
        torch.cuda.synchronize()
        a1 = sum(ev[3 * i].elapsed_time(ev[3 * i + 1]) for i in range(args.steps)) / args.steps
        a2 = sum(ev[3 * i + 1].elapsed_time(ev[3 * i + 2]) for i in range(args.steps)) / args.steps
        return a1, a2

    alt1, alt2 = alternating()
    f1, f2 = 4.0 * A * D * H, 2.0 * A * D * H
    print(json.dumps({
        "metric": "vendor GEMM (hipBLASLt via torch.matmul) TFLOP/s on the dense equivalents of "
                  "the grouped GEMMs",
        "config": {"workload": f"{w.name}: {w.note}", "routed_rows": A, "dim": D, "hidden": H},
        "dtype": w.dtype, "steps": args.steps, "warmup": args.warmup,
        "gate_up": {"shape": [A, 2 * H, D], "ms": ms1, "tflops": f1 / (ms1 * 1e-3) / 1e12,
                    "frac": f1 / (ms1 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS},
        "down": {"shape": [A, D, H], "ms": ms2, "tflops": f2 / (ms2 * 1e-3) / 1e12,
                 "frac": f2 / (ms2 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS},
        "alternating": {"gate_up_ms": alt1, "gate_up_frac": f1 / (alt1 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                        "down_ms": alt2, "down_frac": f2 / (alt2 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS},
    }))
    return 0


def bench_hbm_yardstick(args, w) -> int:
    """torch's own elementwise and reduction kernels moving the bytes of the
    dispatch and the combine at the workload's shape, as a same-box yardstick
    for what the memory system sustains on such traffic:
      - broadcast copy: x (T x D) written k times into a (T*k) x D buffer, the
        dispatch's byte mix with contiguous instead of routed writes;
      - sum over k: (T, k, D) summed over k into T x D, the combine's byte mix
        with contiguous instead of routed reads (bf16 in, f32 sums, bf16 out);
      - fill, read (a full sum) and copy of the (T*k) x D buffer: pure writes,
        pure reads, and reads plus writes of the routed rows' bytes.
    Bytes are counted like the dispatch's and combine's algorithmic bytes.  Not
    part of the MoE path."""
    import torch

    T, D, k = w.rows, w.dim, w.top_k
    A = T * k
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[w.dtype]
    b = torch.tensor([], dtype=dt).element_size()
    g = torch.Generator(device="cuda")
    g.manual_seed(w.base_seed)
    x = torch.randn(T, D, generator=g, device="cuda").to(dt)
    xe = torch.randn(A, D, generator=g, device="cuda").to(dt)
    xe2 = torch.empty_like(xe)
    out = torch.empty(T, D, dtype=dt, device="cuda")
    stream = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(args.steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps

    cases = {
        "broadcast_copy": (lambda: xe.view(T, k, D).copy_(x.unsqueeze(1).expand(T, k, D)),
                           T * D * b + A * D * b),
        "sum_over_k": (lambda: torch.sum(xe.view(T, k, D), dim=1, out=out), A * D * b + T * D * b),
        "fill": (lambda: xe2.fill_(1.0), A * D * b),
        "read": (lambda: xe.sum(), A * D * b),
        "copy": (lambda: xe2.copy_(xe), 2 * A * D * b),
    }
    res = {}
    for name, (fn, nbytes) in cases.items():
        ms = timed(fn)
        tbs = nbytes / (ms * 1e-3) / 1e12
        res[name] = {"us": ms * 1e3, "bytes": nbytes, "TB/s": tbs, "frac": tbs * 1e3 / PEAK_HBM_GBPS}
    print(json.dumps({
        "metric": "torch kernels' HBM rate on the dispatch's and combine's byte mix (yardstick)",
        "config": {"workload": f"{w.name}: {w.note}", "rows": T, "dim": D, "top_k": k},
        "dtype": w.dtype, "steps": args.steps, "warmup": args.warmup, "cases": res,
    }))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="cfg8b")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ffn-hidden", type=int, default=0,
                    help="with --ffn: the FFN's hidden size instead of the workload's (12288 is "
                         "the 8B preset's dense FFN, dim 3072 x mlp_ratio 4.0)")
    ap.add_argument("--ffn", action="store_true",
                    help="time the dense SwiGLU feed-forward (one expert, no routing) at the "
                         "workload's dim, hidden and rows instead of the MoE block")
    ap.add_argument("--block", action="store_true",
                    help="time the FFN half of the DiT block (norm2 + modulate, MoE, gated "
                         "residual) against the plain MoE forward")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="time the vendor GEMM library on dense GEMMs with the workload's "
                         "flops and operand statistics (a yardstick for the grouped GEMMs)")
    ap.add_argument("--hbm-yardstick", action="store_true",
                    help="time torch's own kernels on the dispatch's and combine's byte mix "
                         "(a yardstick for the memory-bound stages)")
    ap.add_argument("--host-tensors", action="store_true",
                    help="time the host-tensor forward (x and y in host memory, PCIe copies "
                         "included; pageable and pinned) against the device-resident one")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="only run a plain copy of this many MB (counter calibration) and exit")
    args = ap.parse_args()
    if args.copy_probe_mb:
        return copy_probe(args.copy_probe_mb)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: the MoE "
              "feed-forward path here is single-GPU (no collectives).", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import nomas_moe as nm
    from nomas_moe import workloads as wl

    w = wl.WORKLOADS[args.workload]
    if args.ffn:
        if args.ffn_hidden:
            import dataclasses
            w = dataclasses.replace(w, hidden=args.ffn_hidden)
        return bench_ffn(args, w)
    if args.block:
        return bench_block(args, w)
    if args.vendor_gemm:
        return bench_vendor_gemm(args, w)
    if args.hbm_yardstick:
        return bench_hbm_yardstick(args, w)
    if args.host_tensors:
        return bench_host_tensors(args, w)
    dt = nm.DataType.of(w.dtype)
    print(f"[bench] workload {w.name}: rows={w.rows} D={w.dim} E={w.experts} k={w.top_k} "
          f"H={w.hidden} {w.dtype}", file=sys.stderr, flush=True)
    params = wl.make_params(w)
    x = wl.make_x(w)
    cfg = nm.MoeConfig(w.experts, w.top_k, 0.0, 0)
    layer = nm.MoeLayer.from_source(nm.Weights.from_tensors(params, dt), wl.moe_path(), w.dim,
                                    w.hidden, cfg)
    raw = nm.to_model_dtype(x, dt)
    xd = torch.from_numpy(raw.view(np.int16) if raw.dtype == np.uint16 else raw)
    xd = xd.view(dt.torch).cuda()
    y = torch.empty_like(xd)
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        layer.forward(xd, out=y)
    torch.cuda.synchronize()

    def timed_steps():
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            layer.forward(xd, out=y)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps

    # the headline: K forwards, nothing else on the stream
    ms = timed_steps()
    # the same K forwards again with the library's per-stage events (HIP
    # events stamped by the runtime at the start and end of each stage's
    # kernels on the forward's stream: the kernels' own durations) for the
    # stage times and the roofline
    layer.set_profiling(True)
    ms_profiled = timed_steps()
    stages = layer.stage_times()
    layer.set_profiling(False)
    finite = bool(torch.isfinite(y.float()).all())
    print(f"[bench] {ms:.3f} ms/step ({ms_profiled:.3f} with stage events), stages {stages}, "
          f"finite={finite}", file=sys.stderr, flush=True)

    b = 2 if w.dtype != "f32" else 4
    alg = algorithmic(w, b)
    gu_tf = alg["gemm_gate_up_flops"] / (stages["gemm_gate_up"] * 1e-3) / 1e12
    dn_tf = alg["gemm_down_flops"] / (stages["gemm_down"] * 1e-3) / 1e12
    both_tf = (alg["gemm_gate_up_flops"] + alg["gemm_down_flops"]) / (
        (stages["gemm_gate_up"] + stages["gemm_down"]) * 1e-3) / 1e12
    gbps = {s: alg[s + "_bytes"] / (stages[s] * 1e-3) / 1e9
            for s in ("router", "dispatch", "combine")}
    result = {
        "metric": METRIC,
        "value": w.rows / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic (seeded N(0,1) rows, random-init weights of this shape)",
        "config": {"workload": f"{w.name}: {w.note}", "rows": w.rows, "dim": w.dim,
                   "experts": w.experts, "top_k": w.top_k, "hidden": w.hidden},
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_gate_up (grouped gate/up GEMM + SwiGLU)",
            "achieved": gu_tf,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gu_tf / PEAK_BF16_TFLOPS,
            "traffic": traffic_from_profile(w.name),
        },
        "stages_ms": stages,
        "ms_per_step_with_stage_events": ms_profiled,
        "gemm_tflops": {"gate_up": gu_tf, "down": dn_tf, "both": both_tf,
                        "both_frac": both_tf / PEAK_BF16_TFLOPS},
        "hbm_gbps": gbps,
        "hbm_frac": {s: v / PEAK_HBM_GBPS for s, v in gbps.items()},
        "output_finite": finite,
    }
    if not args.no_cpu_baseline:
        wparams = {k: nm.widen(nm.to_model_dtype(v, dt), dt) for k, v in params.items()}
        result["cpu_baseline"] = cpu_baseline(w, wparams, nm.widen(raw, dt))
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
