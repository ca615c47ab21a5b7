"""The host-facing interface on the GPU: weight sources, host tensors, readbacks.

Mirrors how the reference builds and calls the layer: MoeLayer::from_source
over Weights::Random / Weights::Loaded (moe.rs:26-62, mod.rs:20-116,
weights.rs:105-145), forward on host tensors, n_params (moe.rs:112-114).
"""
import math

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file

import nomas_moe as nm
import oracle as O
from _common import PATH, rounded, small_case
from _gpu import compare, layer_from_tensors, rel_err, to_device

pytestmark = pytest.mark.gpu


def test_n_params_matches_reference_formula():
    # router (E x D, no bias) + E x (gate + up + down with biases); dense excluded
    E, D, H = 4, 64, 96
    layer = nm.MoeLayer.from_source(nm.Weights.random(1), PATH, D, H, nm.MoeConfig(E, 2, 0.5))
    assert layer.n_params() == E * D + E * (2 * (H * D + H) + (D * H + D))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_random_weights_rounded_to_model_dtype(dtype):
    # Weights::Random: xavier(path_seed(seed, path)) then to_dtype (mod.rs:80-95)
    E, D, H, k, seed = 8, 256, 128, 2, 7
    layer = nm.MoeLayer.from_source(nm.Weights.random(seed, dtype), PATH, D, H, nm.MoeConfig(E, k))
    p = {"wr": O.xavier(E, D, O.path_seed(seed, PATH + ".router"))}
    for name, key, o, i in (("wg", "gate", H, D), ("wu", "up", H, D), ("wd", "down", D, H)):
        p[name] = np.stack([O.xavier(o, i, O.path_seed(seed, f"{PATH}.experts.{e}.{key}"))
                            for e in range(E)])
    p = {kk: nm.widen(nm.to_model_dtype(v, dtype), dtype) for kk, v in p.items()}
    x = nm.randn_affine(11, 120 * D).reshape(120, D)
    compare(layer, to_device(x, dtype), nm.widen(nm.to_model_dtype(x, dtype), dtype), p, k, dtype)


def test_host_tensor_forward_equals_device_forward():
    t, x = small_case(300, 256, 8, 2, 128, 31)
    layer = layer_from_tensors(t, "bf16", 256, 128, 8, 2)
    xd = to_device(x, "bf16").reshape(3, 100, 256)  # (B, S, D): leading dims folded
    yd = layer.forward(xd).cpu()
    yh = layer.forward(xd.cpu())
    assert yh.device.type == "cpu" and tuple(yh.shape) == (3, 100, 256)
    assert torch.equal(yd, yh)


def test_host_tensor_forward_in_several_staging_chunks():
    # 33,333 rows x 264 f32 = 35.2 MB each way: three 16 MB staging chunks, the
    # last one partial and not a multiple of 64 bytes, each split over the copy
    # threads; then a small call on the same handle
    t, x = small_case(33_333, 264, 4, 1, 96, 32)
    layer = layer_from_tensors(t, "f32", 264, 96, 4, 1)
    xd = to_device(x, "f32")
    yd = layer.forward(xd).cpu()
    yh = layer.forward(xd.cpu())  # pageable in (staged), pinned out (direct)
    assert torch.equal(yd, yh)
    yp = torch.empty_like(yd)  # pageable out: staged on the way back too
    layer.forward(xd.cpu(), out=yp)
    assert torch.equal(yd, yp)
    assert torch.equal(layer.forward(xd[:5].cpu()), yd[:5])


def test_host_tensor_forward_in_pieces():
    # 10,000 bf16 rows of 256 (the MFMA path): two pieces of 5,056 and 4,944 rows, the copies of one
    # overlapping the other's forward.  The routing of the whole call is kept (the pieces are whole
    # 64-row router chunks, so it equals a device forward's bit for bit); outputs against the oracle
    # and the device forward (a K-split tile may round differently in a piece).
    rows, D, E, k, H = 10_000, 256, 8, 2, 128
    t, x = small_case(rows, D, E, k, H, 33)
    layer = layer_from_tensors(t, "bf16", D, H, E, k)
    rt, rx = rounded(t, x, "bf16")
    p, _ = nm.workloads.oracle_params(rt, E)
    xd = to_device(x, "bf16")
    yd = layer.forward(xd).float().cpu().numpy()
    d_route = layer.routing(rows)
    yh = layer.forward(xd.cpu())  # pageable in and out, staged
    assert yh.device.type == "cpu"
    h_route = layer.routing(rows)
    for a, b in zip(h_route, d_route):
        assert np.array_equal(a, b)
    got = yh.float().numpy()
    sel = np.arange(0, rows, 37)
    ref, _, _, _ = O.forward_sparse(rx, p, k, rows=sel)
    assert rel_err(got[sel], ref) <= 2e-2
    assert rel_err(got, yd) <= 1e-2  # at most a bf16 ulp where rounding differs
    # pinned in and out: straight DMA, the same pieces, the same bits
    yp = torch.empty_like(yh).pin_memory()
    layer.forward(xd.cpu().pin_memory(), out=yp)
    assert torch.equal(yp, yh)


@pytest.mark.parametrize("src_dtype,model", [(np.float32, "bf16"), (np.float16, "f16"),
                                             (np.float32, "f32")])
def test_safetensors_checkpoint_equals_in_memory_tensors(tmp_path, src_dtype, model):
    E, D, H, k = 6, 256, 128, 2
    t, x = small_case(200, D, E, k, H, 32, dense=True)
    files = [str(tmp_path / "a.safetensors"), str(tmp_path / "b.safetensors")]
    keys = sorted(t)
    half = len(keys) // 2
    # split over two files; the second also overrides one tensor of the first
    save_file({kk: t[kk].astype(src_dtype) for kk in keys[:half] + keys[-1:]}, files[0])
    save_file({kk: t[kk].astype(src_dtype) for kk in keys[half:]}, files[1])
    cfg = nm.MoeConfig(E, k, 0.25)
    a = nm.MoeLayer.from_source(nm.Weights.loaded(files, model), PATH, D, H, cfg)
    ts = {kk: v.astype(src_dtype).astype(np.float32) for kk, v in t.items()}
    b = nm.MoeLayer.from_source(nm.Weights.from_tensors(ts, model), PATH, D, H, cfg)
    xd = to_device(x, model)
    assert torch.equal(a.forward(xd), b.forward(xd))


def test_dtype_mismatch_is_an_error():
    t, x = small_case(10, 256, 8, 2, 128, 33)
    layer = layer_from_tensors(t, "bf16", 256, 128, 8, 2)
    with pytest.raises(nm.NomasError, match="dtype"):
        layer.forward(torch.zeros(10, 256, device="cuda", dtype=torch.float32))
    with pytest.raises(nm.NomasError, match="last dim"):
        layer.forward(torch.zeros(10, 128, device="cuda", dtype=torch.bfloat16))


def test_stage_profiling():
    t, x = small_case(500, 256, 8, 2, 128, 34)
    layer = layer_from_tensors(t, "bf16", 256, 128, 8, 2)
    xd = to_device(x, "bf16")
    layer.set_profiling(True)
    for _ in range(3):
        layer.forward(xd)
    st = layer.stage_times()
    assert set(st) == set(nm.MoeLayer.STAGES)
    # the histogram scan runs inside the dispatch kernel: no kernel, zero time
    assert st["scan"] == 0 and all(v > 0 for k, v in st.items() if k != "scan")
    with pytest.raises(nm.NomasError):
        layer.stage_times()  # nothing recorded since the last read
    # the stage times are the kernels' own: one forward's add up to no more
    # than its wall time between two events
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    layer.forward(xd)
    torch.cuda.synchronize()
    start.record()
    layer.forward(xd)
    end.record()
    torch.cuda.synchronize()
    st = layer.stage_times()
    assert 0 < sum(st.values()) <= start.elapsed_time(end) * 1.001
    layer.set_profiling(False)


def test_forward_on_a_side_stream():
    t, x = small_case(400, 256, 8, 2, 128, 35)
    layer = layer_from_tensors(t, "bf16", 256, 128, 8, 2)
    xd = to_device(x, "bf16")
    ref = layer.forward(xd)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())  # x is ready; the handle orders its own work
    with torch.cuda.stream(s):
        y = layer.forward(xd)
    s.synchronize()
    assert torch.equal(ref, y)
