"""The C ABI (include/nomas_moe.h) on the host -- CPU only.

Loads libnomas_moe.so, checks that it exports every declared entry point, and
exercises every error path that is decided before the GPU is touched: config
validation (config.rs:394-399), shape limits, null arguments, and checkpoint
loading (weights.rs:105-145: missing keys, misshaped tensors, unreadable files).
"""
import ctypes as C
import os
import re

import numpy as np
import pytest
from safetensors.numpy import save_file

import nomas_moe as nm
from nomas_moe import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nomas_moe.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nomas_\w+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 18
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_config_validate_mirrors_reference():
    nm.MoeConfig(experts=8, top_k=2).validate()
    nm.MoeConfig(experts=4, top_k=4).validate()
    for bad in (nm.MoeConfig(4, 0), nm.MoeConfig(4, 5), nm.MoeConfig(0, 1)):
        with pytest.raises(nm.InvalidConfig, match="invalid MoE top_k/experts"):
            bad.validate()


@pytest.mark.parametrize("cfg,dim,hidden,dtype,msg", [
    (nm.MoeConfig(4, 5), 64, 128, 0, "top_k"),
    (nm.MoeConfig(300, 2), 64, 128, 0, "maximum"),
    (nm.MoeConfig(256, 200), 64, 128, 0, "dispatch"),  # slots of a 64-row chunk beyond its LDS
    (nm.MoeConfig(4, 2), 60, 128, 0, "multiple of 8"),
    (nm.MoeConfig(4, 2), 64, 0, 0, "hidden"),
    (nm.MoeConfig(4, 2), 64, 128, 7, "dtype"),
])
def test_create_rejects_invalid_config_before_touching_the_gpu(cfg, dim, hidden, dtype, msg):
    h = C.c_void_p()
    c = cfg._c()
    rc = _lib.lib().nomas_moe_from_random(C.byref(c), b"blocks.0.moe", dim, hidden, dtype, 1, 0,
                                          C.byref(h))
    assert rc == 1, _lib.last_error()
    assert msg in _lib.last_error()
    assert not h.value


def test_null_arguments_are_rejected():
    L = _lib.lib()
    c = nm.MoeConfig(4, 2)._c()
    h = C.c_void_p()
    assert L.nomas_moe_from_random(None, b"p", 64, 128, 0, 1, 0, C.byref(h)) == 2
    assert L.nomas_moe_from_random(C.byref(c), None, 64, 128, 0, 1, 0, C.byref(h)) == 2
    assert L.nomas_moe_from_host(C.byref(c), 64, 128, 0, 0, *([None] * 13), C.byref(h)) == 2
    assert L.nomas_moe_forward(None, None, None, 4, None) == 2
    assert L.nomas_moe_forward_host(None, None, None, 4) == 2
    assert L.nomas_moe_routing(None, None, None, None, None) == 2
    assert L.nomas_moe_n_params(None) == -1
    assert L.nomas_moe_uses_mfma(None) == 0
    L.nomas_moe_destroy(None)  # no-op


def test_block_seam_arguments_are_checked_before_any_launch():
    # block.rs:96,101 entry points: shapes, sequences, dtype and alignment are
    # validated on the host (NOMAS_ERR_INVALID_ARGUMENT) -- no device needed
    L = _lib.lib()
    buf = (C.c_uint8 * 4096)()
    a = (C.addressof(buf) + 15) // 16 * 16
    assert L.nomas_norm_modulate(1, a, a, 10, 256, 3, None, 1e-6, a, a, None) == 2  # 10 % 3
    assert b"sequences" in L.nomas_moe_last_error()
    assert L.nomas_norm_modulate(1, a, a, 4, 252, 4, None, 1e-6, a, a, None) == 2   # dim % 8
    assert L.nomas_norm_modulate(7, a, a, 4, 256, 4, None, 1e-6, a, a, None) == 2   # dtype
    assert L.nomas_norm_modulate(1, a + 2, a, 4, 256, 4, None, 1e-6, a, a, None) == 2  # align
    assert L.nomas_norm_modulate(1, a, a, 4, 256, 4, None, -1.0, a, a, None) == 2   # eps
    assert L.nomas_norm_modulate(1, a, a, 4, 256, 4, None, 1e-6, a, None, None) == 2  # scale
    assert L.nomas_gated_residual(1, a, a, None, a, 4, 256, 4, None) == 2            # gate
    assert L.nomas_norm_modulate(1, None, None, 0, 256, 1, None, 1e-6, None, None, None) == 0
    assert L.nomas_moe_forward_block(None, a, a, 4, 4, None, 1e-6, a, a, a, None) == 2


def _checkpoint(path, E, D, H, dtype=np.float32, drop=(), reshape=None, dense=False):
    rng = np.random.default_rng(0)
    t = {"blocks.0.moe.router.weight": rng.standard_normal((E, D)).astype(dtype)}
    names = [f"blocks.0.moe.experts.{e}" for e in range(E)] + (["blocks.0.moe.dense"] if dense else [])
    for base in names:
        for lin, (o, i) in (("gate", (H, D)), ("up", (H, D)), ("down", (D, H))):
            t[f"{base}.{lin}.weight"] = rng.standard_normal((o, i)).astype(dtype)
            t[f"{base}.{lin}.bias"] = rng.standard_normal(o).astype(dtype)
    t["blocks.0.attn.q.weight"] = np.zeros((2, 2), dtype)  # unrelated keys are ignored
    for k in drop:
        del t[k]
    if reshape:
        t[reshape] = t[reshape].reshape(-1)
    save_file(t, path)
    return t


def _load(files, E=2, k=1, D=16, H=8, dtype=0, s=0.0):
    c = nm.MoeConfig(E, k, s)._c()
    arr = (C.c_char_p * len(files))(*[f.encode() for f in files])
    h = C.c_void_p()
    rc = _lib.lib().nomas_moe_from_safetensors(C.byref(c), arr, len(files), b"blocks.0.moe", D, H,
                                               dtype, 0, C.byref(h))
    msg = _lib.last_error()
    if h.value:  # loaded (hosts with a GPU)
        _lib.lib().nomas_moe_destroy(h)
    return rc, msg


def test_checkpoint_missing_expert_keys(tmp_path):
    # weights.rs:175-188 (moe_keys): with 2 experts, experts.1.* exist and
    # experts.2.* do not; asking for 3 experts reports the missing keys
    f = str(tmp_path / "moe.safetensors")
    _checkpoint(f, 2, 16, 8)
    rc, msg = _load([f], E=3, k=1)
    assert rc == 3
    assert "blocks.0.moe.experts.2.down.bias" in msg and "missing 6 model keys" in msg


def test_checkpoint_missing_router(tmp_path):
    f = str(tmp_path / "moe.safetensors")
    _checkpoint(f, 2, 16, 8, drop=("blocks.0.moe.router.weight",))
    rc, msg = _load([f])
    assert rc == 3 and "router.weight" in msg


def test_checkpoint_misshaped_tensor(tmp_path):
    f = str(tmp_path / "moe.safetensors")
    _checkpoint(f, 2, 16, 8, reshape="blocks.0.moe.experts.1.up.weight")
    rc, msg = _load([f])
    assert rc == 3 and "experts.1.up.weight" in msg


def test_checkpoint_dense_branch_keys_required_when_shared_dense(tmp_path):
    f = str(tmp_path / "moe.safetensors")
    _checkpoint(f, 2, 16, 8, dense=False)
    rc, msg = _load([f], s=0.5)
    assert rc == 3 and "blocks.0.moe.dense" in msg


def test_checkpoint_unreadable(tmp_path):
    rc, msg = _load([str(tmp_path / "nope.safetensors")])
    assert rc == 4 and "cannot open" in msg
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(b"\x10\x00\x00\x00\x00\x00\x00\x00{not json at all")
    rc, msg = _load([str(bad)])
    assert rc == 4


def test_complete_checkpoint_parses_then_needs_a_device(tmp_path):
    # every key present and well-formed: loading proceeds to device creation
    f = str(tmp_path / "moe.safetensors")
    _checkpoint(f, 2, 16, 8, dtype=np.float16)
    rc, msg = _load([f])
    import torch
    if torch.cuda.is_available():
        assert rc == 0, msg
    else:
        assert rc == 5 and "HIP device" in msg


def test_dtype_helpers_round_to_nearest_even():
    import torch
    x = np.concatenate([nm.randn_affine(3, 5000, 0.0, 30.0),
                        np.array([1.00390625, -65519.0, 65520.0, 6e-8, 1e-40], np.float32)])
    bf = nm.to_model_dtype(x, "bf16")
    np.testing.assert_array_equal(nm.widen(bf, "bf16"),
                                  torch.from_numpy(x).to(torch.bfloat16).float().numpy())
    hf = nm.to_model_dtype(x, "f16")
    np.testing.assert_array_equal(nm.widen(hf, "f16"), x.astype(np.float16).astype(np.float32))


# ---- dense feed-forward (mlp.rs:9-59) ---------------------------------------

@pytest.mark.parametrize("dim,hidden,dtype,msg", [
    (60, 128, 0, "multiple of 8"), (64, 0, 1, "hidden"), (64, 128, 9, "dtype")])
def test_ffn_create_rejects_invalid_shape_before_touching_the_gpu(dim, hidden, dtype, msg):
    h = C.c_void_p()
    rc = _lib.lib().nomas_ffn_from_random(b"blocks.0.mlp", dim, hidden, dtype, 1, 0, C.byref(h))
    assert rc == 1, _lib.last_error()
    assert msg in _lib.last_error()
    assert not h.value


def test_ffn_null_arguments_are_rejected():
    L = _lib.lib()
    h = C.c_void_p()
    assert L.nomas_ffn_from_random(None, 64, 128, 0, 1, 0, C.byref(h)) == 2
    assert L.nomas_ffn_from_host(64, 128, 0, 0, *([None] * 6), C.byref(h)) == 2
    assert L.nomas_ffn_forward(None, None, None, 4, None) == 2
    assert L.nomas_ffn_forward_host(None, None, None, 4) == 2
    assert L.nomas_ffn_n_params(None) == -1
    assert L.nomas_ffn_uses_mfma(None) == 0
    L.nomas_ffn_destroy(None)  # no-op


def _ffn_checkpoint(path, D, H, drop=(), reshape=None):
    rng = np.random.default_rng(1)
    t = {}
    for lin, (o, i) in (("gate", (H, D)), ("up", (H, D)), ("down", (D, H))):
        t[f"blocks.0.mlp.{lin}.weight"] = rng.standard_normal((o, i)).astype(np.float32)
        t[f"blocks.0.mlp.{lin}.bias"] = rng.standard_normal(o).astype(np.float32)
    for k in drop:
        del t[k]
    if reshape:
        t[reshape] = t[reshape].reshape(-1)
    save_file(t, path)
    return t


def _load_ffn(files, D=16, H=8, dtype=0):
    arr = (C.c_char_p * len(files))(*[f.encode() for f in files])
    h = C.c_void_p()
    rc = _lib.lib().nomas_ffn_from_safetensors(arr, len(files), b"blocks.0.mlp", D, H, dtype, 0,
                                               C.byref(h))
    msg = _lib.last_error()
    if h.value:  # loaded (hosts with a GPU)
        _lib.lib().nomas_ffn_destroy(h)
    return rc, msg


def test_ffn_checkpoint_missing_keys(tmp_path):
    # FeedForward::from_source reads {path}.gate/up/down (mlp.rs:30-34)
    f = str(tmp_path / "ffn.safetensors")
    _ffn_checkpoint(f, 16, 8, drop=("blocks.0.mlp.up.bias", "blocks.0.mlp.down.weight"))
    rc, msg = _load_ffn([f])
    assert rc == 3
    assert "missing 2 model keys" in msg
    assert msg.index("blocks.0.mlp.down.weight") < msg.index("blocks.0.mlp.up.bias")  # sorted


def test_ffn_checkpoint_misshaped_tensor(tmp_path):
    f = str(tmp_path / "ffn.safetensors")
    _ffn_checkpoint(f, 16, 8, reshape="blocks.0.mlp.gate.weight")
    rc, msg = _load_ffn([f])
    assert rc == 3 and "gate.weight" in msg


def test_ffn_complete_checkpoint_parses_then_needs_a_device(tmp_path):
    f = str(tmp_path / "ffn.safetensors")
    _ffn_checkpoint(f, 16, 8)
    rc, msg = _load_ffn([f])
    import torch
    if torch.cuda.is_available():
        assert rc == 0, msg
    else:
        assert rc == 5 and "HIP device" in msg


# ---- malformed checkpoints: always NOMAS_ERR_IO "loading <path>: ...", never an abort
# (load_dit maps every unreadable file to Error::Msg("loading {path}: {e}"),
# weights.rs:112-115; the format rules are the safetensors crate's, Cargo.toml:11)

def _raw_safetensors(path, entries, payload=b"", pad=b""):
    """Writes a file with a hand-made header: entries maps name -> dict."""
    import json
    hdr = json.dumps(entries).encode() + pad
    with open(path, "wb") as f:
        f.write(len(hdr).to_bytes(8, "little"))
        f.write(hdr)
        f.write(payload)


_MALFORMED = {
    # the advisor's case: a negative dim and end < begin agree in "size" (-4 == -4)
    "negative_shape": ({"t": {"dtype": "F32", "shape": [-1], "data_offsets": [4, 0]}}, b"\0" * 4),
    "end_before_begin": ({"t": {"dtype": "F32", "shape": [1], "data_offsets": [8, 4]}}, b"\0" * 8),
    "end_past_eof": ({"t": {"dtype": "F32", "shape": [1024], "data_offsets": [0, 4096]}}, b"\0" * 16),
    "huge_shape": ({"t": {"dtype": "F32", "shape": [2 ** 62], "data_offsets": [0, 2 ** 62 * 4 % 2 ** 63]}},
                   b""),
    "numel_overflow": ({"t": {"dtype": "BF16", "shape": [2 ** 40, 2 ** 40], "data_offsets": [0, 0]}},
                       b""),
    "offset_beyond_int64": ({"t": {"dtype": "F32", "shape": [1],
                                   "data_offsets": [0, 99999999999999999999999]}}, b"\0" * 4),
    "size_mismatch": ({"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8),
    "hole": ({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},
              "b": {"dtype": "F32", "shape": [1], "data_offsets": [8, 12]}}, b"\0" * 12),
    "overlap": ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
                 "b": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\0" * 8),
    "trailing_bytes": ({"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, b"\0" * 12),
    "unknown_dtype": ({"t": {"dtype": "Q4", "shape": [1], "data_offsets": [0, 4]}}, b"\0" * 4),
    "no_offsets": ({"t": {"dtype": "F32", "shape": [1]}}, b"\0" * 4),
}


@pytest.mark.parametrize("case", sorted(_MALFORMED))
@pytest.mark.parametrize("loader", ["moe", "ffn"])
def test_malformed_checkpoint_is_an_io_error(tmp_path, case, loader):
    entries, payload = _MALFORMED[case]
    f = str(tmp_path / f"{case}.safetensors")
    _raw_safetensors(f, entries, payload)
    rc, msg = _load([f]) if loader == "moe" else _load_ffn([f])
    assert rc == 4, (rc, msg)
    assert msg.startswith(f"loading {f}: "), msg


@pytest.mark.parametrize("loader", ["moe", "ffn"])
def test_truncated_and_oversized_headers(tmp_path, loader):
    load = _load if loader == "moe" else _load_ffn
    short = tmp_path / "short.safetensors"
    short.write_bytes(b"\x05\x00\x00")  # not even the 8-byte length
    bigh = tmp_path / "bigh.safetensors"
    bigh.write_bytes((200_000_000).to_bytes(8, "little") + b"{}")  # beyond the 100 MB limit
    liar = tmp_path / "liar.safetensors"
    liar.write_bytes((4096).to_bytes(8, "little") + b"{}")  # header longer than the file
    junk = tmp_path / "junk.safetensors"
    _raw_safetensors(str(junk), {}, pad=b"  x")  # non-space after the JSON
    for p in (short, bigh, liar, junk):
        rc, msg = load([str(p)])
        assert rc == 4 and msg.startswith(f"loading {p}: "), (p.name, rc, msg)


def _raw_header_file(path, header: bytes, payload=b""):
    """Writes a file whose JSON header is the given bytes, verbatim."""
    with open(path, "wb") as f:
        f.write(len(header).to_bytes(8, "little"))
        f.write(header)
        f.write(payload)


_T = b'"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}'


def _nest(opener, depth):
    if opener == "[":
        return b"[" * depth + b"]" * depth
    return b'{"a":' * depth + b"1" + b"}" * depth


@pytest.mark.parametrize("loader", ["moe", "ffn"])
@pytest.mark.parametrize("opener", ["[", "{"])
@pytest.mark.parametrize("where", ["metadata", "entry_field"])
def test_deeply_nested_header_is_an_io_error(tmp_path, loader, opener, where):
    # 100,000 nested containers: the reference's serde_json parse stops at its
    # recursion limit and load_dit returns Err("loading <path>: ...")
    # (weights.rs:112-115); the parser here must return, not overflow the stack
    deep = _nest(opener, 100_000)
    if where == "metadata":
        hdr = b'{"__metadata__": ' + deep + b", " + _T + b"}"
    else:
        hdr = b'{"t": {"dtype": "F32", "shape": [1], "x": ' + deep + b', "data_offsets": [0, 4]}}'
    f = str(tmp_path / "deep.safetensors")
    _raw_header_file(f, hdr, b"\0" * 4)
    rc, msg = _load([f]) if loader == "moe" else _load_ffn([f])
    assert rc == 4, (rc, msg)
    assert msg == f"loading {f}: malformed safetensors header", msg


_BAD_JSON = {
    "bare_word": b'{"t": {"dtype": "F32", "shape": [1], "x": abc, "data_offsets": [0, 4]}}',
    "bad_literal": b'{"t": {"dtype": "F32", "shape": [1], "x": nul, "data_offsets": [0, 4]}}',
    "bad_number": b'{"t": {"dtype": "F32", "shape": [1], "x": 1.e5, "data_offsets": [0, 4]}}',
    "leading_zero": b'{"t": {"dtype": "F32", "shape": [01], "data_offsets": [0, 4]}}',
    "float_dim": b'{"t": {"dtype": "F32", "shape": [1.0], "data_offsets": [0, 4]}}',
    "bad_escape": b'{"t": {"dtype": "F32", "shape": [1], "x": "\\q", "data_offsets": [0, 4]}}',
    "short_unicode": b'{"t": {"dtype": "F32", "shape": [1], "x": "\\u12", "data_offsets": [0, 4]}}',
    "lone_surrogate": b'{"t": {"dtype": "F32", "shape": [1], "x": "\\udc00", "data_offsets": [0, 4]}}',
    "control_char": b'{"t": {"dtype": "F32", "shape": [1], "x": "a\x01b", "data_offsets": [0, 4]}}',
    "metadata_not_strings": b'{"__metadata__": {"a": 1}, ' + _T + b"}",
    "metadata_array": b'{"__metadata__": [], ' + _T + b"}",
    "unclosed": b'{"t": {"dtype": "F32", "shape": [1], "x": [1, 2, "data_offsets": [0, 4]}}',
    "trailing_comma": b'{"t": {"dtype": "F32", "shape": [1], "x": [1, ], "data_offsets": [0, 4]}}',
    "mismatched_close": b'{"t": {"dtype": "F32", "shape": [1], "x": [1}, "data_offsets": [0, 4]}}',
    "nest_past_limit": b'{"t": {"dtype": "F32", "shape": [1], "x": ' + _nest("[", 127) +
                       b', "data_offsets": [0, 4]}}',
}


@pytest.mark.parametrize("case", sorted(_BAD_JSON))
def test_invalid_json_header_is_an_io_error(tmp_path, case):
    f = str(tmp_path / f"{case}.safetensors")
    _raw_header_file(f, _BAD_JSON[case], b"\0" * 4)
    for load in (_load, _load_ffn):
        rc, msg = load([f])
        assert rc == 4, (case, rc, msg)
        assert msg == f"loading {f}: malformed safetensors header", msg


def test_header_json_the_format_allows_is_accepted(tmp_path):
    # legal JSON the crate accepts: escapes in strings (decoded, so the
    # unicode-escaped name is the plain key), metadata strings, null
    # metadata, numbers and nesting below the limit in an ignored field
    f = str(tmp_path / "moe.safetensors")
    _checkpoint(f, 2, 16, 8)
    raw = open(f, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    import json
    hdr = json.loads(raw[8:8 + n])
    rk = "blocks.0.moe.router.weight"
    ent = hdr.pop(rk)
    body = ", ".join(f"{json.dumps(k)}: {json.dumps(v)}" for k, v in hdr.items())
    router = ('"blocks.0.moe.\\u0072outer.weight": {"dtype": %s, "shape": %s, "x": %s, '
              '"y": [-1.5e-3, 0, true, false, null, "\\ud83d\\ude00\\n\\/"], "data_offsets": %s}'
              % (json.dumps(ent["dtype"]), json.dumps(ent["shape"]), _nest("[", 100).decode(),
                 json.dumps(ent["data_offsets"])))
    for meta in ('{"format": "pt", "note": "\\"q\\" \\u00e9"}', "null"):
        text = ('{"__metadata__": %s, %s, %s}' % (meta, router, body)).encode()
        _raw_header_file(f, text, raw[8 + n:])
        rc, msg = _load([f])
        import torch
        assert rc == (0 if torch.cuda.is_available() else 5), msg


def test_header_mutation_fuzz(tmp_path):
    # seeded mutations of a valid header (byte flips, truncations, inserted
    # and deleted bytes, deep nests spliced in): every load returns a status
    # with the reference's message form -- no crash, no hang (the sanitized
    # suite runs this under ASan/UBSan)
    f = str(tmp_path / "base.safetensors")
    _checkpoint(f, 2, 16, 8)
    raw = open(f, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    hdr, payload = raw[8:8 + n], raw[8 + n:]
    rng = np.random.default_rng(20261202)
    alphabet = b'{}[]",:0123456789-+.eEtrufalsn \\u\x00\xff'
    g = str(tmp_path / "mut.safetensors")
    for it in range(600):
        h = bytearray(hdr)
        for _ in range(int(rng.integers(1, 4))):
            op = int(rng.integers(0, 5))
            pos = int(rng.integers(0, len(h) + 1))
            if op == 0 and h:
                h[min(pos, len(h) - 1)] ^= 1 << int(rng.integers(0, 8))
            elif op == 1:
                h = h[:pos]
            elif op == 2:
                h[pos:pos] = bytes([alphabet[int(rng.integers(0, len(alphabet)))]])
            elif op == 3 and h:
                del h[min(pos, len(h) - 1)]
            else:
                h[pos:pos] = _nest("[" if rng.integers(0, 2) else "{", int(rng.integers(100, 5000)))
        _raw_header_file(g, bytes(h), payload)
        for load in (_load, _load_ffn):
            rc, msg = load([g])
            assert rc in (0, 3, 4, 5), (it, rc, msg)
            if rc == 4:
                assert msg.startswith(f"loading {g}: "), (it, msg)


def test_well_formed_edge_headers_pass_the_parser(tmp_path):
    # whitespace padding after the JSON, __metadata__, and an empty tensor are
    # all legal; the checkpoint is then complete and loading reaches the device
    f = str(tmp_path / "ok.safetensors")
    t = _checkpoint(f, 2, 16, 8)
    from safetensors.numpy import load_file
    back = load_file(f)
    assert set(back) == set(t)
    import json
    raw = open(f, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8:8 + n])
    hdr["__metadata__"] = {"format": "pt"}
    hdr["zz.empty"] = {"dtype": "F32", "shape": [0, 3], "data_offsets": [len(raw) - 8 - n] * 2}
    _raw_safetensors(f, hdr, raw[8 + n:], pad=b"    ")
    rc, msg = _load([f])
    import torch
    assert rc == (0 if torch.cuda.is_available() else 5), msg
