"""Golden fixtures (tests/golden/) against the oracle and the product's generator -- CPU only."""
import json
import os

import numpy as np
import pytest

import nomas_moe as nm
import oracle as O
from golden_cases import CASES, build_case

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _kat():
    with open(os.path.join(GOLDEN, "generator_kat.json")) as f:
        return json.load(f)


def test_generator_fixture_matches_oracle_and_library():
    kat = _kat()
    for s, vals in kat["splitmix64"].items():
        assert [f"{v:016x}" for v in O.splitmix64(int(s), 8)] == vals
    for key, h in kat["path_seed"].items():
        seed, path = key.split(":", 1)
        assert f"{O.path_seed(int(seed), path):016x}" == h
        assert f"{nm.path_seed(int(seed), path):016x}" == h  # the library's path_seed
    for s, bits in kat["randn_f32_bits"].items():
        want = [int(b, 16) for b in bits]
        assert O.randn_affine(int(s), 17).view(np.uint32).tolist() == want
        assert nm.randn_affine(int(s), 17).view(np.uint32).tolist() == want


def test_library_generator_is_bit_identical_to_oracle_at_size():
    # multi-threaded in the library, sequential in the oracle: same bits
    for seed, mean, std in [(99, 0.0, 1.0), (0x5EED0002, 0.25, 0.02)]:
        a = nm.randn_affine(seed, 1_000_003, mean, std)
        b = O.randn_affine(seed, 1_000_003, mean, std)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    c = build_case(name)
    g = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    out, idx, w, gap = O.forward_sparse(c["x"], c["p"], c["k"], shared_dense=c["shared_dense"],
                                        dense=c["dense"])
    np.testing.assert_array_equal(idx, g["idx"])
    np.testing.assert_array_equal(np.bincount(idx.ravel(), minlength=c["E"]), g["counts"])
    np.testing.assert_allclose(out, g["out"], rtol=1e-13, atol=0)
    np.testing.assert_allclose(w, g["w"], rtol=1e-13, atol=0)
    np.testing.assert_allclose(gap, g["gap"], rtol=1e-13, atol=0)
