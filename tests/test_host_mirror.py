"""The Python mirror's argument checks -- CPU only.

A caller-supplied `out` must be rejected before the library is called when its
shape, dtype, layout or device differ from what the kernels write (otherwise
the kernels would write past its end or into the wrong memory).  The library
is replaced by a stub that fails the test if any entry point is reached.
"""
import pytest
import torch

import nomas_moe as nm
from nomas_moe import _lib


class _NoLib:
    def __getattr__(self, name):
        raise AssertionError(f"library called: {name}")


@pytest.fixture
def no_lib(monkeypatch):
    monkeypatch.setattr(_lib, "lib", lambda: _NoLib())


def _fake(cls, dim=16, dtype=nm.DataType.F32):
    layer = object.__new__(cls)
    layer._h = None  # close() / __del__ do nothing
    layer.dim, layer.hidden, layer.dtype, layer.device = dim, 32, dtype, 0
    return layer


BAD_OUTS = {
    "rows": lambda x: torch.empty(x.shape[0] - 1, x.shape[1], dtype=x.dtype),
    "shape": lambda x: torch.empty(x.numel(), dtype=x.dtype),  # same numel, other shape
    "dtype": lambda x: torch.empty(x.shape, dtype=torch.float16),
    "strided": lambda x: torch.empty(x.shape[1], x.shape[0], dtype=x.dtype).t(),
    "device": lambda x: torch.empty(x.shape, dtype=x.dtype, device="meta"),
    "not_a_tensor": lambda x: x.numpy(),
}


@pytest.mark.parametrize("cls", [nm.MoeLayer, nm.FeedForward])
@pytest.mark.parametrize("bad", sorted(BAD_OUTS))
def test_bad_out_is_rejected_before_the_library(no_lib, cls, bad):
    layer = _fake(cls)
    x = torch.randn(8, 16)
    with pytest.raises(nm.NomasError) as ei:
        layer.forward(x, out=BAD_OUTS[bad](x))
    assert ei.value.code == 2


@pytest.mark.parametrize("cls", [nm.MoeLayer, nm.FeedForward])
def test_good_out_reaches_the_library(no_lib, cls):
    layer = _fake(cls)
    x = torch.randn(2, 4, 16)
    with pytest.raises(AssertionError, match="library called"):
        layer.forward(x, out=torch.empty(2, 4, 16))
    with pytest.raises(AssertionError, match="library called"):
        layer.forward(x)  # out allocated by the mirror


@pytest.mark.parametrize("cls", [nm.MoeLayer, nm.FeedForward])
def test_input_checks_come_first(no_lib, cls):
    layer = _fake(cls)
    with pytest.raises(nm.NomasError, match="last dim"):
        layer.forward(torch.randn(4, 8))
    with pytest.raises(nm.NomasError, match="dtype"):
        layer.forward(torch.randn(4, 16, dtype=torch.float64))
