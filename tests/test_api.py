"""CPU checks of the drop-in Python surface (spikingbrain_cpu/quant.py API)."""
import pytest
import torch

import sbq
from sbq import quant


def test_formats_match_reference():
    # quant.py:22
    assert quant.FORMATS == ("float32", "bfloat16", "float16", "int8", "int8-dyn")
    assert sbq.FORMATS is quant.FORMATS


def test_unknown_format_raises_value_error_like_reference():
    # quant.py:111
    with pytest.raises(ValueError, match="^unknown weight format bogus$"):
        quant.make_linear("bogus", torch.zeros(4, 4))


def test_public_names():
    for name in ("quantize_per_channel", "Int8Linear", "DynamicInt8Linear", "FP16Linear", "BF16Linear",
                 "FloatLinear", "make_linear", "fuse_linears", "FusedLinear"):
        assert hasattr(quant, name)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
@pytest.mark.parametrize("fmt", ["int8", "int8-dyn"])
def test_no_cpu_fallback(fmt):
    """Without a GPU the quantized formats refuse to build: there is no CPU path."""
    with pytest.raises(RuntimeError, match="no ROCm GPU"):
        quant.make_linear(fmt, torch.randn(8, 64))
    with pytest.raises(RuntimeError, match="no ROCm GPU"):
        quant.quantize_per_channel(torch.randn(8, 64))


def test_fuse_linears_needs_quantized_parts():
    with pytest.raises(ValueError):
        quant.fuse_linears([])
    with pytest.raises(ValueError):
        quant.fuse_linears([torch.nn.Linear(4, 4)])
