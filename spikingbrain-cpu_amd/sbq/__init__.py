"""sbq - the quantized-linear hot path of spikingbrain-cpu on MI355X (gfx950).

``sbq.quant`` is the drop-in for ``spikingbrain_cpu/quant.py``; ``sbq._lib`` is
the ctypes binding of libsbq.so (C ABI: include/sbq.h).
"""
from .quant import (FORMATS, BF16Linear, DynamicInt8Linear, FloatLinear, FP16Linear, FusedLinear, Int8Linear,
                    act_quant_per_tensor, fuse_linears, greedy_tokens, linear_w8a8_token, load_quantized, make_linear,
                    quantize_per_channel, sample, sample_tokens, save_quantized)

__version__ = "0.1.0"

__all__ = ["FORMATS", "BF16Linear", "DynamicInt8Linear", "FloatLinear", "FP16Linear", "FusedLinear", "Int8Linear",
           "act_quant_per_tensor", "fuse_linears", "greedy_tokens", "linear_w8a8_token", "load_quantized", "make_linear",
           "quantize_per_channel", "sample", "sample_tokens", "save_quantized"]
