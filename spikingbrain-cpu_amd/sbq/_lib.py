"""ctypes binding of libsbq.so (the C ABI declared in include/sbq.h).

The library is loaded from this package directory; a missing or unloadable
library raises immediately - there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsbq.so"

SBQ_OK = 0
SBQ_F32, SBQ_F16, SBQ_BF16 = 0, 1, 2
SBQ_NOALLOC_XQ_BYTES = 8 << 20  # include/sbq.h
SBQ_ARGMAX_WS_BYTES = 16640  # include/sbq.h
SBQ_MAX_GROUP = 4  # linears per sbq_linear_w8_grouped / sbq_linear_w8a8_grouped call (include/sbq.h)

# Every entry point declared in include/sbq.h, with its ctypes signature.
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_S = ctypes.c_size_t
SIGNATURES = {
    "sbq_version": (ctypes.c_char_p, []),
    "sbq_status_string": (ctypes.c_char_p, [_I]),
    "sbq_check_device": (_I, []),
    "sbq_quantize_per_channel": (_I, [_P, _I, _L, _L, _L, _P, _L, _P, _P]),
    "sbq_packed_bytes": (_L, [_L, _L]),
    "sbq_repack_w8": (_I, [_P, _L, _L, _L, _P, _P, _P]),
    "sbq_unpack_w8": (_I, [_P, _L, _L, _P, _L, _P]),
    "sbq_linear_w8": (_I, [_P, _I, _L, _L, _L, _P, _P, _P, _L, _P, _I, _L, _P, _S, _P]),
    "sbq_linear_w8_grouped": (_I, [_I, _P, _P, _I, _L, _L, _P, _P, _P, _P, _P, _P, _I, _P]),
    "sbq_w8_workspace_bytes": (_L, [_L, _L, _I]),
    "sbq_w8a8_workspace_bytes": (_L, [_L, _L]),
    "sbq_linear_workspace_bytes": (_L, [_L, _L, _L, _I, _I]),
    "sbq_gemm_config": (_I, [_L, _L, _L, _I, _I, _P]),
    "sbq_gemv_config": (_I, [_L, _L, _I, _I, _P]),
    "sbq_act_qparams": (_I, [_P, _I, _L, _L, _L, _P, _P, _P, _S, _P]),
    "sbq_act_quant_per_tensor": (_I, [_P, _I, _L, _L, _L, _P, _L, _P, _P, _P, _S, _P]),
    "sbq_linear_w8a8": (_I, [_P, _I, _L, _L, _L, _P, _P, _P, _P, _L, _P, _I, _L, _P, _P, _S, _P]),
    "sbq_linear_w8a8_grouped": (_I, [_I, _P, _P, _I, _L, _L, _P, _P, _P, _P, _P, _P, _P, _I, _P, _S, _P]),
    "sbq_linear_w8a8_token": (_I, [_P, _I, _L, _L, _L, _P, _P, _P, _L, _P, _I, _L, _P, _P, _S, _P]),
    "sbq_linear_w8a8_noalloc": (_I, [_P, _I, _L, _L, _L, _P, _P, _P, _P, _L, _P, _I, _L, _P, _P]),
    "sbq_argmax_rows": (_I, [_P, _L, _L, _L, _P, _P]),
    "sbq_linear_w8_argmax": (_I, [_P, _I, _L, _L, _L, _P, _P, _P, _L, _P, _L, _P, _P, _S, _P, _P]),
    "sbq_linear_w8a8_argmax": (_I, [_P, _I, _L, _L, _L, _P, _P, _P, _P, _L, _P, _L, _P, _P, _S, _P, _P]),
    "sbq_sample_workspace_bytes": (_L, [_L, _L]),
    "sbq_sample_rows": (_I, [_P, _L, _L, _L, ctypes.c_float, _L, ctypes.c_float, _P, _P, _P, _S, _P]),
}

_lib = None


class SbqError(RuntimeError):
    """A libsbq entry point returned a non-zero status."""


def _hip_runtimes_mapped() -> set[str]:
    try:
        with open("/proc/self/maps") as f:
            return {line.split()[-1] for line in f if "libamdhip64" in line}
    except OSError:
        return set()


def load() -> ctypes.CDLL:
    """Load libsbq.so after torch, so that the library binds to the HIP runtime
    torch already mapped (both carry the soname libamdhip64.so.7): one
    runtime per process, so torch's streams and allocations are valid here."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  (must map its HIP runtime first)

        if not LIB_PATH.exists():
            raise ImportError(
                f"libsbq.so not found at {LIB_PATH}; build it with `make -C spikingbrain-cpu_amd` "
                "(or __graft_entry__.build())")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise ImportError("two HIP runtimes are mapped in this process: " + ", ".join(sorted(runtimes)))
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != SBQ_OK:
        msg = load().sbq_status_string(status).decode()
        if status in (-1, -2, -3, -4):
            raise ValueError(f"{what}: {msg} (status {status})")
        raise SbqError(f"{what}: {msg} (status {status})")
