"""CPU oracle for the quantized-linear path (TEST INFRASTRUCTURE ONLY).

This package is the oracle the HIP kernels are compared against.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import it; the product package (``sbq``) never does, and it never stands
in for a GPU result.

Two layers, each citing the reference (paths relative to the reference
repository):

* ``_build/libsbq_oracle.so`` (``sbq_oracle.c``): plain-C restatement with
  explicit IEEE roundings - ``quantize_per_channel`` (quant.py:25-29),
  ``Int8Linear.forward`` (quant.py:41-53), and the fbgemm dynamic linear that
  ``DynamicInt8Linear.forward`` calls (quant.py:63-66).
* numpy wrappers below with the same arithmetic, using float64 matmul for the
  exact integer / near-exact dot products so that large shapes finish fast.

How each function is pinned (tests/test_oracle.py):

* ``quantize_per_channel``: C vs numpy vs torch CPU ops (the reference's own
  expression); all-zero rows, exact .5 ties, bf16 inputs.
* ``int8_linear``: integer-valued activations (every dot product exact, so the
  result is fixed by "scale after the sum"), scale-before-sum and
  transposed-operand mutants must fail, torch float64 matmul agreement.
* ``choose_qparams`` / ``quantize_act`` / ``dyn_linear``: bit-exact against the
  live ``torch.ops.quantized.linear_dynamic`` (fbgemm) across shapes, seeds,
  outliers, all-zero, tiny-range, one-signed and constant inputs; against the
  committed golden fixtures in tests/golden/; mutants (mul-then-round
  quantization, (acc*s_x)*s_w epilogue) must fail.
* ``dyn_linear_token`` (per-token symmetric W8A8, an opt-in granularity with
  no counterpart in the reference): its quantizer is ``quantize_per_channel``
  applied to activation rows (pinned above), the int32 product is checked
  against ``torch._int_mm``, and per-tensor-scale and (acc*s_t)*s_w epilogue
  mutants must fail.
* ``sample_probs`` / ``sample_token`` (the engine's sample, engine.py:29-42,
  with the caller's uniform in place of torch.multinomial's generator):
  against the reference's own expression evaluated with torch CPU ops (topk,
  masked_fill, softmax, sort, cumsum, scatter); the defining properties (the
  kept mass reaches top_p and the smallest kept token is needed for it, top_k
  = 1 keeps the argmax, ties at the k-th value are kept); inverse-CDF draw
  frequencies over a fine grid of uniforms; mutants (inclusive cumsum, ties
  dropped at the k-th value, temperature multiplied) must fail.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libsbq_oracle.so"
_lib = None


def build(force: bool = False) -> Path:
    """Compile the C oracle with the committed Makefile (gcc)."""
    import subprocess

    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-C", str(_HERE), "-B" if force else "-s"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        I = ctypes.c_int64
        L.oracle_quantize_per_channel.argtypes = [P, I, I, P, P]
        L.oracle_int8_linear.argtypes = [P, I, I, P, P, P, I, P]
        L.oracle_choose_qparams.argtypes = [ctypes.c_float, ctypes.c_float, P, P]
        L.oracle_quantize_act.argtypes = [P, I, ctypes.c_float, ctypes.c_int32, P]
        L.oracle_dyn_linear.argtypes = [P, I, I, P, P, P, I, P, P, P, P, P]
        L.oracle_dyn_epilogue.argtypes = [P, I, I, ctypes.c_float, P, P, P]
        L.oracle_dyn_epilogue_token.argtypes = [P, I, I, P, P, P, P]
        for f in ("oracle_quantize_per_channel", "oracle_int8_linear", "oracle_choose_qparams",
                  "oracle_quantize_act", "oracle_dyn_linear", "oracle_dyn_epilogue", "oracle_dyn_epilogue_token"):
            getattr(L, f).restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ---------------------------------------------------------------------------
# quant.py:25-29 quantize_per_channel
# ---------------------------------------------------------------------------
def quantize_per_channel_c(w) -> tuple[np.ndarray, np.ndarray]:
    w = _f32(w)
    N, K = w.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N,), np.float32)
    lib().oracle_quantize_per_channel(_ptr(w), N, K, _ptr(q), _ptr(s))
    return q, s


def quantize_per_channel(w) -> tuple[np.ndarray, np.ndarray]:
    """numpy restatement of quant.py:25-29 (fp32 IEEE divisions, rint = half-even)."""
    w = _f32(w)
    amax = np.abs(w).max(axis=1)
    scale = (np.maximum(amax, np.float32(1e-8)) / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint(w / scale[:, None]), -127, 127).astype(np.int8)
    return q, scale


# ---------------------------------------------------------------------------
# quant.py:41-53 Int8Linear.forward
# ---------------------------------------------------------------------------
def int8_linear_c(x, q, scale, bias=None) -> np.ndarray:
    x = _f32(x)
    q = np.ascontiguousarray(q, dtype=np.int8)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float32)
    b = None if bias is None else _f32(bias)
    lib().oracle_int8_linear(_ptr(x), M, K, _ptr(q), _ptr(_f32(scale)), _ptr(b), N, _ptr(y))
    return y


def int8_linear(x, q, scale, bias=None) -> np.ndarray:
    """y = fp32(sum_k x*q) * scale (+ bias); the scale multiplies the finished
    dot product, as quant.py:50 does after the block matmuls."""
    x = _f32(x)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1]).astype(np.float64)
    acc = (x2 @ np.asarray(q, np.float64).T).astype(np.float32)
    out = acc * _f32(scale)
    if bias is not None:
        out = out + _f32(bias)
    return out.reshape(*shape[:-1], -1)


# ---------------------------------------------------------------------------
# quant.py:63-66 DynamicInt8Linear.forward (fbgemm linear_dynamic)
# ---------------------------------------------------------------------------
def choose_qparams(xmin: float, xmax: float) -> tuple[float, int]:
    s = ctypes.c_float()
    z = ctypes.c_int32()
    lib().oracle_choose_qparams(ctypes.c_float(xmin), ctypes.c_float(xmax), ctypes.byref(s),
                                ctypes.byref(z))
    return float(np.float32(s.value)), int(z.value)


def quantize_act(x, scale: float, zp: int) -> np.ndarray:
    x = _f32(x)
    xq = np.empty(x.shape, np.uint8)
    lib().oracle_quantize_act(_ptr(x), x.size, ctypes.c_float(scale), ctypes.c_int32(zp), _ptr(xq))
    return xq


def act_qparams(x) -> tuple[float, int]:
    x = _f32(x)
    return choose_qparams(float(x.min()), float(x.max()))


def dyn_linear(x, q, scale, bias=None, return_intermediates: bool = False):
    """Bit-exact restatement of linear_dynamic(x.float(), prepack(q, scale)).

    The integer GEMM runs as a float64 matmul, exact because every partial
    sum is an integer below 2**53."""
    x = _f32(x)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    sx, zp = act_qparams(x2)
    xq = quantize_act(x2, sx, zp)
    acc64 = (xq.astype(np.float64) - zp) @ np.asarray(q, np.float64).T
    acc = np.ascontiguousarray(acc64.astype(np.int64).astype(np.int32))
    y = dyn_epilogue(acc, sx, scale, bias).reshape(*shape[:-1], -1)
    if return_intermediates:
        return y, {"scale": sx, "zero_point": zp, "xq": xq, "acc": acc}
    return y


def dyn_epilogue(acc, sx: float, scale, bias=None) -> np.ndarray:
    """fp32(acc) * fp32(s_x*scale[n]); with a bias one fused multiply-add,
    which is what fbgemm's float output stage computes."""
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    y = np.empty((M, N), np.float32)
    b = None if bias is None else _f32(bias)
    lib().oracle_dyn_epilogue(_ptr(acc), M, N, ctypes.c_float(sx), _ptr(_f32(scale)), _ptr(b), _ptr(y))
    return y


def dyn_linear_c(x, q, scale, bias=None):
    x = _f32(x)
    q = np.ascontiguousarray(q, dtype=np.int8)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float32)
    acc = np.empty((M, N), np.int32)
    xq = np.empty((M, K), np.uint8)
    sx = np.zeros(1, np.float32)
    zp = np.zeros(1, np.int32)
    b = None if bias is None else _f32(bias)
    lib().oracle_dyn_linear(_ptr(x), M, K, _ptr(q), _ptr(_f32(scale)), _ptr(b), N, _ptr(y),
                            _ptr(acc), _ptr(xq), _ptr(sx), _ptr(zp))
    return y, {"scale": float(sx[0]), "zero_point": int(zp[0]), "xq": xq, "acc": acc}


# ---------------------------------------------------------------------------
# Per-token symmetric W8A8 (opt-in granularity; not the reference's int8-dyn)
# ---------------------------------------------------------------------------
def dyn_linear_token(x, q, scale, bias=None, return_intermediates: bool = False):
    """Each activation row quantized as quant.py:25-29 quantizes a weight row,
    acc = sum_k xq * q in int32 (exact here as float64), then
    y = fp32(acc) * fp32(s_t[m] * scale[n]), with a bias one fused multiply-add."""
    x = _f32(x)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    xq, st = quantize_per_channel(x2)
    acc64 = xq.astype(np.float64) @ np.asarray(q, np.float64).T
    acc = np.ascontiguousarray(acc64.astype(np.int64).astype(np.int32))
    M, N = acc.shape
    y = np.empty((M, N), np.float32)
    b = None if bias is None else _f32(bias)
    lib().oracle_dyn_epilogue_token(_ptr(acc), M, N, _ptr(_f32(st)), _ptr(_f32(scale)), _ptr(b), _ptr(y))
    y = y.reshape(*shape[:-1], -1)
    if return_intermediates:
        return y, {"scale": st, "xq": xq, "acc": acc}
    return y


# ---------------------------------------------------------------------------
# Packed weight layout (the build's own format; see include/sbq.h)
# ---------------------------------------------------------------------------
def pack_w8(q) -> np.ndarray:
    """Reference model of sbq_repack_w8: [N/16][K/64] tiles of 1 KiB, byte
    lane*16+j (lane = g*16+r) = q[nt*16+r][kc*64+g*16+j] ^ 0x80, zero-padded."""
    q = np.asarray(q, np.int8)
    N, K = q.shape
    Np, Kp = -(-N // 16) * 16, -(-K // 64) * 64
    pad = np.zeros((Np, Kp), np.int8)
    pad[:N, :K] = q
    u = (pad.view(np.uint8) ^ 0x80).reshape(Np // 16, 16, Kp // 64, 4, 16)  # nt, r, kc, g, j
    return np.ascontiguousarray(u.transpose(0, 2, 3, 1, 4)).reshape(-1)      # nt, kc, g, r, j


def rel_l2(a, b) -> float:
    """||a - b|| / ||b|| (tools/upstream-reference/upstream_reference.py:282-283)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def cpu_threads() -> int:
    return len(os.sched_getaffinity(0))


def sample_probs(logits, temperature: float, top_k: int = 0, top_p: float = 1.0) -> np.ndarray:
    """engine.py:32-41 for one row of logits: the (unnormalized) probabilities
    the reference hands to torch.multinomial, float32 [V].  fp32 division by
    the temperature; top-k masks z below the k-th largest to -inf (ties with
    it stay); softmax (exp and sum in float64, rounded to fp32); top-p keeps a
    token in the descending order while cumsum - p < top_p, with torch CPU's
    cumsum (float64 accumulation, fp32 results) and a stable sort."""
    x = np.asarray(logits, np.float32)
    z = (x / np.float32(temperature)).astype(np.float32)
    if top_k > 0:
        k = min(int(top_k), z.size)
        kth = np.sort(z)[-k]
        z = np.where(z < kth, np.float32(-np.inf), z).astype(np.float32)
    m = z.max()
    e = np.exp((z - m).astype(np.float32).astype(np.float64))
    p = (e / e.sum()).astype(np.float32)
    if 0 < top_p < 1:
        order = np.argsort(-p, kind="stable")
        sp = p[order]
        csum = np.cumsum(sp.astype(np.float64)).astype(np.float32)
        keep = (csum - sp) < np.float32(top_p)
        out = np.zeros_like(p)
        out[order] = sp * keep
        p = out
    return p


def sample_token(logits, temperature: float, top_k: int = 0, top_p: float = 1.0, u: float = 0.5) -> int:
    """engine.py:29-42 with the draw made from the uniform u in [0, 1): the
    greedy token for temperature <= 0; otherwise the first index whose prefix
    of sample_probs exceeds u times their sum (the inverse of the distribution
    torch.multinomial samples).  -1 where the reference raises: a NaN logit,
    or an infinite maximum after the division."""
    x = np.asarray(logits, np.float32)
    if temperature <= 0:
        nan = np.flatnonzero(np.isnan(x))
        return int(nan[0]) if nan.size else int(np.argmax(x))
    z = (x / np.float32(temperature)).astype(np.float32)
    if np.isnan(z).any() or not np.isfinite(z.max()):
        return -1
    c = np.cumsum(sample_probs(x, temperature, top_k, top_p).astype(np.float64))
    return int(np.searchsorted(c, u * c[-1], side="right"))

