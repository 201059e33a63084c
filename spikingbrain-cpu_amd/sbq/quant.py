"""Weight storage formats for linear layers, MI355X (gfx950) edition.

Drop-in for ``spikingbrain_cpu/quant.py`` (same names, arguments, attributes
and errors; paths relative to the reference repository).  The two quantized
formats run on hand-written gfx950 kernels through libsbq.so:

``int8``      symmetric per-output-channel int8 weights with fp32 scales,
              weight-only (quant.py:32-53).  Decode shapes stream the packed
              weights from HBM through MFMA; prefill shapes use an LDS-tiled
              MFMA GEMM.  fp16/bf16 activations are used exactly; fp32
              activations as bf16 high + remainder planes at decode sizes
              and as one power-of-two scaled fp16 plane in the GEMM.
``int8-dyn``  int8 weights with activations quantized per tensor at run time
              (quant.py:56-66): the fbgemm dynamic-linear arithmetic,
              reproduced bit for bit (uint8 activations, exact int32
              accumulation on i8 MFMA, fp32 epilogue).
``float32`` / ``bfloat16`` / ``float16``
              plain torch GPU linears kept so that ``make_linear`` accepts every
              format the reference does; they are not part of the quantized
              path.

Device placement: modules are built on the GPU that holds the weight (the
current GPU for a CPU weight).  ``forward`` accepts a GPU tensor on that device
or a CPU tensor; a CPU input is copied to the GPU and the result copied back,
so the module also works inside the CPU-resident reference model.  Without a
ROCm GPU every entry point raises: there is no CPU implementation here.
"""
from __future__ import annotations

import ctypes
import weakref

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib

FORMATS = ("float32", "bfloat16", "float16", "int8", "int8-dyn")

_DTYPE_CODE = {torch.float32: _lib.SBQ_F32, torch.float16: _lib.SBQ_F16, torch.bfloat16: _lib.SBQ_BF16}


# ---------------------------------------------------------------------------
# device plumbing
# ---------------------------------------------------------------------------
def _gpu_for(t: torch.Tensor) -> torch.device:
    if t.is_cuda:
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("sbq: no ROCm GPU is available; the quantized formats run only on gfx950 GPUs")
    return torch.device("cuda", torch.cuda.current_device())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"sbq: unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def _as_activation(x2: torch.Tensor) -> torch.Tensor:
    """x2 [M, K] with unit column stride and rows that do not overlap (the
    kernels read row m at m * ldx).  Broadcast rows (stride 0, from expand)
    and other overlapping layouts are copied; one row is passed as it is."""
    if x2.dtype not in _DTYPE_CODE:
        x2 = x2.float()
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < x2.shape[1]):
        x2 = x2.contiguous()
    return x2


def _ldx(x2: torch.Tensor) -> int:
    """Row stride to pass for a 2-D operand with unit column stride (an
    activation from _as_activation, an output, a weight): a single row is
    contiguous whatever its stride(0) says (e.g. a transposed [K, 1])."""
    return x2.shape[1] if x2.shape[0] <= 1 else x2.stride(0)


def packed_bytes(N: int, K: int) -> int:
    """Size of the packed tiles of an int8 [N, K] weight (sbq_packed_bytes)."""
    return ((N + 15) // 16) * 16 * ((K + 63) // 64) * 64


def _check_operands(fn: str, x2: torch.Tensor, packed: torch.Tensor, N: int, y: torch.Tensor,
                    vectors: tuple = (), ws: torch.Tensor | None = None) -> None:
    """The sizes, dtypes and devices the kernels assume: the C ABI sees raw
    pointers only, so a short buffer here would be read or written out of
    bounds on the GPU.  vectors: (name, tensor or None, dtype) of the [N]
    per-channel operands."""
    M, K = x2.shape
    dev = x2.device
    if not x2.is_cuda:
        raise ValueError(f"{fn}: x must be a GPU tensor")
    if N < 1:
        raise ValueError(f"{fn}: N must be >= 1")
    need = packed_bytes(N, K)
    if (packed.dtype != torch.uint8 or packed.device != dev or not packed.is_contiguous()
            or packed.numel() < need):
        raise ValueError(f"{fn}: packed must be contiguous uint8 on {dev} with >= {need} bytes (N={N}, K={K})")
    for name, t, dt in vectors:
        if t is not None and (t.dtype != dt or t.device != dev or not t.is_contiguous() or t.numel() < N):
            raise ValueError(f"{fn}: {name} must be a contiguous {dt} tensor of N={N} elements on {dev}")
    if y.device != dev or y.dim() != 2 or tuple(y.shape) != (M, N) or y.stride(-1) != 1:
        raise ValueError(f"{fn}: out must be a [M={M}, N={N}] tensor with unit column stride on {dev}")
    if ws is not None and (ws.device != dev or not ws.is_contiguous()):
        raise ValueError(f"{fn}: workspace must be a contiguous tensor on {dev}")


def _nbytes(t: torch.Tensor | None) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def _check_in_features(x: torch.Tensor, K: int) -> None:
    # torch's matmul in the reference forward raises RuntimeError on this
    if x.dim() == 0 or x.shape[-1] != K:
        raise RuntimeError(f"sbq: input of shape {tuple(x.shape)} does not end in in_features={K}")


# ---------------------------------------------------------------------------
# functional API over the C ABI (GPU tensors in, GPU tensors out)
# ---------------------------------------------------------------------------
def quantize_per_channel_gpu(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """quant.py:25-29 on the GPU: (int8 [N,K], fp32 scale [N])."""
    if weight.dim() != 2:
        raise ValueError("quantize_per_channel expects a 2-D weight")
    w = weight if weight.dtype in _DTYPE_CODE else weight.float()
    if w.stride(-1) != 1:
        w = w.contiguous()
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    scale = torch.empty((N,), dtype=torch.float32, device=w.device)
    with torch.cuda.device(w.device):
        _lib.check(_lib.load().sbq_quantize_per_channel(_ptr(w), _code(w.dtype), N, K, _ldx(w), _ptr(q),
                                                        _ldx(q), _ptr(scale), _stream(w.device)),
                   "sbq_quantize_per_channel")
    return q, scale


def repack(q: torch.Tensor, with_colsum: bool = True) -> tuple[torch.Tensor, torch.Tensor | None]:
    """int8 [N,K] (GPU) -> (packed uint8 tiles, int32 colsum [N] or None)."""
    if q.dtype != torch.int8 or q.dim() != 2 or not q.is_cuda:
        raise ValueError("repack expects a 2-D int8 GPU tensor")
    if q.stride(-1) != 1:
        q = q.contiguous()
    N, K = q.shape
    L = _lib.load()
    packed = torch.empty((L.sbq_packed_bytes(N, K),), dtype=torch.uint8, device=q.device)
    colsum = torch.empty((N,), dtype=torch.int32, device=q.device) if with_colsum else None
    with torch.cuda.device(q.device):
        _lib.check(L.sbq_repack_w8(_ptr(q), N, K, _ldx(q), _ptr(packed), _ptr(colsum), _stream(q.device)),
                   "sbq_repack_w8")
    return packed, colsum


def unpack(packed: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """Packed tiles -> int8 [N, K] (the inverse of repack)."""
    if (packed.dtype != torch.uint8 or not packed.is_cuda or not packed.is_contiguous()
            or packed.numel() < packed_bytes(N, K)):
        raise ValueError(f"unpack expects contiguous uint8 GPU tiles of >= {packed_bytes(N, K)} bytes")
    q = torch.empty((N, K), dtype=torch.int8, device=packed.device)
    with torch.cuda.device(packed.device):
        _lib.check(_lib.load().sbq_unpack_w8(_ptr(packed), N, K, _ptr(q), K, _stream(packed.device)),
                   "sbq_unpack_w8")
    return q


def w8_workspace(M: int, K: int, device: torch.device, dtype: torch.dtype = torch.float16,
                 N: int | None = None) -> torch.Tensor:
    """Scratch for linear_w8's prefill path with [M, K] activations of `dtype`;
    with N, also the split-K partials of shapes that need them."""
    L = _lib.load()
    n = L.sbq_w8_workspace_bytes(M, K, _code(dtype)) if N is None else L.sbq_linear_workspace_bytes(
        M, N, K, _code(dtype), 0)
    return torch.empty((n,), dtype=torch.uint8, device=device)


def linear_w8(x2: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None, N: int,
              out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None,
              workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y = (x2 @ q^T) * scale (+ bias) for x2 [M, K] on the GPU.

    Prefill-sized inputs (M > 16) get the scratch of the fastest GEMM path
    (row sums; staged fp16 planes for fp32 / bf16 activations) unless the
    caller passes one; the library itself never allocates."""
    x2 = _as_activation(x2)
    M, K = x2.shape
    y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=x2.device)
    ws = workspace
    if ws is None and M > 16:  # decode sizes run the GEMV, which needs none
        ws = w8_workspace(M, K, x2.device, x2.dtype, N)
    _check_operands("linear_w8", x2, packed, N, y, (("scale", scale, torch.float32), ("bias", bias, torch.float32)),
                    ws)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sbq_linear_w8(_ptr(x2), _code(x2.dtype), M, K, _ldx(x2), _ptr(packed),
                                             _ptr(scale), _ptr(bias), N, _ptr(y), _code(y.dtype), _ldx(y),
                                             _ptr(ws), _nbytes(ws), _stream(x2.device)),
                   "sbq_linear_w8")
    return y


MAX_GROUP = _lib.SBQ_MAX_GROUP  # linears per grouped launch


def linear_w8_grouped(xs, packeds, scales, biases, Ns, out_dtype: torch.dtype = torch.float32, outs=None):
    """Independent weight-only linears of one step in one launch:
    ys[i] = linear_w8(xs[i], packeds[i], scales[i], biases[i], Ns[i]).

    All xs are [M, K] GPU tensors of one dtype and device, all outputs one
    dtype.  Decode shapes (M <= 16) run as a single GEMV launch over the
    summed rows (the per-launch ramp and tail paid once); other shapes run one
    by one.  Results can differ from separate calls in the fp32 summation
    order.  More than MAX_GROUP linears are split into groups."""
    return _run_grouped("linear_w8_grouped", xs, packeds, scales, None, biases, Ns, out_dtype, outs, None)


def linear_w8a8_grouped(xs, packeds, scales, colsums, biases, Ns, out_dtype: torch.dtype = torch.float32, outs=None,
                        workspace: torch.Tensor | None = None):
    """Independent int8-dyn linears of one step in one launch:
    ys[i] = linear_w8a8(xs[i], packeds[i], scales[i], colsums[i], biases[i],
    Ns[i]), each x quantized with its own (s_x, zp).

    Shapes as in linear_w8_grouped.  Decode shapes whose x fits the fused
    GEMV run as one launch; others run one by one, sharing `workspace`
    (default: allocated for [M, K]).  Bit-exact with separate calls."""
    return _run_grouped("linear_w8a8_grouped", xs, packeds, scales, colsums, biases, Ns, out_dtype, outs, workspace)


def _run_grouped(name, xs, packeds, scales, colsums, biases, Ns, out_dtype, outs, workspace):
    w8a8 = colsums is not None
    n = len(xs)
    if not (len(packeds) == len(scales) == len(biases) == len(Ns) == n) or (outs is not None and len(outs) != n) \
            or (w8a8 and len(colsums) != n):
        raise ValueError(f"{name}: the argument lists differ in length")
    if n == 0:
        return []
    xs = [_as_activation(x) for x in xs]
    M, K = xs[0].shape
    dev, xdt = xs[0].device, xs[0].dtype
    for x in xs:
        if tuple(x.shape) != (M, K) or x.device != dev or x.dtype != xdt:
            raise ValueError(f"{name}: every x must have the shape, dtype and device of xs[0]")
    ys = list(outs) if outs is not None else [torch.empty((M, N), dtype=out_dtype, device=dev) for N in Ns]
    ydt = ys[0].dtype
    if not w8a8 and M > 16:
        # no grouped launch past decode sizes: each linear runs as linear_w8
        # does on its own, with the prefill workspace it allocates (the C
        # entry point's one-by-one fallback has none, which for fp32 x is a
        # different, slower path)
        if any(y.dtype != ydt for y in ys):
            raise ValueError(f"{name}: every output must have one dtype")
        return [linear_w8(xs[i], packeds[i], scales[i], biases[i], Ns[i], out=ys[i]) for i in range(n)]
    ws = None
    if w8a8:
        ws = workspace if workspace is not None else w8a8_workspace(M, K, dev)
    for i in range(n):
        if ys[i].dtype != ydt:
            raise ValueError(f"{name}: every output must have one dtype")
        ops = (("scale", scales[i], torch.float32), ("bias", biases[i], torch.float32))
        if w8a8:
            ops += (("colsum", colsums[i], torch.int32),)
        _check_operands(name, xs[i], packeds[i], Ns[i], ys[i], ops, ws)
    L = _lib.load()
    for g0 in range(0, n, MAX_GROUP):
        idx = range(g0, min(n, g0 + MAX_GROUP))
        c = len(idx)
        arr = lambda ctype, vals: (ctype * c)(*vals)  # noqa: E731
        head = (c, arr(ctypes.c_void_p, [xs[i].data_ptr() for i in idx]), arr(ctypes.c_int64, [_ldx(xs[i]) for i in idx]),
                _code(xdt), M, K, arr(ctypes.c_void_p, [packeds[i].data_ptr() for i in idx]),
                arr(ctypes.c_void_p, [scales[i].data_ptr() for i in idx]))
        tail = (arr(ctypes.c_void_p, [0 if biases[i] is None else biases[i].data_ptr() for i in idx]),
                arr(ctypes.c_int64, [Ns[i] for i in idx]), arr(ctypes.c_void_p, [ys[i].data_ptr() for i in idx]),
                arr(ctypes.c_int64, [_ldx(ys[i]) for i in idx]), _code(ydt))
        with torch.cuda.device(dev):
            if w8a8:
                rc = L.sbq_linear_w8a8_grouped(*head, arr(ctypes.c_void_p, [colsums[i].data_ptr() for i in idx]),
                                               *tail, _ptr(ws), _nbytes(ws), _stream(dev))
            else:
                rc = L.sbq_linear_w8_grouped(*head, *tail, _stream(dev))
            _lib.check(rc, "sbq_" + name)
    return ys


def grouped_forward(pairs):
    """Outputs of several Int8Linear layers, or several per-tensor
    DynamicInt8Linear layers, on their own inputs [(layer, x), ...] as one
    grouped launch per MAX_GROUP layers: the drop-in for a model step that
    holds independent projections (model.py: lora_q[1] / lora_k[1], sse_o /
    swa_o of a hybrid layer).  Each output equals layer(x) (Int8Linear: to
    fp32 summation order; DynamicInt8Linear: bit for bit).  Mixed or other
    kinds of layers, or inputs of differing shape, run through their own
    forward."""
    layers = [m for m, _ in pairs]
    xs = [x for _, x in pairs]
    if not pairs:
        return []
    if all(isinstance(m, Int8Linear) and m.qweight.is_cuda for m in layers):
        dyn = False
    elif all(isinstance(m, DynamicInt8Linear) and m.packed.is_cuda
             and getattr(m, "granularity", "tensor") == "tensor" for m in layers):
        dyn = True
    else:
        return [m(x) for m, x in pairs]
    shape0, dev = xs[0].shape, layers[0].packed.device if dyn else layers[0].qweight.device
    if any(x.shape != shape0 or x.dtype != xs[0].dtype or x.device != dev or m.out_dtype != layers[0].out_dtype
           or (m.packed.device if dyn else m.qweight.device) != dev for m, x in pairs):
        return [m(x) for m, x in pairs]
    for m, x in pairs:
        _check_in_features(x, m.in_features)
        if not dyn:
            m._refresh()
    x2s = [x.reshape(-1, shape0[-1]) for x in xs]
    args = ([m.packed for m in layers], [m.scale if m.scale.dtype == torch.float32 else m.scale.float() for m in layers])
    rest = ([None if m.bias is None else m.bias.float() for m in layers], [m.out_features for m in layers],
            layers[0].out_dtype)
    if dyn:
        ys = linear_w8a8_grouped(x2s, *args, [m.colsum for m in layers], *rest)
    else:
        ys = linear_w8_grouped(x2s, *args, *rest)
    return [y.reshape(*shape0[:-1], y.shape[-1]) for y in ys]


def gemm_config(M: int, N: int, K: int, dtype: torch.dtype = torch.float16, w8a8: bool = False) -> tuple[int, int]:
    """(configuration id, K splits) of the tiled prefill GEMM for y [M, N] =
    x [M, K] * W^T as the int8 (w8a8=False) / int8-dyn linears run it with
    their default workspace (sbq_gemm_config; host-only, needs no GPU)."""
    L = _lib.load()
    splits = ctypes.c_int(0)
    rc = L.sbq_gemm_config(M, N, K, _code(dtype), int(bool(w8a8)), ctypes.byref(splits))
    if rc < 0:
        raise ValueError(f"gemm_config: {L.sbq_status_string(rc).decode()} (M={M}, N={N}, K={K})")
    return rc, splits.value


def w8a8_workspace(M: int, K: int, device: torch.device, N: int | None = None,
                   dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Scratch for the int8-dyn paths; with N, also the split-K partials of
    prefill shapes that need them."""
    L = _lib.load()
    n = L.sbq_w8a8_workspace_bytes(M, K) if N is None else L.sbq_linear_workspace_bytes(M, N, K, _code(dtype), 1)
    return torch.empty((n,), dtype=torch.uint8, device=device)


def linear_w8a8(x2: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, colsum: torch.Tensor,
                bias: torch.Tensor | None, N: int, out_dtype: torch.dtype = torch.float32,
                acc_out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """fbgemm dynamic linear (per-tensor asymmetric uint8 activations)."""
    x2 = _as_activation(x2)
    M, K = x2.shape
    y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=x2.device)
    ws = workspace if workspace is not None else w8a8_workspace(M, K, x2.device, N, x2.dtype)
    if acc_out is not None and (acc_out.dtype != torch.int32 or tuple(acc_out.shape) != (M, N)
                                or not acc_out.is_contiguous() or acc_out.device != x2.device):
        raise ValueError("acc_out must be a contiguous int32 [M, N] tensor on the input's device")
    _check_operands("linear_w8a8", x2, packed, N, y, (("scale", scale, torch.float32), ("bias", bias, torch.float32),
                                                      ("colsum", colsum, torch.int32)), ws)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sbq_linear_w8a8(_ptr(x2), _code(x2.dtype), M, K, _ldx(x2), _ptr(packed),
                                               _ptr(scale), _ptr(colsum), _ptr(bias), N, _ptr(y), _code(y.dtype),
                                               _ldx(y), _ptr(acc_out), _ptr(ws), _nbytes(ws),
                                               _stream(x2.device)),
                   "sbq_linear_w8a8")
    return y


def linear_w8a8_noalloc(x2: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, colsum: torch.Tensor,
                        bias: torch.Tensor | None, N: int, out: torch.Tensor,
                        acc_out: torch.Tensor | None = None) -> torch.Tensor:
    """linear_w8a8 with no workspace (sbq_linear_w8a8_noalloc): the library's
    static per-GPU scratch holds the activation statistics and quantized
    activations, and nothing is allocated, here or in the library; the caller
    supplies `out` (and `acc_out`).  x2 must already be a GPU tensor the
    kernels take as it is (fp32 / fp16 / bf16, unit column stride).  Calls that
    overlap on one GPU race on the shared scratch."""
    if x2.dim() != 2 or x2.dtype not in _DTYPE_CODE or x2.stride(-1) != 1 or (
            x2.shape[0] > 1 and x2.stride(0) < x2.shape[1]):
        raise ValueError("linear_w8a8_noalloc: x must be a 2-D fp32/fp16/bf16 tensor with unit column stride")
    M, K = x2.shape
    if acc_out is not None and (acc_out.dtype != torch.int32 or tuple(acc_out.shape) != (M, N)
                                or not acc_out.is_contiguous() or acc_out.device != x2.device):
        raise ValueError("acc_out must be a contiguous int32 [M, N] tensor on the input's device")
    _check_operands("linear_w8a8_noalloc", x2, packed, N, out, (("scale", scale, torch.float32),
                                                                 ("bias", bias, torch.float32),
                                                                 ("colsum", colsum, torch.int32)))
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sbq_linear_w8a8_noalloc(_ptr(x2), _code(x2.dtype), M, K, _ldx(x2), _ptr(packed),
                                                       _ptr(scale), _ptr(colsum), _ptr(bias), N, _ptr(out),
                                                       _code(out.dtype), _ldx(out), _ptr(acc_out),
                                                       _stream(x2.device)),
                   "sbq_linear_w8a8_noalloc")
    return out


def linear_w8a8_token(x2: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
                      N: int, out_dtype: torch.dtype = torch.float32, acc_out: torch.Tensor | None = None,
                      workspace: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-token symmetric W8A8 (opt-in; not the reference's int8-dyn): each
    activation row is quantized as quantize_per_channel quantizes a weight
    row, the int32 GEMM is exact, y = fp32(acc) * fp32(s_t[m] * scale[n])."""
    x2 = _as_activation(x2)
    M, K = x2.shape
    y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=x2.device)
    ws = workspace if workspace is not None else w8a8_workspace(M, K, x2.device)
    if acc_out is not None and (acc_out.dtype != torch.int32 or tuple(acc_out.shape) != (M, N)
                                or not acc_out.is_contiguous() or acc_out.device != x2.device):
        raise ValueError("acc_out must be a contiguous int32 [M, N] tensor on the input's device")
    _check_operands("linear_w8a8_token", x2, packed, N, y,
                    (("scale", scale, torch.float32), ("bias", bias, torch.float32)), ws)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sbq_linear_w8a8_token(_ptr(x2), _code(x2.dtype), M, K, _ldx(x2), _ptr(packed),
                                                     _ptr(scale), _ptr(bias), N, _ptr(y), _code(y.dtype),
                                                     _ldx(y), _ptr(acc_out), _ptr(ws), _nbytes(ws),
                                                     _stream(x2.device)),
                   "sbq_linear_w8a8_token")
    return y


def greedy_tokens(logits: torch.Tensor) -> torch.Tensor:
    """engine.py:30-31 on the GPU: int64 [...] of row argmaxes of fp32 logits
    [..., V] (first index of the maximum, NaN above every number)."""
    if logits.dtype != torch.float32 or not logits.is_cuda:
        raise ValueError("greedy_tokens expects fp32 GPU logits")
    shape = logits.shape
    y = logits.reshape(-1, shape[-1])
    if y.stride(-1) != 1 or (y.shape[0] > 1 and y.stride(0) < y.shape[1]):
        y = y.contiguous()
    ld = _ldx(y)
    out = torch.empty((y.shape[0],), dtype=torch.int64, device=y.device)
    with torch.cuda.device(y.device):
        _lib.check(_lib.load().sbq_argmax_rows(_ptr(y), y.shape[0], y.shape[1], ld, _ptr(out),
                                               _stream(y.device)), "sbq_argmax_rows")
    return out.reshape(shape[:-1])


def sample_workspace(M: int, V: int, device: torch.device) -> torch.Tensor:
    """Scratch of sample_tokens for M rows of V logits."""
    return torch.empty((_lib.load().sbq_sample_workspace_bytes(M, V),), dtype=torch.uint8, device=device)


def sample_tokens(logits: torch.Tensor, temperature: float, top_p: float = 1.0, top_k: int = 0,
                  u: torch.Tensor | None = None, generator: torch.Generator | None = None,
                  workspace: torch.Tensor | None = None) -> torch.Tensor:
    """engine.py:29-42 (`sample`) on the GPU: int64 [...] of tokens drawn from
    fp32 GPU logits [..., V] with the engine's temperature, top-k and top-p,
    one draw per row, without copying the logits to the host.

    temperature <= 0 is the greedy token (greedy_tokens).  Otherwise the draw
    takes one uniform in [0, 1) per row: `u` (fp32, on the logits' device), or
    torch.rand from `generator` (a CPU generator, as the engine passes, or one
    on the logits' device) - the randomness stays the caller's, as with
    torch.multinomial.  The top-p rule takes the tokens in the order of z
    (of two tokens of equal fp32 probability, whose order the reference's
    sort leaves open, the larger z first); of tokens whose z ties at the
    top-p boundary, as many as the rule admits are kept, the first ones in
    vocabulary order (a stable sort's order).
    A row with a NaN (or an infinite maximum after the division) gets -1, where
    the reference raises."""
    if logits.dtype != torch.float32 or not logits.is_cuda:
        raise ValueError("sample_tokens expects fp32 GPU logits")
    if temperature != temperature or top_p != top_p:
        raise ValueError("temperature and top_p must be numbers")
    if temperature <= 0:
        return greedy_tokens(logits)
    shape = logits.shape
    y = logits.reshape(-1, shape[-1])
    if y.stride(-1) != 1 or (y.shape[0] > 1 and y.stride(0) < y.shape[1]):
        y = y.contiguous()
    M, V = y.shape
    ld = _ldx(y)
    out = torch.empty((M,), dtype=torch.int64, device=y.device)
    if u is None:
        if generator is not None and generator.device.type == "cuda":
            u = torch.rand((M,), generator=generator, device=y.device)
        else:
            u = torch.rand((M,), generator=generator).to(y.device)
    if u.dtype != torch.float32 or u.device != y.device or u.numel() != M or not u.is_contiguous():
        raise ValueError("u must be a contiguous fp32 tensor of one uniform per row on the logits' device")
    ws = workspace if workspace is not None else sample_workspace(M, V, y.device)
    if ws.dtype != torch.uint8 or ws.device != y.device or not ws.is_contiguous():
        raise ValueError("workspace must be a contiguous uint8 tensor on the logits' device")
    with torch.cuda.device(y.device):
        _lib.check(_lib.load().sbq_sample_rows(_ptr(y), M, V, ld, float(temperature), int(top_k),
                                               float(top_p), _ptr(u), _ptr(out), _ptr(ws), _nbytes(ws),
                                               _stream(y.device)), "sbq_sample_rows")
    return out.reshape(shape[:-1])


def sample(logits: torch.Tensor, params, generator: torch.Generator | None = None) -> int:
    """Drop-in for the engine's sample(logits, params, generator)
    (engine.py:29-42) with the logits on the GPU: the same SamplingParams
    fields (temperature, top_k, top_p), one uniform drawn from `generator`,
    and only the token crosses to the host."""
    tok = sample_tokens(logits.reshape(1, -1), params.temperature, params.top_p, params.top_k,
                        generator=generator)
    return int(tok[0])


def argmax_state(device: torch.device) -> torch.Tensor:
    """The zeroed state (keys and count) of linear_w8_argmax /
    linear_w8a8_argmax: every call leaves it zero again, so one state serves
    every call on one stream."""
    return torch.zeros((_lib.SBQ_ARGMAX_WS_BYTES,), dtype=torch.uint8, device=device)


def _check_argmax(fn: str, x2: torch.Tensor, state: torch.Tensor, idx: torch.Tensor | None) -> torch.Tensor:
    M = x2.shape[0]
    if (state.dtype != torch.uint8 or state.device != x2.device or not state.is_contiguous()
            or state.numel() < _lib.SBQ_ARGMAX_WS_BYTES or state.data_ptr() % 8):
        raise ValueError(f"{fn}: argmax state must come from argmax_state() on {x2.device}")
    if idx is None:
        return torch.empty((M,), dtype=torch.int64, device=x2.device)
    if idx.dtype != torch.int64 or idx.device != x2.device or not idx.is_contiguous() or idx.numel() < M:
        raise ValueError(f"{fn}: idx must be a contiguous int64 tensor of M={M} elements on {x2.device}")
    return idx


def linear_w8_argmax(x2: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None, N: int,
                     state: torch.Tensor, out: torch.Tensor | None = None, idx: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """lm_head (model.py:445-447) and its greedy token (engine.py:30-31) in one
    pass: (fp32 logits [M, N], int64 token [M]), the token being the first
    index of each row's maximum with NaN above every number.  `state` comes
    from argmax_state() (one per stream).  The logits are linear_w8's (the
    same workspace rule for prefill sizes)."""
    x2 = _as_activation(x2)
    M, K = x2.shape
    y = out if out is not None else torch.empty((M, N), dtype=torch.float32, device=x2.device)
    if y.dtype != torch.float32:
        raise ValueError("linear_w8_argmax: the logits are fp32")
    ws = workspace
    if ws is None and M > 16:
        ws = w8_workspace(M, K, x2.device, x2.dtype, N)
    _check_operands("linear_w8_argmax", x2, packed, N, y, (("scale", scale, torch.float32),
                                                           ("bias", bias, torch.float32)), ws)
    idx = _check_argmax("linear_w8_argmax", x2, state, idx)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sbq_linear_w8_argmax(_ptr(x2), _code(x2.dtype), M, K, _ldx(x2), _ptr(packed),
                                                    _ptr(scale), _ptr(bias), N, _ptr(y), _ldx(y), _ptr(idx),
                                                    _ptr(ws), _nbytes(ws), _ptr(state), _stream(x2.device)),
                   "sbq_linear_w8_argmax")
    return y, idx


def linear_w8a8_argmax(x2: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, colsum: torch.Tensor,
                       bias: torch.Tensor | None, N: int, state: torch.Tensor, workspace: torch.Tensor | None = None,
                       out: torch.Tensor | None = None,
                       idx: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """int8-dyn lm_head and its greedy token in one pass (see linear_w8_argmax)."""
    x2 = _as_activation(x2)
    M, K = x2.shape
    y = out if out is not None else torch.empty((M, N), dtype=torch.float32, device=x2.device)
    if y.dtype != torch.float32:
        raise ValueError("linear_w8a8_argmax: the logits are fp32")
    ws = workspace if workspace is not None else w8a8_workspace(M, K, x2.device, N, x2.dtype)
    _check_operands("linear_w8a8_argmax", x2, packed, N, y, (("scale", scale, torch.float32),
                                                             ("bias", bias, torch.float32),
                                                             ("colsum", colsum, torch.int32)), ws)
    idx = _check_argmax("linear_w8a8_argmax", x2, state, idx)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sbq_linear_w8a8_argmax(_ptr(x2), _code(x2.dtype), M, K, _ldx(x2), _ptr(packed),
                                                      _ptr(scale), _ptr(colsum), _ptr(bias), N, _ptr(y),
                                                      _ldx(y), _ptr(idx), _ptr(ws), _nbytes(ws), _ptr(state),
                                                      _stream(x2.device)),
                   "sbq_linear_w8a8_argmax")
    return y, idx


def _greedy_state(module: nn.Module, device: torch.device) -> torch.Tensor:
    """The module's fused-argmax state for the current stream on `device`:
    calls on one stream run one after another and leave the state zero, so
    they share it; calls on another stream get their own."""
    states = module.__dict__.setdefault("_argmax_states", {})
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    st = states.get(key)
    if st is None:
        st = states[key] = argmax_state(device)
    return st


def act_qparams(x2: torch.Tensor) -> tuple[float, int]:
    """The per-tensor (scale, zero_point) the int8-dyn path uses for x2 [M, K]
    (a GPU tensor)."""
    if not x2.is_cuda or x2.dim() != 2:
        raise ValueError("act_qparams: x must be a 2-D GPU tensor")
    x2 = _as_activation(x2)
    M, K = x2.shape
    s = torch.empty((1,), dtype=torch.float32, device=x2.device)
    z = torch.empty((1,), dtype=torch.int32, device=x2.device)
    ws = w8a8_workspace(M, K, x2.device)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sbq_act_qparams(_ptr(x2), _code(x2.dtype), M, K, _ldx(x2), _ptr(s), _ptr(z),
                                               _ptr(ws), _nbytes(ws), _stream(x2.device)),
                   "sbq_act_qparams")
    return float(s.item()), int(z.item())


def act_quant_per_tensor(x2: torch.Tensor, out: torch.Tensor | None = None
                         ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The activation quantization inside linear_dynamic (quant.py:65) on its
    own: (xq uint8 [M, K], scale fp32 [1], zero_point int32 [1]) on x2's GPU,
    xq = clamp(rint(fma(x, 1/scale, zero_point)), 0, 255).  `out`: a uint8
    [M, >= K] GPU tensor with unit column stride to write xq into."""
    if not x2.is_cuda or x2.dim() != 2:
        raise ValueError("act_quant_per_tensor: x must be a 2-D GPU tensor")
    x2 = _as_activation(x2)
    M, K = x2.shape
    if out is None:
        out = torch.empty((M, K), dtype=torch.uint8, device=x2.device)
    if (out.dtype != torch.uint8 or out.dim() != 2 or out.shape[0] != M or out.shape[1] < K or out.stride(1) != 1
            or out.device != x2.device):
        raise ValueError("out must be a uint8 [M, >= K] tensor on x's device with unit column stride")
    s = torch.empty((1,), dtype=torch.float32, device=x2.device)
    z = torch.empty((1,), dtype=torch.int32, device=x2.device)
    ws = w8a8_workspace(M, K, x2.device)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sbq_act_quant_per_tensor(_ptr(x2), _code(x2.dtype), M, K, _ldx(x2), _ptr(out),
                                                        _ldx(out), _ptr(s), _ptr(z), _ptr(ws), _nbytes(ws),
                                                        _stream(x2.device)),
                   "sbq_act_quant_per_tensor")
    return out[:, :K], s, z


# ---------------------------------------------------------------------------
# reference API (spikingbrain_cpu/quant.py)
# ---------------------------------------------------------------------------
def quantize_per_channel(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """quant.py:25-29.  Runs on the GPU; results are returned on the weight's
    device (a CPU weight is uploaded, quantized, and the results copied back)."""
    q, scale = quantize_per_channel_gpu(weight.to(_gpu_for(weight)))
    if not weight.is_cuda:
        q, scale = q.cpu(), scale.cpu()
    return q, scale


def _run_on_device(x: torch.Tensor, device: torch.device, fn):
    """Run fn on x moved to `device`; return the result on x's device."""
    if x.device == device:
        return fn(x)
    if x.is_cuda:
        raise ValueError(f"sbq: input on {x.device} but the layer lives on {device}")
    return fn(x.to(device, non_blocking=False)).cpu()


class Int8Linear(nn.Module):
    """quant.py:32-53.  Buffers ``qweight`` (int8 [N,K]) and ``scale`` (fp32
    [N]) as in the reference state_dict; ``packed`` is the tiled device layout
    the kernels stream (not persisted).  ``block`` is kept for API parity: the
    GPU kernels need no block-wise dequantization."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, block: int = 128):
        super().__init__()
        device = _gpu_for(weight)
        q, scale = quantize_per_channel_gpu(weight.to(device))
        self.register_buffer("qweight", q)
        self.register_buffer("scale", scale)
        self.bias = None if bias is None else nn.Parameter(bias.to(device).float(), requires_grad=False)
        self.block = block
        packed, _ = repack(q, with_colsum=False)
        self.register_buffer("packed", packed, persistent=False)
        self.out_dtype = torch.float32
        # a loaded state_dict replaces qweight in place: rebuild the tiles from it
        self.register_load_state_dict_post_hook(lambda module, incompatible: module._repack())

    def _repack(self):
        self.packed = repack(self.qweight.contiguous(), with_colsum=False)[0]

    @classmethod
    def from_quantized(cls, qweight: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None = None,
                       block: int = 128) -> "Int8Linear":
        """An Int8Linear from an already quantized int8 [N,K] / fp32 [N] pair (the
        state_dict entries of quant.py:36-37): no re-quantization at load."""
        if qweight.dtype != torch.int8 or qweight.dim() != 2 or scale.shape != (qweight.shape[0],):
            raise ValueError("from_quantized expects int8 qweight [N, K] and scale [N]")
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        device = _gpu_for(qweight)
        self.register_buffer("qweight", qweight.to(device).contiguous())
        self.register_buffer("scale", scale.to(device=device, dtype=torch.float32).contiguous())
        self.bias = None if bias is None else nn.Parameter(bias.to(device).float(), requires_grad=False)
        self.block = block
        self.register_buffer("packed", repack(self.qweight, with_colsum=False)[0], persistent=False)
        self.out_dtype = torch.float32
        self.register_load_state_dict_post_hook(lambda module, incompatible: module._repack())
        return self

    @property
    def in_features(self) -> int:
        return self.qweight.shape[1]

    @property
    def out_features(self) -> int:
        return self.qweight.shape[0]

    def _refresh(self):
        # packed follows qweight across .to()/.cuda(); rebuild if it was lost
        if self.packed.device != self.qweight.device or self.packed.numel() == 0:
            self._repack()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self.qweight.is_cuda:
            raise RuntimeError("sbq Int8Linear: weights are on the CPU; move the module to a ROCm GPU")
        _check_in_features(x, self.in_features)
        self._refresh()
        shape = x.shape
        N = self.out_features

        def run(xd):
            x2 = xd.reshape(-1, shape[-1])
            scale = self.scale if self.scale.dtype == torch.float32 else self.scale.float()
            bias = None if self.bias is None else self.bias.float()
            return linear_w8(x2, self.packed, scale, bias, N, self.out_dtype)

        out = _run_on_device(x, self.qweight.device, run)
        return out.reshape(*shape[:-1], out.shape[-1])

    def forward_greedy(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """forward(x) and the greedy token of each row in one pass, for the
        lm_head (model.py:445-447, engine.py:30-31): (fp32 logits [..., N],
        int64 tokens [...]).  x must be on the module's GPU."""
        _check_in_features(x, self.in_features)
        self._refresh()
        if x.device != self.qweight.device:
            raise ValueError(f"sbq: input on {x.device} but the layer lives on {self.qweight.device}")
        shape = x.shape
        bias = None if self.bias is None else self.bias.float()
        y, idx = linear_w8_argmax(x.reshape(-1, shape[-1]), self.packed, self.scale.float(), bias, self.out_features,
                                  _greedy_state(self, x.device))
        return y.reshape(*shape[:-1], y.shape[-1]), idx.reshape(shape[:-1])


class _Fp32Buffers:
    """Mixin: the buffers named in ``_fp32_buffers`` keep their fp32 values
    across module dtype conversions (``.half()``, ``.to(torch.bfloat16)``);
    device moves still apply.  quant.py:61 keeps the int8-dyn scales and bias
    inside fbgemm's packed weight, which those conversions never touch."""

    _fp32_buffers: tuple = ()

    def _apply(self, fn, recurse=True):
        keep = {n: self._buffers.get(n) for n in self._fp32_buffers}
        super()._apply(fn, recurse)
        for n, old in keep.items():
            new = self._buffers.get(n)
            if old is not None and new is not None and new.dtype != old.dtype:
                self._buffers[n] = old.to(new.device)
        return self


class DynamicInt8Linear(_Fp32Buffers, nn.Module):
    """quant.py:56-66.  The reference keeps only an opaque fbgemm prepacked
    weight (``packed``) and no state_dict entries; here ``packed`` is the tiled
    device layout and ``scale``/``colsum`` are non-persistent buffers.  The
    scales and bias stay fp32 under ``.half()`` / ``.to(dtype)``, as they do
    inside the reference's packed weight.

    ``granularity="tensor"`` (default) is the reference's fbgemm semantics,
    bit for bit.  ``granularity="token"`` opts into per-token symmetric
    activation quantization (linear_w8a8_token), which has no counterpart in
    the reference and does not reproduce its outputs."""

    _fp32_buffers = ("scale", "bias")

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, granularity: str = "tensor"):
        super().__init__()
        if granularity not in ("tensor", "token"):
            raise ValueError("granularity must be 'tensor' or 'token'")
        self.granularity = granularity
        device = _gpu_for(weight)
        q, scale = quantize_per_channel_gpu(weight.to(device))
        packed, colsum = repack(q, with_colsum=True)
        self.register_buffer("packed", packed, persistent=False)
        self.register_buffer("scale", scale, persistent=False)
        self.register_buffer("colsum", colsum, persistent=False)
        self.register_buffer("bias", None if bias is None else bias.to(device).float(), persistent=False)
        self.in_features = q.shape[1]
        self.out_features = q.shape[0]
        self.out_dtype = torch.float32

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self.packed.is_cuda:
            raise RuntimeError("sbq DynamicInt8Linear: weights are on the CPU; move the module to a ROCm GPU")
        _check_in_features(x, self.in_features)
        shape = x.shape

        def run(xd):
            x2 = xd.reshape(-1, shape[-1])
            scale = self.scale.float()
            bias = None if self.bias is None else self.bias.float()
            if getattr(self, "granularity", "tensor") == "token":
                return linear_w8a8_token(x2, self.packed, scale, bias, self.out_features, self.out_dtype)
            return linear_w8a8(x2, self.packed, scale, self.colsum, bias, self.out_features, self.out_dtype)

        out = _run_on_device(x, self.packed.device, run)
        return out.reshape(*shape[:-1], out.shape[-1])

    def forward_greedy(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """forward(x) and the greedy token of each row in one pass (see
        Int8Linear.forward_greedy); per-tensor granularity only."""
        if getattr(self, "granularity", "tensor") != "tensor":
            raise ValueError("forward_greedy: per-tensor int8-dyn only")
        _check_in_features(x, self.in_features)
        if x.device != self.packed.device:
            raise ValueError(f"sbq: input on {x.device} but the layer lives on {self.packed.device}")
        shape = x.shape
        bias = None if self.bias is None else self.bias.float()
        y, idx = linear_w8a8_argmax(x.reshape(-1, shape[-1]), self.packed, self.scale.float(), self.colsum, bias,
                                    self.out_features, _greedy_state(self, x.device))
        return y.reshape(*shape[:-1], y.shape[-1]), idx.reshape(shape[:-1])


def _dyn_from_quantized(qweight: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None) -> "DynamicInt8Linear":
    if qweight.dtype != torch.int8 or qweight.dim() != 2 or scale.shape != (qweight.shape[0],):
        raise ValueError("from_quantized expects int8 qweight [N, K] and scale [N]")
    self = DynamicInt8Linear.__new__(DynamicInt8Linear)
    nn.Module.__init__(self)
    device = _gpu_for(qweight)
    packed, colsum = repack(qweight.to(device).contiguous(), with_colsum=True)
    self.register_buffer("packed", packed, persistent=False)
    self.register_buffer("scale", scale.to(device=device, dtype=torch.float32).contiguous(), persistent=False)
    self.register_buffer("colsum", colsum, persistent=False)
    self.register_buffer("bias", None if bias is None else bias.to(device).float(), persistent=False)
    self.in_features = qweight.shape[1]
    self.out_features = qweight.shape[0]
    self.out_dtype = torch.float32
    return self


DynamicInt8Linear.from_quantized = staticmethod(_dyn_from_quantized)


def save_quantized(layers: dict[str, nn.Module], path: str) -> None:
    """Write the int8 rows and fp32 scales (and biases) of Int8Linear /
    DynamicInt8Linear layers to a safetensors file (keys <name>.qweight,
    <name>.scale, <name>.bias), so a later load skips quant.py:25-29."""
    from safetensors.torch import save_file

    tensors = {}
    for name, mod in layers.items():
        if isinstance(mod, Int8Linear):
            q = mod.qweight
        elif isinstance(mod, DynamicInt8Linear):
            q = unpack(mod.packed, mod.out_features, mod.in_features)
        else:
            raise ValueError(f"save_quantized: {name} is not an int8 layer")
        tensors[name + ".qweight"] = q.contiguous().cpu()
        tensors[name + ".scale"] = mod.scale.float().contiguous().cpu()
        if mod.bias is not None:
            tensors[name + ".bias"] = mod.bias.detach().float().contiguous().cpu()
    save_file(tensors, path, metadata={"format": "sbq-int8-per-channel"})


def load_quantized(path: str, fmt: str = "int8", device: torch.device | None = None) -> dict[str, nn.Module]:
    """Layers of a save_quantized file as Int8Linear (fmt "int8") or
    DynamicInt8Linear (fmt "int8-dyn") on the GPU, without re-quantizing."""
    from safetensors.torch import load_file

    if fmt not in ("int8", "int8-dyn"):
        raise ValueError("unknown weight format " + fmt)
    t = load_file(path, device="cpu")
    out = {}
    for key in sorted(k for k in t if k.endswith(".qweight")):
        name = key[: -len(".qweight")]
        q, s, b = t[key], t[name + ".scale"], t.get(name + ".bias")
        if device is not None:
            q = q.to(device)
        out[name] = (Int8Linear.from_quantized(q, s, b) if fmt == "int8"
                     else DynamicInt8Linear.from_quantized(q, s, b))
    return out


class FP16Linear(nn.Module):
    """quant.py:69-77 (fp16 weights, fp32 activations): plain torch GPU linear,
    outside the quantized path."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None):
        super().__init__()
        device = _gpu_for(weight)
        self.register_buffer("weight", weight.to(device=device, dtype=torch.float16).contiguous())
        self.bias = None if bias is None else nn.Parameter(bias.to(device).float(), requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _run_on_device(x, self.weight.device,
                              lambda xd: F.linear(xd.float(), self.weight.float(), self.bias))


class BF16Linear(nn.Module):
    """quant.py:80-87: plain torch GPU bf16 linear, outside the quantized path."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None):
        super().__init__()
        device = _gpu_for(weight)
        self.register_buffer("weight", weight.to(device=device, dtype=torch.bfloat16).contiguous())
        self.bias = None if bias is None else nn.Parameter(bias.to(device=device, dtype=torch.bfloat16),
                                                           requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _run_on_device(x, self.weight.device,
                              lambda xd: F.linear(xd.to(torch.bfloat16), self.weight, self.bias).float())


class FloatLinear(nn.Module):
    """quant.py:90-97: plain torch GPU fp32 linear, outside the quantized path."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None):
        super().__init__()
        device = _gpu_for(weight)
        self.register_buffer("weight", weight.to(device=device, dtype=torch.float32).contiguous())
        self.bias = None if bias is None else nn.Parameter(bias.to(device).float(), requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _run_on_device(x, self.weight.device, lambda xd: F.linear(xd.float(), self.weight, self.bias))


class FusedLinear(_Fp32Buffers, nn.Module):
    """Quantized linears that read the same input, run as one launch over their
    row-concatenated weights (the q/k/v and gate/up projections of model.py
    call their modules back to back on one x: model.py:262-264, 363-365).
    quant.py:25-29 quantizes every output row on its own, so the concatenated
    qweight / scale rows are exactly the parts' rows; int8-dyn outputs are
    bit-identical to the separate layers' (one activation quantization for the
    same x, exact int32 sums), int8 outputs agree to fp32 summation order.

    forward(x) returns one tensor per part (contiguous, like the parts').
    part(i) is a drop-in module for part i: the parts of one call sequence
    share the result of one launch.  The first part called on an input
    launches; the other parts called on the same tensor object (same address,
    same version counter) take their outputs from that launch, and once every
    part has taken its output the shared result is dropped, so a part called
    again (the next step, or the same part twice) launches anew.  Inference
    tensors (torch.inference_mode, as model.py:427 runs the model) carry no
    version counter: for them an in-place edit of x between two parts' calls
    of one sequence is not detected.  Scales and bias stay fp32 under
    .half() / .to(dtype)."""

    _fp32_buffers = ("scale", "bias")

    def __init__(self, parts: list[nn.Module]):
        super().__init__()
        parts = list(parts)
        kinds = {type(p) for p in parts}
        if not parts or len(kinds) != 1 or not kinds <= {Int8Linear, DynamicInt8Linear}:
            raise ValueError("fuse_linears: the parts must all be Int8Linear or all DynamicInt8Linear")
        if len({p.in_features for p in parts}) != 1:
            raise ValueError("fuse_linears: the parts must share in_features")
        self.w8a8 = kinds == {DynamicInt8Linear}
        device = parts[0].packed.device
        self.sizes = [p.out_features for p in parts]
        self.in_features = parts[0].in_features
        self.out_features = sum(self.sizes)
        if self.w8a8:
            q = torch.cat([unpack(p.packed, p.out_features, p.in_features) for p in parts])
        else:
            q = torch.cat([p.qweight.to(device) for p in parts])
        scale = torch.cat([p.scale.to(device).float() for p in parts])
        bias = None
        if any(p.bias is not None for p in parts):
            bias = torch.cat([p.bias.to(device).float() if p.bias is not None
                              else torch.zeros(p.out_features, device=device) for p in parts])
        packed, colsum = repack(q, with_colsum=self.w8a8)
        self.register_buffer("packed", packed, persistent=False)
        self.register_buffer("scale", scale, persistent=False)
        self.register_buffer("colsum", colsum, persistent=False)
        self.register_buffer("bias", bias, persistent=False)
        self.out_dtype = torch.float32
        self._memo_ref = None
        self._memo_key = None
        self._memo_out = None
        self._memo_taken = set()

    def forward(self, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
        _check_in_features(x, self.in_features)
        shape = x.shape

        def run(xd):
            x2 = xd.reshape(-1, shape[-1])
            scale = self.scale.float()
            bias = None if self.bias is None else self.bias.float()
            if self.w8a8:
                return linear_w8a8(x2, self.packed, scale, self.colsum, bias, self.out_features, self.out_dtype)
            return linear_w8(x2, self.packed, scale, bias, self.out_features, self.out_dtype)

        y = _run_on_device(x, self.packed.device, run)
        outs = torch.split(y, self.sizes, dim=-1)
        return tuple(o.contiguous().reshape(*shape[:-1], o.shape[-1]) for o in outs)

    def _shared(self, x: torch.Tensor, i: int) -> torch.Tensor:
        """Part i's output for x from the launch of the current call
        sequence, launching when there is none for x or part i already took
        its output from it."""
        ref = self._memo_ref() if self._memo_ref is not None else None
        # inference tensors raise on ._version: their key is the address only
        key = (x.data_ptr(), -1 if x.is_inference() else x._version)
        if ref is not x or key != self._memo_key or i in self._memo_taken:
            out = self.forward(x)
            self._memo_ref, self._memo_key, self._memo_out = weakref.ref(x), key, out
            self._memo_taken = set()
        out = self._memo_out[i]
        self._memo_taken.add(i)
        if len(self._memo_taken) == len(self.sizes):  # every part has its output: the sequence is over
            self._memo_ref = self._memo_key = self._memo_out = None
            self._memo_taken = set()
        return out

    def part(self, i: int) -> nn.Module:
        return _FusedPart(self, i)


class _FusedPart(nn.Module):
    """Part i of a FusedLinear as a module with the part's own forward."""

    def __init__(self, fused: FusedLinear, i: int):
        super().__init__()
        self._fused = (fused,)  # not a registered child: the fused weights belong to the FusedLinear
        self.index = i
        self.in_features = fused.in_features
        self.out_features = fused.sizes[i]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._fused[0]._shared(x, self.index)


def fuse_linears(parts: list[nn.Module]) -> FusedLinear:
    """One launch for several Int8Linear (or DynamicInt8Linear) layers that
    read the same input; see FusedLinear."""
    return FusedLinear(parts)


def make_linear(fmt: str, weight: torch.Tensor, bias: torch.Tensor | None = None) -> nn.Module:
    """quant.py:100-111 - same dispatch and the same ValueError for unknown formats."""
    if fmt == "float32":
        return FloatLinear(weight, bias)
    if fmt == "bfloat16":
        return BF16Linear(weight, bias)
    if fmt == "float16":
        return FP16Linear(weight, bias)
    if fmt == "int8":
        return Int8Linear(weight, bias)
    if fmt == "int8-dyn":
        return DynamicInt8Linear(weight, bias)
    raise ValueError("unknown weight format " + fmt)
