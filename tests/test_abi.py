"""CPU checks of the C ABI: libsbq.so loads, exports every entry point that
include/sbq.h declares, and rejects bad arguments before touching a GPU."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sbq.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sbq_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from sbq import _lib

    return _lib.load()


def test_header_declares_the_expected_entry_points():
    syms = declared_symbols()
    for s in ("sbq_quantize_per_channel", "sbq_repack_w8", "sbq_linear_w8", "sbq_linear_w8a8", "sbq_act_qparams",
              "sbq_argmax_rows"):
        assert s in syms


def test_every_declared_symbol_is_exported(lib):
    from sbq import _lib

    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
    assert set(_lib.SIGNATURES) == set(declared_symbols())


def test_version_and_status_strings(lib):
    assert lib.sbq_version().decode().startswith("sbq ")
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert lib.sbq_status_string(code).decode() != "unknown status"
    assert lib.sbq_status_string(-99).decode() == "unknown status"


def test_packed_bytes(lib):
    assert lib.sbq_packed_bytes(4096, 4096) == 4096 * 4096
    assert lib.sbq_packed_bytes(4, 4096) == 16 * 4096
    assert lib.sbq_packed_bytes(151936, 4096) == 151936 * 4096
    assert lib.sbq_packed_bytes(13, 200) == 16 * 256
    assert lib.sbq_packed_bytes(0, 5) == 0
    assert lib.sbq_w8a8_workspace_bytes(1, 4096) >= 256 * 8
    assert lib.sbq_w8_workspace_bytes(2048, 4096, 1) >= 2 * 2048 * 4 + 255  # fp16: row sums and scales
    assert lib.sbq_w8_workspace_bytes(2048, 4096, 2) >= 2048 * 4096 * 2     # bf16: one staged plane
    assert lib.sbq_w8_workspace_bytes(2048, 4096, 0) >= 2048 * 4096 * 2     # fp32: one staged fp16 plane
    assert lib.sbq_w8_workspace_bytes(-1, 4096, 1) == 0
    assert lib.sbq_w8_workspace_bytes(16, 64, 7) == 0


def test_argument_validation_without_gpu(lib):
    P = ctypes.c_void_p
    dummy = P(4096)  # never dereferenced: every call below fails validation first
    # unknown activation dtype
    assert lib.sbq_linear_w8(dummy, 7, 1, 64, 64, dummy, dummy, None, 16, dummy, 0, 16, None, 0, None) == -2
    # N < 1, K < 1, ldx < K
    assert lib.sbq_linear_w8(dummy, 0, 1, 64, 64, dummy, dummy, None, 0, dummy, 0, 16, None, 0, None) == -1
    assert lib.sbq_linear_w8(dummy, 0, 1, 0, 64, dummy, dummy, None, 16, dummy, 0, 16, None, 0, None) == -1
    assert lib.sbq_linear_w8(dummy, 0, 1, 64, 32, dummy, dummy, None, 16, dummy, 0, 16, None, 0, None) == -1
    # M == 0 is a no-op
    assert lib.sbq_linear_w8(None, 0, 0, 64, 64, None, None, None, 16, None, 0, 16, None, 0, None) == 0
    # null pointers, misaligned packed weights
    assert lib.sbq_linear_w8(None, 0, 1, 64, 64, dummy, dummy, None, 16, dummy, 0, 16, None, 0, None) == -1
    assert lib.sbq_linear_w8(dummy, 0, 1, 64, 64, P(4097), dummy, None, 16, dummy, 0, 16, None, 0, None) == -3
    # W8A8 needs colsum and a workspace
    assert lib.sbq_linear_w8a8(dummy, 0, 1, 64, 64, dummy, dummy, None, None, 16, dummy, 0, 16, None, dummy,
                               4096, None) == -1
    assert lib.sbq_linear_w8a8(dummy, 0, 1, 64, 64, dummy, dummy, dummy, None, 16, dummy, 0, 16, None, None,
                               0, None) == -4
    assert lib.sbq_linear_w8a8(dummy, 0, 1, 64, 64, dummy, dummy, dummy, None, 16, dummy, 0, 16, None, dummy,
                               16, None) == -4
    assert lib.sbq_quantize_per_channel(dummy, 5, 4, 4, 4, dummy, 4, dummy, None) == -2
    assert lib.sbq_repack_w8(dummy, 4, 64, 32, dummy, None, None) == -1
    assert lib.sbq_act_qparams(dummy, 0, 1, 64, 64, dummy, dummy, None, 0, None) == -4
    # activation quantization on its own: ldq < K, null xq, bad dtype, short workspace
    wsq = lib.sbq_w8a8_workspace_bytes(2, 64)
    assert lib.sbq_act_quant_per_tensor(dummy, 0, 2, 64, 64, dummy, 63, dummy, dummy, dummy, wsq, None) == -1
    assert lib.sbq_act_quant_per_tensor(dummy, 0, 2, 64, 64, None, 64, dummy, dummy, dummy, wsq, None) == -1
    assert lib.sbq_act_quant_per_tensor(dummy, 7, 2, 64, 64, dummy, 64, dummy, dummy, dummy, wsq, None) == -2
    assert lib.sbq_act_quant_per_tensor(dummy, 0, 2, 64, 64, dummy, 64, dummy, dummy, dummy, wsq - 1, None) == -4
    # the no-allocation W8A8 entry point: colsum required; quantized activations
    # beyond its static scratch (M * ceil(K/64)*64 > SBQ_NOALLOC_XQ_BYTES) rejected
    from sbq import _lib
    assert lib.sbq_linear_w8a8_noalloc(dummy, 0, 1, 64, 64, dummy, dummy, None, None, 16, dummy, 0, 16, None,
                                       None) == -1
    m_over = _lib.SBQ_NOALLOC_XQ_BYTES // 4096 + 1
    assert lib.sbq_linear_w8a8_noalloc(dummy, 1, m_over, 4096, 4096, dummy, dummy, dummy, None, 16, dummy, 0, 16,
                                       None, None) == -4
    # argmax: N < 1, ldy < N, null pointers; M == 0 is a no-op
    assert lib.sbq_argmax_rows(dummy, 1, 0, 0, dummy, None) == -1
    assert lib.sbq_argmax_rows(dummy, 1, 8, 4, dummy, None) == -1
    assert lib.sbq_argmax_rows(None, 1, 8, 8, dummy, None) == -1
    assert lib.sbq_argmax_rows(None, 0, 8, 8, None, None) == 0
    # grouped weight-only linears: 1..SBQ_MAX_GROUP linears, each checked as
    # sbq_linear_w8 checks one; M == 0 is a no-op
    def arr(ct, vals):
        return (ct * len(vals))(*vals)

    def grouped(count, M, K, ldx, N, ldy, packed=4096, xdt=0):
        n = max(count, 1)
        return lib.sbq_linear_w8_grouped(count, arr(P, [4096] * n), arr(ctypes.c_int64, [ldx] * n), xdt, M, K,
                                         arr(P, [packed] * n), arr(P, [4096] * n), None, arr(ctypes.c_int64, [N] * n),
                                         arr(P, [4096] * n), arr(ctypes.c_int64, [ldy] * n), 0, None)

    assert grouped(0, 1, 64, 64, 16, 16) == -1
    assert grouped(_lib.SBQ_MAX_GROUP + 1, 1, 64, 64, 16, 16) == -1
    assert grouped(2, 1, 64, 32, 16, 16) == -1        # ldx < K
    assert grouped(2, 1, 64, 64, 16, 8) == -1         # ldy < N
    assert grouped(2, 1, 64, 64, 16, 16, xdt=7) == -2
    assert grouped(2, 1, 64, 64, 16, 16, packed=4097) == -3
    assert grouped(2, 0, 64, 64, 16, 16) == 0

    # grouped int8-dyn linears: checked as sbq_linear_w8a8 checks one, and
    # the column sums and the workspace are required
    def grouped8(count, M, K, ldx, N, ldy, colsum=4096, ws=4096, ws_bytes=1 << 20):
        n = max(count, 1)
        return lib.sbq_linear_w8a8_grouped(count, arr(P, [4096] * n), arr(ctypes.c_int64, [ldx] * n), 0, M, K,
                                           arr(P, [4096] * n), arr(P, [4096] * n), arr(P, [colsum] * n), None,
                                           arr(ctypes.c_int64, [N] * n), arr(P, [4096] * n),
                                           arr(ctypes.c_int64, [ldy] * n), 0, ws, ws_bytes, None)

    assert grouped8(0, 1, 64, 64, 16, 16) == -1
    assert grouped8(_lib.SBQ_MAX_GROUP + 1, 1, 64, 64, 16, 16) == -1
    assert grouped8(2, 1, 64, 32, 16, 16) == -1       # ldx < K
    assert grouped8(2, 1, 64, 64, 16, 16, colsum=None) == -1
    assert grouped8(2, 1, 64, 64, 16, 16, ws=None) == -4
    assert grouped8(2, 1, 64, 64, 16, 16, ws_bytes=16) == -4
    assert grouped8(2, 0, 64, 64, 16, 16) == 0
    # row / column counts beyond 2^31 - 1 are rejected before any launch
    big = 1 << 31
    assert lib.sbq_linear_w8(dummy, 0, big, 64, 64, dummy, dummy, None, 16, dummy, 0, 16, None, 0, None) == -1
    assert lib.sbq_quantize_per_channel(dummy, 0, big, 4, 4, dummy, 4, dummy, None) == -1
    assert lib.sbq_repack_w8(dummy, big, 64, 64, dummy, None, None) == -1
    assert lib.sbq_unpack_w8(dummy, 16, big, dummy, big, None) == -1
    assert lib.sbq_w8a8_workspace_bytes(big, 64) == 0


def test_python_binding_maps_status_to_exceptions():
    from sbq import _lib

    _lib.check(0, "ok")
    with pytest.raises(ValueError, match="unsupported dtype"):
        _lib.check(-2, "x")
    with pytest.raises(_lib.SbqError, match="launch failed"):
        _lib.check(-5, "x")


# Prefill GEMM configuration choices (host-only, no GPU): M > 128 runs the
# fitted kernel-time model, M <= 128 the grid rules with K split over
# workgroups for small grids.  One shape per configuration the picker uses;
# the GPU tests run these same shapes against the oracle.
PICKS_W8 = [(264, 19648, 4096, 0), (648, 10816, 4096, 2), (136, 16384, 4096, 3), (136, 5504, 4096, 5),
            (136, 256, 4096, 8), (136, 21824, 4096, 16), (136, 10944, 4096, 17), (392, 20992, 4096, 18),
            (2048, 12288, 4096, 0), (512, 12288, 4096, 16), (8192, 12288, 4096, 0)]
PICKS_W8A8 = [(520, 21824, 4096, 0), (648, 16384, 4096, 2), (328, 16384, 4096, 3), (136, 256, 4096, 8),
              (1536, 8192, 12288, 12), (520, 19648, 4096, 13), (264, 19648, 4096, 14), (136, 5504, 4096, 15),
              (264, 21824, 4096, 16), (392, 20992, 4096, 18), (648, 22336, 4096, 19), (136, 21824, 4096, 20),
              (2048, 12288, 4096, 18), (512, 12288, 4096, 20)]


@pytest.mark.parametrize("w8a8,cases", [(0, PICKS_W8), (1, PICKS_W8A8)])
def test_gemm_config_picks(lib, w8a8, cases):
    splits = ctypes.c_int(-1)
    for M, N, K, cfg in cases:
        for dt in (0, 1, 2):  # every activation dtype reaches the GEMM as fp16 / s8
            assert lib.sbq_gemm_config(M, N, K, dt, w8a8, ctypes.byref(splits)) == cfg, (M, N, K, dt)
            assert splits.value == 1


# Mid-sized M (M <= 128): 64 x 64 blocks (configuration 22), K split over
# min(4, budget / blocks) workgroups (budget 288 for W8A8, 768 for fp16
# weight-only), each split keeping >= 4 stage steps; (M, N, K, w8a8, splits).
MID_PLANS = [(128, 4096, 4096, 1, 2), (128, 4096, 4096, 0, 4), (64, 4096, 4096, 1, 4), (100, 2048, 4096, 1, 4),
             (128, 12288, 4096, 1, 1), (128, 12288, 4096, 0, 2), (128, 2560, 9728, 1, 3), (128, 9728, 2560, 1, 1),
             (128, 4096, 1024, 1, 2), (120, 1024, 2560, 1, 4), (128, 4096, 4160, 1, 2), (80, 2560, 9728, 0, 4)]


def test_gemm_config_split_plans_and_errors(lib):
    splits = ctypes.c_int(-1)
    for M, N, K, w8a8, S in MID_PLANS:
        assert lib.sbq_gemm_config(M, N, K, 1, w8a8, ctypes.byref(splits)) == 22, (M, N, K, w8a8)
        assert splits.value == S, (M, N, K, w8a8, splits.value)
    # grids of more than 512 blocks of 64 x 64 keep the picker's configuration
    assert lib.sbq_gemm_config(128, 24576, 4096, 1, 1, ctypes.byref(splits)) != 22 and splits.value == 1
    assert lib.sbq_gemm_config(128, 4096, 4096, 1, 1, None) == 22  # splits may be NULL
    assert lib.sbq_gemm_config(0, 4096, 4096, 1, 0, None) == -1
    assert lib.sbq_gemm_config(128, 0, 4096, 1, 0, None) == -1
    assert lib.sbq_gemm_config(128, 4096, 4096, 1, 2, None) == -1
    assert lib.sbq_gemm_config(128, 4096, 4096, 7, 0, None) == -2


# Shapes that do not reach the tiled GEMM report 0 splits (and add no split
# area to the workspace): decode sizes (the decode GEMVs) and 16 < M <= 64 on
# narrow layers (the row-tile GEMV); (M, N, K, x dtype, w8a8).
NOT_GEMM = [(1, 4096, 4096, 1, 1), (8, 4096, 4096, 0, 0), (16, 4096, 4096, 1, 0), (32, 4096, 4096, 1, 1),
            (24, 4096, 4096, 1, 0), (48, 2048, 4096, 2, 0), (33, 1000, 2048, 1, 1)]
GEMM = [(48, 12288, 4096, 1, 1), (64, 4096, 4096, 1, 1), (64, 4096, 4096, 1, 0), (32, 9728, 2560, 1, 1),
        (40, 4096, 8192, 1, 0), (40, 4096, 8192, 1, 1)]


def test_gemm_config_reports_the_route(lib):
    splits = ctypes.c_int(-1)
    for M, N, K, dt, w8a8 in NOT_GEMM:
        lib.sbq_gemm_config(M, N, K, dt, w8a8, ctypes.byref(splits))
        assert splits.value == 0, (M, N, K, dt, w8a8)
        base = lib.sbq_w8a8_workspace_bytes(M, K) if w8a8 else lib.sbq_w8_workspace_bytes(M, K, dt)
        assert lib.sbq_linear_workspace_bytes(M, N, K, dt, w8a8) == base, (M, N, K, dt, w8a8)
    for M, N, K, dt, w8a8 in GEMM:
        lib.sbq_gemm_config(M, N, K, dt, w8a8, ctypes.byref(splits))
        assert splits.value >= 1, (M, N, K, dt, w8a8)


def test_sample_rows_validation_without_gpu(lib):
    """sbq_sample_rows (engine.py:29-42) rejects bad arguments before any
    launch; its workspace size grows with the rows only."""
    P = ctypes.c_void_p
    dummy = P(4096)
    per_row = lib.sbq_sample_workspace_bytes(1, 151936) - lib.sbq_sample_workspace_bytes(0, 151936)
    assert per_row > 0
    assert lib.sbq_sample_workspace_bytes(3, 151936) == lib.sbq_sample_workspace_bytes(0, 151936) + 3 * per_row
    assert lib.sbq_sample_workspace_bytes(3, 10) == lib.sbq_sample_workspace_bytes(3, 151936)
    assert lib.sbq_sample_workspace_bytes(-1, 10) == 0 and lib.sbq_sample_workspace_bytes(1, 0) == 0
    # at most 65535 rows and 2^23 tokens (a row's 2^-40 fixed-point mass fits 64 bits)
    assert lib.sbq_sample_workspace_bytes(1, 1 << 23) > 0 and lib.sbq_sample_workspace_bytes(1, (1 << 23) + 1) == 0
    assert lib.sbq_sample_workspace_bytes(65536, 10) == 0
    ws_ok = lib.sbq_sample_workspace_bytes(1, 1000)
    nan = float("nan")
    # M < 0, V < 1, ld < V, too many rows
    assert lib.sbq_sample_rows(dummy, -1, 1000, 1000, 0.7, 0, 0.9, dummy, dummy, dummy, ws_ok, None) == -1
    assert lib.sbq_sample_rows(dummy, 1, 0, 1000, 0.7, 0, 0.9, dummy, dummy, dummy, ws_ok, None) == -1
    assert lib.sbq_sample_rows(dummy, 1, 1000, 999, 0.7, 0, 0.9, dummy, dummy, dummy, ws_ok, None) == -1
    assert lib.sbq_sample_rows(dummy, 70000, 1000, 1000, 0.7, 0, 0.9, dummy, dummy, dummy, ws_ok, None) == -1
    big = (1 << 23) + 1
    assert lib.sbq_sample_rows(dummy, 1, big, big, 0.7, 0, 0.9, dummy, dummy, dummy, ws_ok, None) == -1
    # NaN temperature or top_p
    assert lib.sbq_sample_rows(dummy, 1, 1000, 1000, nan, 0, 0.9, dummy, dummy, dummy, ws_ok, None) == -1
    assert lib.sbq_sample_rows(dummy, 1, 1000, 1000, 0.7, 0, nan, dummy, dummy, dummy, ws_ok, None) == -1
    # no rows: nothing to do
    assert lib.sbq_sample_rows(None, 0, 1000, 1000, 0.7, 0, 0.9, None, None, None, 0, None) == 0
    # null logits or tokens; a draw without uniforms; a short workspace
    assert lib.sbq_sample_rows(None, 1, 1000, 1000, 0.7, 0, 0.9, dummy, dummy, dummy, ws_ok, None) == -1
    assert lib.sbq_sample_rows(dummy, 1, 1000, 1000, 0.7, 0, 0.9, dummy, None, dummy, ws_ok, None) == -1
    assert lib.sbq_sample_rows(dummy, 1, 1000, 1000, 0.7, 0, 0.9, None, dummy, dummy, ws_ok, None) == -1
    assert lib.sbq_sample_rows(dummy, 1, 1000, 1000, 0.7, 0, 0.9, dummy, dummy, dummy, ws_ok - 1, None) == -4
    assert lib.sbq_sample_rows(dummy, 1, 1000, 1000, 0.7, 0, 0.9, dummy, dummy, None, ws_ok, None) == -4


def test_sample_tokens_rejects_host_logits():
    import torch
    from sbq import quant

    with pytest.raises(ValueError):
        quant.sample_tokens(torch.zeros(1, 10), 0.7, 0.9)
    with pytest.raises(ValueError):
        quant.sample_tokens(torch.zeros(1, 10, dtype=torch.float16), 0.7, 0.9)


def test_general_gemv_configurations_are_launchable(lib):
    """Every configuration the general GEMV picks (M = 1..32, K = 1..12288,
    both formats, every activation dtype) has a kernel instance and satisfies
    the launch invariants its kernel relies on: at most 16 waves; the waves'
    K ranges cover every K tile; one epilogue thread per output pair
    (waves >= row tiles x weight tiles; too few once left rows 16..M-1
    unwritten); LDS-staged activations fully staged by the threads' chunks;
    LDS within the 160 KiB of a CU."""
    info = (ctypes.c_int32 * 9)()
    Ks = sorted(set(list(range(1, 300)) + list(range(300, 12289, 37)) + [64 * i for i in range(1, 193)]))
    checked = 0
    for w8a8 in (0, 1):
        for dt in (0, 1, 2):
            xb = 4 if dt == 0 else 2
            for M in range(1, 33):
                for K in Ks:
                    assert lib.sbq_gemv_config(M, K, dt, w8a8, info) == 0
                    ok, mt, g, p, waves, xm, sc, lds, inst = list(info)
                    if not ok:
                        continue
                    Kc = (K + 63) // 64
                    where = (M, K, dt, w8a8, list(info))
                    assert inst == 1, where
                    assert 1 <= waves <= 16, where
                    assert p * waves >= Kc, where
                    assert waves >= mt * g, where
                    assert mt == (1 if M <= 16 else 2), where
                    if xm == 1:  # staged in LDS: sc 16-byte chunks per thread cover x[M][Kc*64]
                        assert sc * 64 * waves * 16 >= M * Kc * 64 * xb, where
                    assert lds <= 160 * 1024, where
                    checked += 1
    assert checked > 50000
    assert lib.sbq_gemv_config(0, 64, 1, 0, info) == -1
    assert lib.sbq_gemv_config(1, 64, 9, 0, info) == -2
    assert lib.sbq_gemv_config(1, 64, 1, 0, None) == -1


@pytest.mark.parametrize("lang,std", [("c", "c99"), ("c++", "c++17")])
def test_header_compiles_standalone(tmp_path, lang, std):
    """include/sbq.h is a plain C interface: it compiles on its own as C99 and
    as C++ with every warning an error (what a cgo / FFI binding includes)."""
    import shutil
    import subprocess

    cc = shutil.which("gcc" if lang == "c" else "g++")
    if cc is None:
        pytest.skip("no host compiler")
    src = tmp_path / ("use.c" if lang == "c" else "use.cpp")
    src.write_text('#include "sbq.h"\nint sbq_use(void) { return SBQ_OK + SBQ_F16 + SBQ_MAX_GROUP; }\n')
    r = subprocess.run([cc, f"-std={std}", "-Wall", "-Wextra", "-pedantic", "-Werror", "-fsyntax-only",
                        f"-I{HEADER.parent}", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
