"""CPU checks of the prefill GEMM's configuration model: the coefficients in
csrc/sbq_gemm.hip are what tune/fit.py fits to the committed MI355X sweep,
the library's picks (sbq_gemm_config) are the model's argmin on every swept
shape, and those picks stay within 1% of the fastest configuration in sum."""
import ctypes
import sys
from pathlib import Path

import pytest

TUNE = Path(__file__).resolve().parents[1] / "spikingbrain-cpu_amd" / "tune"
sys.path.insert(0, str(TUNE))

import fit  # noqa: E402


@pytest.fixture(scope="module")
def lib():
    from sbq import _lib

    return _lib.load()


@pytest.mark.parametrize("fmt", ["w8", "w8a8"])
def test_table_is_the_fit_of_the_committed_sweep(fmt):
    f, rows = fit.load(TUNE / f"sweep_mi355x_{fmt}.jsonl")
    assert f == fmt and len(rows) == 255
    new = fit.cpp_rows(fmt, fit.fit(fmt, rows))
    src = fit.table_in_source(fmt)
    assert [r[:4] for r in src] == [r[:4] for r in new]  # ids, block geometry, workgroups per CU
    for s, n in zip(src, new):
        for a, b in zip(s[4] + [s[5], s[6]], n[4] + [n[5], n[6]]):
            assert abs(a - b) < 2e-3, (s, n)


@pytest.mark.parametrize("fmt", ["w8", "w8a8"])
def test_library_picks_are_the_model_argmin(lib, fmt):
    _, rows = fit.load(TUNE / f"sweep_mi355x_{fmt}.jsonl")
    coef = fit.fit(fmt, rows)
    ev = fit.evaluate(fmt, coef, rows)
    assert ev["pick_vs_best"] < 1.01, ev
    for r in rows:
        got = lib.sbq_gemm_config(r["M"], r["N"], r["K"], 1, int(fmt == "w8a8"), None)
        assert got == fit.pick(fmt, coef, r["M"], r["N"], r["K"]), r


@pytest.mark.parametrize("fmt,bar", [("w8", 1.01), ("w8a8", 1.03)])
def test_library_picks_on_held_out_checkpoint_shapes(lib, fmt, bar):
    """The real checkpoint's prefill projections (hidden 2560, FFN 9728; K = 128,
    2560, 4096, 9728; M = 137 .. 512, the reference's prompt chunk, and lm_head
    at M = 512), timed on MI355X and not used in the fit."""
    _, rows = fit.load(TUNE / f"sweep_mi355x_checkpoint_{fmt}.jsonl")
    assert len(rows) == 37
    picked = best = 0.0
    for r in rows:
        t = {int(k): v for k, v in r["t"].items()}
        picked += t[lib.sbq_gemm_config(r["M"], r["N"], r["K"], 1, int(fmt == "w8a8"), None)]
        best += min(t.values())
    assert picked / best < bar, picked / best


def test_occupancy_matches_the_kernel_lds_model():
    # two worked cases of dl_lds_bytes: 192x128 fp16 (two 28 KiB stages; the
    # 52 KiB output tile and the operand table fit in them) and 256x256 W8A8
    # with two K tiles per stage (the 256 rows x 544 bytes output tile exceeds
    # the 128 KiB of stages, and the 5136-byte operand table is appended)
    assert fit.lds_bytes(fit.W8[18], False) == 2 * (12 * 1024 + 128 * 128)
    assert fit.lds_bytes(fit.W8A8[13], True) == 256 * (256 * 2 + 32) + ((3 * 256 + 2 * 256 + 2) * 4 + 15) // 16 * 16
    assert fit.occupancy(fit.W8[18], False) == 2 and fit.occupancy(fit.W8A8[13], True) == 1
    assert fit.occupancy(fit.W8[5], False) == 1  # K split over 4 wave groups: 128 KiB of rings
