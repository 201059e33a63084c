"""Fit the prefill GEMM's configuration model (PickCost in csrc/sbq_gemm.hip)
to the timings sweep.py measured, and report how well it picks.

Model of configuration c at shape (M, N, K), Kc = ceil(K / 64): the grid of
G = ceil(Nt / wt) * ceil(M / bm) workgroups puts B = ceil(G / 256) on the
busiest CU, which runs them in rounds of up to occ at once; a round of j
workgroups costs round[j-1] us per K tile, so

    t = (B // occ) * round[occ-1] * Kc + (round[B % occ - 1] * Kc if B % occ) + kc * Kc + c0

fitted by least squares on relative error, one configuration at a time.

    python fit.py sweep_mi355x_w8.jsonl            # coefficients as C++ rows, fit quality
    python fit.py sweep_mi355x_w8a8.jsonl --check  # compare with the table in csrc/sbq_gemm.hip
"""
from __future__ import annotations

import argparse
import json
import re
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
GEMM_SRC = HERE.parent / "csrc" / "sbq_gemm.hip"

# Direct-to-LDS configurations the picker chooses from, by id: (BN, BM, WN, WM,
# NS, KG, KT), as SBQ_DL_CONFIGS and launch_dl_i8 / launch_dl_rsp build them.
W8 = {0: (256, 128, 4, 2, 2, 1, 1), 2: (128, 128, 2, 2, 2, 1, 1), 3: (128, 64, 2, 2, 2, 1, 1),
      5: (128, 64, 2, 2, 2, 4, 1), 8: (64, 64, 1, 2, 2, 4, 1), 10: (256, 128, 4, 1, 2, 1, 1),
      16: (192, 64, 4, 1, 2, 1, 1), 17: (192, 64, 4, 1, 2, 4, 1), 18: (192, 128, 4, 1, 2, 1, 1)}
W8A8 = {0: (256, 128, 4, 2, 2, 1, 1), 1: (256, 128, 4, 2, 3, 1, 1), 2: (128, 128, 2, 2, 2, 1, 1),
        3: (128, 64, 2, 2, 2, 1, 1), 8: (64, 64, 1, 2, 2, 4, 1), 12: (256, 256, 4, 2, 2, 1, 1),
        13: (256, 256, 4, 2, 2, 1, 2), 14: (128, 128, 2, 2, 2, 1, 2), 15: (128, 64, 2, 2, 2, 1, 2),
        16: (192, 64, 4, 1, 2, 1, 1), 18: (192, 128, 4, 1, 2, 1, 1), 19: (192, 128, 4, 1, 3, 1, 1),
        20: (192, 64, 4, 1, 2, 1, 2)}
CONFIGS = {"w8": W8, "w8a8": W8A8}
CUS = 256
LDS_PER_CU = 160 * 1024


def lds_bytes(cfg, i8):
    """dl_lds_bytes of csrc/sbq_gemm.hip for fp16 W-only with precomputed row
    sums (RSP) or W8A8."""
    BN, BM, WN, WM, NS, KG, KT = cfg
    stage = KT * ((BN // 16) * 1024 + BM * (64 if i8 else 128))
    red = (KG - 1) * WN * WM * (BN // WN // 16) * (BM // WM // 16) * 1024
    ldsb = max(KG * NS * stage, red)
    epi = BM * (BN * 2 + 32) if KG == 1 else 0
    ldsa = max(epi, ldsb)
    post = epi if KG == 1 else red
    epb = ((3 * BN + 2 * BM + 2) * 4 + 15) & ~15
    return ldsa + (0 if post + epb <= ldsa else epb)


def occupancy(cfg, i8):
    """Workgroups per CU: what the LDS admits, and the register budget of the
    kernel's launch bounds (4 waves per SIMD, 2 for wave tiles over 64x64)."""
    BN, BM, WN, WM, NS, KG, KT = cfg
    regs = 2 if (BN // WN) * (BM // WM) > 64 * 64 else 4
    waves = KG * WN * WM
    return max(1, min(LDS_PER_CU // lds_bytes(cfg, i8), 4 * regs // waves))


def features(cfg, occ, M, N, K):
    BN, BM = cfg[0], cfg[1]
    nt, kc = (N + 15) // 16, (K + 63) // 64
    G = -(-nt // (BN // 16)) * -(-M // BM)
    B = -(-G // CUS)
    f = [0.0] * (occ + 2)
    full, rem = divmod(B, occ)
    f[occ - 1] += full * kc
    if rem:
        f[rem - 1] += kc
    f[occ] = kc
    f[occ + 1] = 1.0
    return f


def load(path):
    rows = [json.loads(line) for line in open(path) if line.strip()]
    fmt = rows[0]["f"]
    return fmt, rows


def fit(fmt, rows):
    i8 = fmt == "w8a8"
    coef = {}
    for c, cfg in CONFIGS[fmt].items():
        occ = occupancy(cfg, i8)
        pts = [(r["M"], r["N"], r["K"], r["t"][str(c)]) for r in rows if str(c) in r["t"]]
        X = np.array([features(cfg, occ, M, N, K) for M, N, K, _ in pts])
        y = np.array([t for *_, t in pts])
        w = 1.0 / y
        coef[c] = np.linalg.lstsq(X * w[:, None], y * w, rcond=None)[0]
    return coef


def predict(fmt, coef, c, M, N, K):
    cfg = CONFIGS[fmt][c]
    return float(np.dot(coef[c], features(cfg, occupancy(cfg, fmt == "w8a8"), M, N, K)))


def pick(fmt, coef, M, N, K):
    """The picker's choice: the smallest predicted time (first in id order on a tie)."""
    best = None
    for c in sorted(CONFIGS[fmt]):
        t = predict(fmt, coef, c, M, N, K)
        if best is None or t < best[0]:
            best = (t, c)
    return best[1]


def evaluate(fmt, coef, rows):
    errs, tp, tb, bad = [], 0.0, 0.0, []
    for r in rows:
        t = {int(k): v for k, v in r["t"].items()}
        errs += [abs(predict(fmt, coef, c, r["M"], r["N"], r["K"]) - v) / v for c, v in t.items()]
        pk, best = pick(fmt, coef, r["M"], r["N"], r["K"]), min(t.values())
        tp += t[pk]
        tb += best
        if t[pk] > 1.08 * best:
            bad.append((round(t[pk] / best, 2), r["M"], r["N"], r["K"], pk))
    return {"median_err": float(np.median(errs)), "pick_vs_best": tp / tb, "over_8pct": sorted(bad, reverse=True)}


def cpp_rows(fmt, coef):
    i8 = fmt == "w8a8"
    out = []
    for c in sorted(CONFIGS[fmt]):
        cfg = CONFIGS[fmt][c]
        occ = occupancy(cfg, i8)
        rnd = list(coef[c][:occ]) + [0.0] * (4 - occ)
        out.append((c, cfg[0] // 16, cfg[1], occ, [round(v, 4) for v in rnd], round(coef[c][occ], 4),
                    round(coef[c][occ + 1], 3)))
    return out


def table_in_source(fmt):
    """The PickCost rows of csrc/sbq_gemm.hip for this format."""
    text = GEMM_SRC.read_text()
    name = "kPickI8" if fmt == "w8a8" else "kPickF16"
    body = text[text.index(f"constexpr PickCost {name}[] = {{"):]
    body = body[:body.index("};")]
    rows = []
    for m in re.finditer(r"\{(\d+), (\d+), (\d+), (\d+), \{([^}]*)\}, ([-0-9.]+)f, ([-0-9.]+)f\}", body):
        rnd = [float(v.strip().rstrip("f")) for v in m.group(5).split(",")]
        rows.append((int(m.group(1)), int(m.group(2)), int(m.group(3)), int(m.group(4)), rnd, float(m.group(6)),
                     float(m.group(7))))
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("sweep", help="JSON lines from sweep.py")
    ap.add_argument("--check", action="store_true", help="compare the fit with the table in csrc/sbq_gemm.hip")
    args = ap.parse_args()
    fmt, rows = load(args.sweep)
    coef = fit(fmt, rows)
    ev = evaluate(fmt, coef, rows)
    half = fit(fmt, rows[0::2])
    ev_half = evaluate(fmt, half, rows[1::2])
    print(f"{fmt}: {len(rows)} shapes; median error {ev['median_err']:.3f}; picks {ev['pick_vs_best']:.4f}x the "
          f"fastest configuration in sum; {len(ev['over_8pct'])} shapes over 1.08x {ev['over_8pct'][:4]}; "
          f"fitted on half, the other half {ev_half['pick_vs_best']:.4f}x")
    new = cpp_rows(fmt, coef)
    for c, wt, bm, occ, rnd, kc, c0 in new:
        print(f"    {{{c}, {wt}, {bm}, {occ}, {{{', '.join(f'{v:.4f}f' for v in rnd)}}}, {kc:.4f}f, {c0:.3f}f}},")
    if args.check:
        src = table_in_source(fmt)
        assert [r[:4] for r in src] == [r[:4] for r in new], "configuration ids / geometry / occupancy differ"
        worst = max(max(abs(a - b) for a, b in zip(s[4] + [s[5], s[6]], n[4] + [n[5], n[6]])) for s, n in zip(src, new))
        print(f"largest coefficient difference from csrc/sbq_gemm.hip: {worst:.4f}")
        return 0 if worst < 2e-3 else 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
