"""Host-side checks of kernel index arithmetic (no GPU).

tests/host/bounds_check.cpp includes the index functions the kernels use
(spikingbrain-cpu_amd/csrc/sbq_index.h) and is compiled with g++:
  * bounds: every work item of a launch is walked through an index map and
    each range is checked against its buffer; a planted out-of-bounds form
    (the map without its clamp) must be caught;
  * the fused greedy token (the lm_head GEMV's argmax epilogue) ranks values by
    argmax_key: the largest key must be torch.argmax's pick (engine.py:30-31:
    first index of the maximum, NaN above every number, -0 equal to +0) on
    crafted rows; a planted key order with -0 below +0 must disagree."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "host" / "bounds_check.cpp"
INC = ROOT / "spikingbrain-cpu_amd" / "csrc"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("bounds") / "bounds_check"
    subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-I", str(INC), str(SRC), "-o", str(exe)], check=True)
    return exe


def run(checker, *args):
    return subprocess.run([str(checker), *map(str, args)], capture_output=True, text=True)


@pytest.mark.parametrize("M,K,ldx", [(1, 16, 16), (3, 1312, 1312), (512, 1312, 1312), (7, 4096, 4096),
                                     (5, 48, 48), (2, 80, 96), (33, 9728, 9728), (1, 12288, 12288)])
def test_act_quantizer_chunks_stay_in_rows(checker, M, K, ldx):
    r = run(checker, "act", M, K, ldx)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout


def test_act_quantizer_unclamped_form_is_caught(checker):
    # K % 64 == 32: the last padding chunk of the last row would read past x
    r = run(checker, "act-unclamped", 4, 1312, 1312)
    assert r.returncode == 1 and "violation" in r.stdout


def pick(checker, values, mode="argmax"):
    text = "\n".join(repr(float(v)) for v in values) + "\n"
    r = subprocess.run([str(checker), mode], input=text, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return int(r.stdout)


ROWS = [
    [1.0, 3.0, 3.0, 2.0],                              # tie: first index
    [float("-inf"), float("-inf")],                    # all -inf
    [-1.0, float("nan"), 5.0, float("nan")],           # NaN above numbers, first NaN
    [float("inf"), 1e38, float("inf")],                # +inf tie
    [-0.0, 0.0, -0.0],                                 # zeros are equal
    [-3.0, -0.0, -1e-45],                              # -0 above negatives, denormal
    [-5.0, -2.5, -2.5, -7.0],                          # negative tie
    [1e-45, 0.0, 2e-45],                               # denormals order
    [float("nan")],
    [0.0],
]


@pytest.mark.parametrize("row", ROWS)
def test_argmax_key_order_is_torch_argmax(checker, row):
    import torch

    assert pick(checker, row) == int(torch.argmax(torch.tensor(row, dtype=torch.float32)))


def test_argmax_key_order_random_rows(checker):
    import numpy as np
    import torch

    rng = np.random.default_rng(5)
    for i in range(30):
        v = rng.standard_normal(257).astype(np.float32)
        v[rng.integers(0, 257, 3)] = v.max()           # ties at the maximum
        if i % 3 == 0:
            v[rng.integers(0, 257, 2)] = np.nan
        if i % 5 == 0:
            v = -np.abs(v)
            v[rng.integers(0, 257, 4)] = -0.0
        assert pick(checker, v) == int(torch.argmax(torch.from_numpy(v))), i


def test_argmax_key_planted_zero_order_disagrees(checker):
    import torch

    row = [-0.0, 0.0]
    assert pick(checker, row, "argmax-unfolded-zero") != int(torch.argmax(torch.tensor(row)))


def test_argmax_slot_counts(checker):
    """The fused argmax counts workgroups per slot (blockIdx % 64) and the
    slots in use; brute-force counting must agree for every grid size up to
    5000 (the 151936-row lm_head launches 4748 workgroups)."""
    r = run(checker, "argmax-slots")
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout
