"""Host-side bounds checks of kernel index maps (no GPU).

tests/host/bounds_check.cpp includes the index functions the kernels use
(spikingbrain-cpu_amd/csrc/sbq_index.h), walks every work item of a launch
through them with g++ and checks each range against its buffer.  A planted
out-of-bounds form (the map without its clamp) must be caught."""
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
