"""CPU bounds check of the GEMV kernels' load windows (no GPU needed).

Compiles tests/block_window_check.cpp against the kernels' own address
helpers (google-classic_amd/csrc/block_window.h) and checks every (row, unit)
window for the GPU test shapes, the benchmark shapes and a sweep of small
ragged shapes, including rows that start on a 2-byte boundary (odd block
count per row).
"""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "google-classic_amd" / "csrc"
Q4_0, Q8_0, Q4_K = 0, 1, 2  # holo::Fmt


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("bw") / "block_window_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", f"-I{CSRC}", str(ROOT / "tests" / "block_window_check.cpp"),
                    "-o", str(exe)], check=True)
    return exe


def _run(checker, shapes):
    args = [str(a) for s in shapes for a in s]
    r = subprocess.run([str(checker), *args], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr


def test_gpu_test_shapes(checker):
    from test_gpu_gemv import CASES
    fmt = {2: Q4_0, 8: Q8_0, 12: Q4_K}
    _run(checker, [(fmt[t], o, i) for t, o, i in CASES])


def test_bench_shapes(checker):
    shapes = [(Q4_0, 4096, 4096), (Q4_0, 11008, 4096), (Q4_0, 4096, 11008), (Q8_0, 4096, 4096),
              (Q8_0, 32000, 4096), (Q4_K, 14336, 4096), (Q4_K, 4096, 14336)]
    _run(checker, shapes)


def test_small_ragged_sweep(checker):
    shapes = []
    for f, qk in ((Q4_0, 32), (Q8_0, 32), (Q4_K, 256)):
        for rows in range(1, 10):
            for nb in range(1, 21):
                shapes.append((f, rows, qk * nb))
    _run(checker, shapes)
