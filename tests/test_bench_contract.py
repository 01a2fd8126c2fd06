"""bench.py's contract with the driver, checked without a GPU: one GPU only
(any other count exits with a message), argument checks before any device
work, and the algorithmic byte counts the JSON line divides by, each against
its closed form."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, env={**os.environ, "WORLD_SIZE": "1"})


@pytest.mark.parametrize("n", ["2", "8", "0"])
def test_only_one_gpu(n):
    r = _run("--gpus", n)
    assert r.returncode == 2 and "one GPU" in r.stderr
    assert r.stdout == "", "no JSON line for a refused run"


def test_argument_checks_before_device_work():
    r = _run("--steps", "0")
    assert r.returncode == 2 and "--steps >= 1" in r.stderr


def test_headline_bytes():
    # 11008 rows of 128 Q4_0 blocks (18 bytes each), x and y in fp16
    assert bench.ALGO_BYTES_CFG0 == 11008 * (4096 // 32) * 18 + 2 * 4096 + 2 * 11008 == 25_392_640


def test_decode_sweep_bytes():
    # 32 layers of q, k, v, o (4096 x 4096), gate, up (11008 x 4096) and down
    # (4096 x 11008), each packed weights + x + y, then lm_head 32000 x 4096
    def gemv(m, k):
        return m * (k // 32) * 18 + 2 * k + 2 * m

    layer = 4 * gemv(4096, 4096) + 2 * gemv(11008, 4096) + gemv(4096, 11008)
    assert bench.sweep_bytes() == 32 * layer + gemv(32000, 4096) == 3_721_550_336


def test_moe_gather_bytes():
    # 10 experts; gate and up [1024 x 4096], down [4096 x 1024]; 4-bit codes,
    # one fp16 scale and bias per 64 weights
    per_matrix = 1024 * 4096 // 2 + 2 * 2 * (1024 * 4096 // 64)
    assert bench.MOE_GATE_UP_BYTES == 10 * 2 * per_matrix + 2 * 4096
    assert bench.MOE_DOWN_BYTES == 10 * per_matrix + 2 * 10 * 1024
    # with y instead of h, the gather's algorithmic bytes (70,795,264)
    assert bench.MOE_GATE_UP_BYTES + bench.MOE_DOWN_BYTES - 2 * 10 * 1024 + 2 * 4096 == 70_795_264


def test_traffic_comes_from_the_committed_profile():
    t = bench.measured_traffic()
    assert t is not None and 1.0 <= t / bench.ALGO_BYTES_CFG0 < 1.05
