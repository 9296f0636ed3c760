"""CPU: bench.py's command-line contract without a GPU. One GPU is the only supported count
(the driver may ask for more; the line must say why it refuses), and with no GPU visible the
bench fails loudly rather than timing anything on the host."""

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_reason():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "--gpus 2 is not supported" in r.stderr and "one MI355X" in r.stderr


def test_no_gpu_visible_fails_without_a_host_fallback():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    r = _run("--steps", "1", "--warmup", "0")
    assert r.returncode == 1 and "no GPU visible" in r.stderr
    assert r.stdout.strip() == ""
