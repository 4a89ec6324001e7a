"""bench.py's command line on the CPU: the flags the benchmark contract names, and the refusal of a multi-GPU
run (each GPU runs the single-GPU call on its own share; the benchmark measures one)."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_help_lists_the_contract_flags():
    r = _run("--help")
    assert r.returncode == 0, r.stderr
    for flag in ("--gpus", "--steps", "--warmup", "--tune", "--profile"):
        assert flag in r.stdout


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "--gpus 1" in r.stderr
    assert r.stdout.strip() == ""  # no JSON line for a run that did not happen
