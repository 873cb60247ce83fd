"""bench.py's command-line contract, checked without a GPU: more than one GPU
is refused with a message before any device work (one GPU per box), and the
usage text names the modes the driver and the profiles use."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2")
    assert r.returncode != 0
    assert "one GPU" in r.stderr and "--gpus 2" in r.stderr, r.stderr
    assert r.stdout == ""  # no JSON line


def test_usage_lists_the_modes():
    r = run_bench("--help")
    assert r.returncode == 0
    for opt in ("--gpus", "--steps", "--warmup", "--batch2", "--kernels", "--copy-probe", "--reps",
                "--no-cpu", "--no-configs"):
        assert opt in r.stdout, opt
