"""bench.py's command-line contract that holds without a GPU: more than one
GPU is refused with a message (this build measures one MI355X), and the
flags the driver passes parse."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2",
                        "--steps", "3", "--warmup", "1"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "--gpus 2 is not supported" in r.stderr and "single MI355X" in r.stderr
    assert r.stdout.strip() == ""


def test_flags_parse():
    sys.path.insert(0, ROOT)
    import bench
    old = sys.argv
    try:
        sys.argv = ["bench.py", "--gpus", "1", "--steps", "7", "--warmup", "2", "--configs",
                    "--no-cpu"]
        a = bench.parse()
    finally:
        sys.argv = old
    assert (a.gpus, a.steps, a.warmup, a.configs, a.no_cpu) == (1, 7, 2, True, True)
