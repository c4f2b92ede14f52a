"""Host logic of bench.py that needs no GPU: the one-GPU contract and the
launch plan of the timed region."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_launch_plan_covers_every_step_and_copy():
    import bench
    for steps, copies in ((200, 8), (1000, 32), (100, 2), (20, 1), (20, 8), (7, 8), (50, 48)):
        R, s = bench.plan_launches(steps, copies)
        assert R * s == steps, (steps, copies)
        assert s >= min(copies, steps), (steps, copies)  # every launch rotates over all copies
        assert 1 <= R <= 20
    assert bench.plan_launches(200, 8) == (20, 10)
