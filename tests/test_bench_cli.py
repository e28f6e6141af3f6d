"""bench.py's contract checks that run without a GPU: more than one GPU is refused with a message and exit code 2,
before anything touches a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=60, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_bench_refuses_a_multi_rank_launch():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True, timeout=60,
                       cwd=ROOT, env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_hbm_rows_get_their_read_probe():
    """Each HBM-bound line is set against the read probe of its own byte size; MFMA lines are left alone."""
    import bench
    configs = {"c2": [dict(M=1, bound="hbm", bytes=100, GBps=3000.0), dict(M=64, bound="hbm", bytes=200, GBps=10.0)],
               "c3": [dict(M=2048, bound="mfma", bytes=100, TOPS=1.0)], "deferred": {"x": 1}}
    assert sorted(bench.hbm_sizes(configs)) == [100, 200]
    bench.annotate_hbm_rows(configs, {100: (2.0, 5000.0), 200: (4.0, 50.0)})
    assert configs["c2"][0]["frac_of_measured"] == 0.6 and configs["c2"][0]["read_probe_us"] == 2.0
    assert configs["c2"][1]["frac_of_measured"] == 0.2
    assert "frac_of_measured" not in configs["c3"][0]
