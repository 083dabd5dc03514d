"""Host-side checks of bench.py's contract (no GPU): the one-GPU refusal and
the committed traffic summary it reads its ``roofline.traffic`` from."""

import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_newton_traffic_summary_parses():
    sys.path.insert(0, REPO)
    import bench

    traffic = bench._traffic_from_profile("slstm_newton_cfg3.md")
    assert traffic is not None
    # bytes per launch over B*T*d = 2^27 elements: at least the compulsory
    # 24 B/element (read wx and the guess, write the result), at most the
    # algorithmic K*40 = 80 B/element the roofline counts
    per_element = traffic / (bench.B * bench.T * bench.D)
    assert 24.0 <= per_element <= 80.0, per_element
    assert bench._traffic_from_profile("no_such_profile.md") is None
