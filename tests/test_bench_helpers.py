"""CPU checks of bench.py's own arithmetic and its one-GPU contract.

- flowshop_bound (the config-5 bound) is max over k of (copies 0..k) +
  (computes k..end).  It is checked against an event-by-event simulation of
  the two-machine flow shop it stands for: copy j runs after copy j-1 on the
  link; compute j starts when compute j-1 has ended and copy j has landed.
  Random instances are used, plus the cases that reduce to one machine.
- _copy_stats: the link's busy time is the union of the copies' intervals,
  and copies in flight on average is the sum of durations over that union.
  Both are checked on hand-made logs.
- bench.py --gpus 2 exits with status 2 and says that this build runs on one
  GPU, before touching the GPU.
- line_kernel_check (the stats summary's comparison of the line's event time
  with rocprof's) takes the dominant kernel's last steps x launches_per_step
  dispatches of the trace, and no other kernel's; checked on a hand-made
  line and trace.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def simulate_flowshop(copy_ms, compute_ms):
    copy_end = compute_end = 0.0
    for c, w in zip(copy_ms, compute_ms):
        copy_end += c
        compute_end = max(compute_end, copy_end) + w
    return compute_end


def test_flowshop_bound_matches_simulation():
    rng = np.random.default_rng(7)
    for _ in range(500):
        n = int(rng.integers(1, 40))
        copies = rng.uniform(0.0, 2.0, n).tolist()
        computes = rng.uniform(0.0, 2.0, n).tolist()
        assert bench.flowshop_bound(copies, computes) == pytest.approx(simulate_flowshop(copies, computes),
                                                                       rel=1e-12, abs=1e-12)


def test_flowshop_bound_single_machine_cases():
    comp = [0.5, 1.5, 0.25]
    assert bench.flowshop_bound([0.0, 0.0, 0.0], comp) == pytest.approx(sum(comp))
    assert bench.flowshop_bound([1.0, 2.0, 3.0], [0.0, 0.0, 0.0]) == pytest.approx(6.0)
    # the config-5 shape in miniature: copy-bound first half, compute-bound second
    copies = [1.0] * 4 + [1.0] * 4
    computes = [0.5] * 4 + [2.0] * 4
    assert bench.flowshop_bound(copies, computes) == pytest.approx(4.0 + 1.0 + 8.0)
    assert bench.flowshop_bound(copies, computes) > max(sum(copies), sum(computes))


def test_copy_stats_busy_union_and_rates():
    # two overlapping copies, then a gap, then one copy
    log = [(0.0, 2.0), (1.0, 3.0), (5.0, 6.0)]
    s = bench._copy_stats(log, 1_000_000)
    assert s["busy_ms"] == pytest.approx(4.0)  # [0, 3] and [5, 6]
    assert s["span_ms"] == pytest.approx(6.0)
    assert s["sum_copy_ms"] == pytest.approx(5.0)
    assert s["copies_in_flight_avg"] == pytest.approx(5.0 / 4.0, abs=1e-3)
    assert s["busy_gbs"] == pytest.approx(3 * 1e6 / 4e-3 / 1e9, rel=1e-3)
    assert s["median_copy_ms"] == pytest.approx(2.0)
    # order of the log does not matter, and a single copy is its own union
    assert bench._copy_stats(list(reversed(log)), 1_000_000)["busy_ms"] == pytest.approx(4.0)
    one = bench._copy_stats([(1.0, 1.5)], 500_000)
    assert one["busy_ms"] == pytest.approx(0.5) and one["copies_in_flight_avg"] == pytest.approx(1.0)
    assert bench._copy_stats([], 1) is None


def test_more_than_one_gpu_exits():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_line_kernel_check_uses_the_last_dispatches(tmp_path):
    import json
    grouped = "void dfk::" + bench.TRAFFIC_FAMILIES["gemm_bwd"][0] + "(unsigned char const*, int)"
    line = {"steps": 2, "kernels": {"gemm_bwd": {"launches_per_step": 3}},
            "roofline": {"kernel": "gemm_bwd", "avg_launch_ms": 0.3, "work_per_launch": 6e11, "peak": 5000.0}}
    (tmp_path / "prof_bench_line.json").write_text("rocprofv3 noise\n" + json.dumps(line) + "\n")
    (tmp_path / "prof_bench").mkdir()
    rows = ["Kernel_Name,Start_Timestamp,End_Timestamp"]
    t = 1_000_000
    for i in range(10):  # 4 early dispatches of 0.5 ms, then the pass's 6 of 0.303 ms
        dur = 500_000 if i < 4 else 303_000
        rows.append(f'"{grouped}",{t},{t + dur}')
        rows.append(f'"void dfk::other_kernel<int>(int)",{t + dur},{t + dur + 900_000}')
        t += 2_000_000
    (tmp_path / "prof_bench" / "bench_kernel_trace.csv").write_text("\n".join(rows) + "\n")
    out = "\n".join(bench.line_kernel_check(str(tmp_path)))
    assert "| rocprof, same 6 dispatches | 0.3030 |" in out
    assert "| HIP events (the line) | 0.3000 |" in out
    assert "They differ by 1.0%." in out
    assert bench.line_kernel_check(str(tmp_path / "missing")) == []
