"""bench.py's host-side pieces without a GPU: the kernel-trace summary cuts a rocprofv3 trace at
the marker kernels that bracket the timed steps (and only there), and refuses traces without
marker pairs or with a timed region that is not a whole number of steps."""
import csv
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
import bench  # noqa: E402

FIELDS = ["Kind", "Agent_Id", "Queue_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]


def _trace(path, events):
    """events: (name, start_ns, end_ns); written in a shuffled order (the summary sorts by start)."""
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for name, t0, t1 in reversed(events):
            w.writerow({"Kind": "KERNEL_DISPATCH", "Agent_Id": "Agent 1", "Queue_Id": 1, "Kernel_Name": name,
                        "Start_Timestamp": t0, "End_Timestamp": t1})


def _run(tmp_path, steps, region=-1, period=None, untimed_after=True):
    ev, t = [], 0

    def k(name, dur):
        nonlocal t
        ev.append((name, t, t + dur))
        t += dur + 500

    k("warm_a", 9000)                         # warmup / eager launches: never counted
    for _r in range(2):                       # two timed regions, 3 steps of (a 4 us, b 6 us)
        k(bench.MARK_KERNEL, 100)
        for _ in range(steps):
            k("kern_a", 4000)
            k("kern_b", 6000)
        k(bench.MARK_KERNEL, 100)
        if untimed_after:
            k("naive_leg", 50000)
    p = tmp_path / "t_kernel_trace.csv"
    _trace(p, ev)
    return bench.trace_summary(str(p), steps, region, period)


def test_summary_counts_only_the_timed_region(tmp_path):
    s = _run(tmp_path, steps=3)
    assert "6 dispatches = 3 steps x 2" in s
    assert "**kernel time per step 10.00 µs**" in s
    assert "naive_leg" not in s and "warm_a" not in s and bench.MARK_KERNEL not in s.split("\n", 1)[1]
    assert "| `kern_b` | 3 | 6.000 |" in s and "| `kern_a` | 3 | 4.000 |" in s


def test_summary_region_and_positions(tmp_path):
    s = _run(tmp_path, steps=3, region=0, period=2)
    assert s.startswith("timed region 0 of 2")
    assert "| 0 | `kern_a` | 4.000 |" in s and "| 1 | `kern_b` | 6.000 |" in s


def test_summary_refuses_wrong_steps_and_missing_markers(tmp_path):
    with pytest.raises(SystemExit):
        _run(tmp_path, steps=3, period=None) and bench.trace_summary(str(tmp_path / "t_kernel_trace.csv"), 4)
    p = tmp_path / "none.csv"
    _trace(p, [("kern_a", 0, 10)])
    with pytest.raises(SystemExit):
        bench.trace_summary(str(p), 1)
