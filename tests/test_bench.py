"""bench.py's measurement logic on the host: the union of launch intervals that the roofline of a
chained step divides by, and the rocprofv3 kernel-trace summary that must agree with it."""
from __future__ import annotations

import csv

import bench


def test_union_of_intervals():
    assert bench._union_us([]) == 0.0
    assert bench._union_us([(0.0, 1.0)]) == 1.0
    assert bench._union_us([(0.0, 1.0), (2.0, 3.0)]) == 2.0            # disjoint: the sum
    assert bench._union_us([(0.0, 2.0), (1.0, 3.0)]) == 3.0            # overlapping
    assert bench._union_us([(1.0, 3.0), (0.0, 2.0), (0.5, 0.7)]) == 3.0   # unsorted, nested
    assert bench._union_us([(0.0, 5.0), (1.0, 2.0), (3.0, 4.0)]) == 5.0   # contained


def _trace(path, rows):
    cols = ['Kind', 'Agent_Id', 'Queue_Id', 'Stream_Id', 'Thread_Id', 'Dispatch_Id', 'Kernel_Id', 'Kernel_Name',
            'Correlation_Id', 'Start_Timestamp', 'End_Timestamp']
    with open(path, 'w', newline='') as f:
        w = csv.writer(f)
        w.writerow(cols)
        for i, (stream, name, a, b) in enumerate(rows):
            w.writerow(['KERNEL_DISPATCH', 'Agent 1', 1, stream, 1, i, 0, name, i, int(a * 1000), int(b * 1000)])


def test_trace_summary_takes_the_union_over_the_last_steps(tmp_path):
    """Two chains on two streams, three steps of one prologue and two overlapping Newton-Schulz
    launches each: the summary counts the last two steps only, and their union (not the sum)."""
    rows = []
    for s in range(3):
        t = 1000.0 * s
        for st, off in ((1, 0.0), (2, 10.0)):
            rows.append((st, 'thorn::ortho_pre_kernel(x)', t + off, t + off + 5))
            rows.append((st, 'thorn::ns_phase_kernel(x)', t + off + 20, t + off + 120))
            rows.append((st, 'thorn::ns_phase_kernel(x)', t + off + 130, t + off + 230))
    path = tmp_path / 'run_kernel_trace.csv'
    _trace(path, rows)
    out = '\n'.join(bench.ns_trace_lines(str(path), steps=2))
    # per step: stream 1 covers 20-120 and 130-230, stream 2 30-130 and 140-240: union 220 us
    assert '(2 stream(s)): 4 launches per step' in out
    assert 'summed durations 100.0 us per launch' in out
    assert 'union of their intervals 0.220 ms per step, 55.0 us per launch' in out
    assert 'launch | ops' not in out          # no per-launch table with two streams
