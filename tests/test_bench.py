"""bench.py's pieces that need no GPU: the one-GPU refusal, the traffic
figure it reads from the committed rocprofv3 summary, and the reference
sweep's matrices and trace summary."""
import json
import os
import subprocess
import sys

import numpy as np

import bench
from sparsewavecomp_amd import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"),
                        "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_traffic_comes_from_the_headline_profile():
    t = bench.traffic_from_profile(bench.HEADLINE_SPMV)
    alg = W.algorithmic_bytes_spmv(1 << 20, 1 << 20, 33_597_418)
    # the summary was taken for the headline mapping: its HBM bytes per
    # launch exceed the algorithmic bytes (x is re-fetched by every XCD)
    assert isinstance(t, int) and t > alg
    assert bench.traffic_from_profile(
        "spmv-mapping=thread-per-row spmv-block-size=256") is None


def test_reference_sweep_matrices_match_the_reference_report():
    """The reference's sweep table (docs/benchmarks/spmv-mapping-sweep-
    gfx1101.md:97-102) lists mean and maximum NNZ per row of its synthetic
    65,536-row matrices: the restated generator gives the same shapes, its
    columns are position mod columns and its values 1."""
    want_max = {("uniform", 4): 4, ("uniform", 32): 32, ("uniform", 256): 256,
                ("skewed", 4): 25, ("skewed", 32): 249, ("skewed", 256): 2041}
    for (dist, per_row), mx in want_max.items():
        m = W.reference_sweep_matrix(dist, per_row)
        lengths = np.diff(m.row_offsets)
        assert m.rows == m.cols == 65536
        assert lengths.max() == mx and lengths.mean() == per_row
        assert m.nnz == 65536 * per_row
        assert np.array_equal(m.column_indices,
                              np.arange(m.nnz) % 65536)
        assert np.all(m.values == 1.0)
    alt = np.diff(W.reference_sweep_matrix("alternating", 4).row_offsets)
    assert list(alt[:4]) == [1, 7, 1, 7]


def test_reference_sweep_summary_from_a_kernel_trace(tmp_path, capsys):
    """The summarizer splits a kernel trace at the gather-floor marks, adds
    the kernels of each call, and takes medians of the measured calls."""
    steps = bench.REFERENCE_SWEEP_WARMUP + bench.REFERENCE_SWEEP_MEASURED
    t = [0]

    def row(name, us):
        t[0] += 1000
        r = {"Kernel_Name": name, "Start_Timestamp": str(t[0]),
             "End_Timestamp": str(t[0] + int(us * 1000))}
        t[0] += int(us * 1000)
        return r
    rows = []
    for ci, case in enumerate(bench.REFERENCE_SWEEP_CASES):
        rows.append(row("void spmv_gather_floor(int const*)", 1.0))
        for s in range(steps):
            if case.startswith("rocsparse"):
                rows += [row("void csrmvn_general_kernel", 30.0),
                         row("void csrmvn_tail", 2.0)]
            elif "wave-per-position" in case:
                rows += [row("void fill_zero_f32(float*, long)", 1.0),
                         row("void spmv_wave_position<4, true>", 9.0)]
            else:  # case ci takes 20 + ci us, with slow warm-up calls
                rows.append(row("void spmv_kernel",
                                (20.0 + ci) * (3 if s < 10 else 1)))
    rows.append(row("void spmv_gather_floor(int const*)", 1.0))
    d = tmp_path / "uniform-32" / "host" / "run"
    d.mkdir(parents=True)
    with open(d / "kt_kernel_trace.csv", "w", newline="") as f:
        import csv
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp",
                                          "End_Timestamp"])
        w.writeheader()
        w.writerows(reversed(rows))  # the summarizer orders by start time
    bench.summarize_reference_sweep(str(tmp_path))
    out = capsys.readouterr().out
    line = [l for l in out.splitlines() if l.startswith("| uniform | 32 |")]
    assert len(line) == 2  # the mapping table and the position table
    cells = [c.strip() for c in line[0].split("|")]
    # rocSPARSE 32 us per call; the best case is a wave-per-position case at
    # 1 + 9 us; 3.20x
    assert cells[3] == "32.00" and "wave-per-position" in cells[4]
    assert cells[5] == "10.00" and cells[6] == "3.20x"
    # thread-per-position at block 64 is case 24 of the list: 44 us
    pcells = [c.strip() for c in line[1].split("|")]
    assert pcells[4].endswith("10.00, 3.20x")
    assert pcells[5] == "block-size=64, 44.00, 0.73x"
    assert pcells[6] == "35.98"
    assert "thread-per-row spmv-block-size=64 20.00" in out.replace(
        ", spmv-", " spmv-")
