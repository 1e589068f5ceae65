"""CPU checks of bench.py's bookkeeping: the algorithmic byte counts behind the
roofline, the one-GPU refusal of ``--gpus N``, and the rocprofv3 CSV summaries
(kernel-trace durations and SQ instruction mix) on small hand-made CSVs."""
import csv
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_algorithmic_bytes_counts_every_array():
    # q_proj 4096 x 4096: planes 3OK/8, fp16 scales 2GO, uint8 zeros GO, x 2K, y 2O
    assert bench.algorithmic_bytes(4096, 4096) == 6291456 + 262144 + 131072 + 8192 + 8192
    assert bench.algorithmic_bytes(4096, 4096, zeros=False) == 6291456 + 262144 + 8192 + 8192
    assert bench.algorithmic_bytes(4096, 4096, perm=True) == bench.algorithmic_bytes(4096, 4096) + 8192
    # M activation rows: x and y scale with M, the payload does not
    assert (bench.algorithmic_bytes(12288, 4096, m=8) - bench.algorithmic_bytes(12288, 4096, m=1)
            == 7 * (2 * 4096 + 2 * 12288))
    # the gate/up roofline kernel's figure
    assert bench.algorithmic_bytes(12288, 4096) == 20086784


def test_more_than_one_gpu_is_refused():
    run = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         cwd=ROOT, timeout=120)
    assert run.returncode != 0
    assert "one MI355X" in run.stderr


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summarize_trace_groups_the_last_dispatches(tmp_path, capsys):
    path = tmp_path / "trace.csv"
    rows = [[1000 * i, 1000 * i + 500 + 100 * (i % 2), f"kernel_{'ab'[i % 2]}(int)", 256] for i in range(10)]
    _write(path, ["Start_Timestamp", "End_Timestamp", "Kernel_Name", "Grid_Size_X"], rows)
    bench.summarize_trace(str(path), 4)
    out = capsys.readouterr().out
    # the last four dispatches: i = 6..9, span 6000 .. 9600 ns
    assert "last 4 dispatches: span 3.6 us" in out
    assert "| `kernel_a` | 256 | 2 | 1.0 | 0.50 | 0.50 |" in out
    assert "| `kernel_b` | 256 | 2 | 1.2 | 0.60 | 0.60 |" in out


def test_summarize_sq_per_wave_figures(tmp_path, capsys):
    path = tmp_path / "sq.csv"
    counters = {"SQ_WAVES": 100, "SQ_WAVE_CYCLES": 5000, "SQ_INSTS_VALU": 20000, "SQ_INSTS_MFMA": 1800,
                "SQ_INSTS_LDS": 3000, "SQ_INSTS_VMEM": 4000, "SQ_LDS_BANK_CONFLICT": 50, "SQ_ACTIVE_INST_LDS": 200}
    rows = [["fx::hybrid_kernel<1, 8, 2, 0>(HybridArgs)", 131072, name, value] for name, value in counters.items()]
    rows.append(["other_kernel(int)", 64, "SQ_WAVES", 1])
    _write(path, ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"], rows)
    bench.summarize_sq(str(path), "hybrid_kernel")
    out = capsys.readouterr().out
    assert "| `fx::hybrid_kernel<1, 8, 2, 0>` | 131072 | 100 | 50 | 200.0 | 18.0 | 30.0 | 40.0 | 0.25 |" in out
    assert "other_kernel" not in out
