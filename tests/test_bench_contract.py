"""bench.py's host-side contract, checked without a GPU: one GPU only (a
request for more exits with a message), the workload table, the FLOP
convention and the PMC ingest's calibration scaling."""

from __future__ import annotations

import csv
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert p.returncode == 2
    assert "one GPU" in p.stderr
    assert p.stdout.strip() == ""


def test_flop_convention_of_the_headline_workload():
    """12 * B * H * Lq * Lk * D per fwd+bwd step (src/avgen/simulate/compute.py
    :126,142): 8.78e13 at c3."""
    cfg = bench.CONFIGS["c3"]
    flops, dense = bench.flops_per_step(cfg, {"mask": None})
    assert flops == dense == 12.0 * 1 * 40 * 18900 * 75600 * 128
    assert abs(flops - 8.78e13) / 8.78e13 < 1e-3
    assert bench.kernel_flops_per_step(cfg, {"mask": None}, "bwd_dkdv") == 3 * 2.0 * 40 * 18900 * 75600 * 128


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5", "varlen", "window", "qknorm"])
def test_every_workload_names_itself(name):
    cfg = bench.CONFIGS[name]
    assert cfg["desc"] and cfg["D"] in (64, 128)


def test_pmc_ingest_scales_by_the_calibration_kernel(tmp_path, monkeypatch):
    """Counters are scaled by what they read for the 1 GiB calibration copy;
    the workload's own small neg kernels are not mistaken for it."""
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    (tmp_path / "profiles").mkdir()
    cal_kib = bench.CALIBRATION_BYTES / 1024.0

    def write(path, counter, kern_kib, cal_raw_kib):
        with open(path, "w", newline="") as fh:
            w = csv.DictWriter(fh, fieldnames=["Counter_Name", "Kernel_Name", "Counter_Value"])
            w.writeheader()
            w.writerow({"Counter_Name": counter, "Kernel_Name": "void avattn::qk_norm_fwd_kernel<128>(x)",
                        "Counter_Value": kern_kib})
            w.writerow({"Counter_Name": counter, "Kernel_Name": "at::native::neg_kernel small", "Counter_Value": 3.0})
            w.writerow({"Counter_Name": counter, "Kernel_Name": "at::native::neg_kernel", "Counter_Value": cal_raw_kib})

    write(tmp_path / "f.csv", "FETCH_SIZE", 1000.0, cal_kib / 2)  # fetch reads half: scale 2
    write(tmp_path / "w.csv", "WRITE_SIZE", 500.0, cal_kib)       # write exact: scale 1
    r = bench.ingest_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), "qk_norm", "qknorm")
    assert r["fetch_bytes_per_launch"] == pytest.approx(2000.0 * 1024)
    assert r["write_bytes_per_launch"] == pytest.approx(500.0 * 1024)
    stored = json.loads((tmp_path / "profiles" / "traffic_qk_norm_qknorm.json").read_text())
    assert stored["bytes_per_launch"] == pytest.approx(2500.0 * 1024)
