"""CPU test of bench.py's rocprof summary (calibrated HBM traffic per launch)."""
import csv
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _pmc(d: Path, sub: str, counter: str, rows):
    """One counter row per dispatch, dispatch ids in list order."""
    (d / sub).mkdir(parents=True)
    with open(d / sub / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for i, (k, v) in enumerate(rows):
            w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": k, "Counter_Name": counter, "Counter_Value": v})


def test_summary_scales_counters_by_the_copy(tmp_path):
    k = f"void w4::{bench.ROOFLINE_KERNEL}(w4::DecGroupedArgs)"
    # the 32 MiB copy (the run's first device copy) reads as 16384 KiB (factor
    # 2) and writes 32768 KiB (factor 1); a later, larger copy is not the
    # calibration
    _pmc(tmp_path, "fetch", "FETCH_SIZE", [("__amd_rocclr_copyBuffer", 16384.0), (k, 100.0), (k, 300.0),
                                           ("__amd_rocclr_copyBuffer", 524288.0)])
    _pmc(tmp_path, "write", "WRITE_SIZE", [("__amd_rocclr_copyBuffer", 32768.0), (k, 10.0),
                                           ("__amd_rocclr_copyBuffer", 1048576.0)])
    (tmp_path / "trace").mkdir()
    with open(tmp_path / "trace" / "run_kernel_stats.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "AverageNs", "MinNs", "MaxNs"])
        w.writeheader()
        w.writerow({"Name": k, "Calls": 4, "AverageNs": 10000.0, "MinNs": 9000, "MaxNs": 11000})
    text = bench.summarize_prof(tmp_path)
    line = [ln for ln in text.splitlines() if ln.startswith("- traffic_bytes_per_launch:")][0]
    # mean FETCH 200 KiB x 2 + WRITE 10 KiB x 1 = 410 KiB
    assert int(line.split(":")[1]) == 410 * 1024
    assert "average 10.000 us" in text
