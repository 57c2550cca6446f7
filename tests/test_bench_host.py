"""Host logic of bench.py's traffic accounting (no GPU): the counter CSVs of
two rocprofv3 --pmc runs -> bytes per launch, and the per-call sums that go
into a bench line's roofline.traffic."""
import csv
import json
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)
import bench  # noqa: E402


def _write_counters(d, counter, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "p_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for name, value in rows:
            w.writerow({"Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value})


@pytest.fixture
def traffic_json(tmp_path, monkeypatch):
    path = tmp_path / "traffic.json"
    monkeypatch.setattr(bench, "TRAFFIC_JSON", str(path))
    return path


def test_traffic_scales_by_the_calibration_copy(tmp_path, traffic_json):
    kib = bench.CALIB_BYTES / 1024.0
    # The copy's FETCH_SIZE reads twice its bytes (as the counter does on the
    # box), so every fetch is scaled by 1/2; WRITE_SIZE is exact.
    fetch = [("__amd_rocclr_copyBuffer(...)", 2 * kib), ("__amd_rocclr_copyBuffer(...)", 10.0),
             ("void loop_row_kernel<8, 6, 3, 6>(args)", 200.0), ("void loop_row_kernel<8, 6, 3, 6>(args)", 100.0),
             ("void loop_tail_kernel<192, 6>(args)", 40.0)]
    write = [("__amd_rocclr_copyBuffer(...)", kib), ("void loop_row_kernel<8, 6, 3, 6>(args)", 8.0),
             ("void loop_row_kernel<8, 6, 3, 6>(args)", 8.0), ("void loop_tail_kernel<192, 6>(args)", 4.0)]
    _write_counters(tmp_path / "F", "FETCH_SIZE", fetch)
    _write_counters(tmp_path / "W", "WRITE_SIZE", write)
    rec = bench.traffic("wl", str(tmp_path / "F"), str(tmp_path / "W"))
    assert rec["_calibration"]["fetch_scale"] == pytest.approx(0.5)
    assert rec["_calibration"]["write_scale"] == pytest.approx(1.0)
    row = rec["void loop_row_kernel<8, 6, 3, 6>"]
    assert row["fetch_bytes"] == round(150.0 * 1024 * 0.5)     # mean of the two dispatches, scaled
    assert row["write_bytes"] == 8 * 1024
    assert row["dispatches"] == 2
    assert "__amd_rocclr_copyBuffer" not in rec
    assert json.loads(traffic_json.read_text())["wl"] == rec


def test_traffic_for_weights_kernels_by_launches_per_call(traffic_json):
    traffic_json.write_text(json.dumps({"wl": {
        "_calibration": {"kernel": "copy", "fetch_scale": 1.0, "write_scale": 1.0},
        "void loop_row_kernel<8>": {"total_bytes": 1000, "dispatches": 40},
        "void loop_tail_kernel<192>": {"total_bytes": 300, "dispatches": 10},
        "void quant_vec_kernel<8, 4>": {"total_bytes": 7, "dispatches": 3},
    }}))
    # Four row launches and one tail launch per call; the setup kernel is not matched.
    assert bench.traffic_for("wl", ["loop_row", "loop_tail"], "loop_tail_kernel") == 4 * 1000 + 300
    # Without a once-per-call kernel each matched kernel counts once.
    assert bench.traffic_for("wl", ["loop_row", "loop_tail"]) == 1300
    assert bench.traffic_for("wl", ["absent"]) is None
    assert bench.traffic_for("other", ["loop_row"]) is None
    # A per-call kernel that was not profiled leaves the figure unknown, not wrong.
    assert bench.traffic_for("wl", ["loop_row"], "loop_tail_kernel") is None
