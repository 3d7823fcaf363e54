"""rocprof_summary.py (no GPU): kernel names grouped as the library's timer
groups them, per-kernel trace statistics, and HBM bytes per forward scaled
by the copy calibration -- on small synthetic rocprofv3 CSV files."""
import csv
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import rocprof_summary as rs  # noqa: E402


def write_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    return str(path)


def test_block_kernel_names():
    assert rs.block_kernel("void tie::mfma_experts_kernel<12, false, 32>(tie::MfmaArgs)") == "mfma_gate_up"
    assert rs.block_kernel("tie::mfma_experts_kernel<14, true, 0>(tie::MfmaArgs)") == "mfma_down"
    assert rs.block_kernel("tie::route_bucket_kernel<1>(tie::BucketArgs)") == "router"
    assert rs.block_kernel("tie::decode_one_kernel<12, 12, 14, true>(tie::OneArgs)") == "decode_one"
    assert rs.block_kernel("tie::combine_fix_kernel<12, 12, 14>(...)") == "combine"
    assert rs.block_kernel("at::native::copy_kernel(...)") is None
    # a prefix of another name is not a match
    assert rs.block_kernel("tie::router_topk_kernelX(...)") is None


def test_stats_groups_by_kernel_and_grid(tmp_path):
    rows = [
        {"Kernel_Name": "void tie::combine_kernel(float*)", "Grid_Size_X": "512", "Grid_Size_Y": "1",
         "Grid_Size_Z": "1", "Workgroup_Size_X": "256", "Start_Timestamp": "1000", "End_Timestamp": "5000"},
        {"Kernel_Name": "void tie::combine_kernel(float*)", "Grid_Size_X": "512", "Grid_Size_Y": "1",
         "Grid_Size_Z": "1", "Workgroup_Size_X": "256", "Start_Timestamp": "9000", "End_Timestamp": "11000"},
        {"Kernel_Name": "void tie::combine_kernel(float*)", "Grid_Size_X": "1024", "Grid_Size_Y": "1",
         "Grid_Size_Z": "1", "Workgroup_Size_X": "256", "Start_Timestamp": "20000", "End_Timestamp": "26000"},
        {"Kernel_Name": "at::elementwise(...)", "Grid_Size_X": "1", "Grid_Size_Y": "1", "Grid_Size_Z": "1",
         "Workgroup_Size_X": "64", "Start_Timestamp": "0", "End_Timestamp": "1"},
    ]
    st = rs.stats(write_csv(tmp_path / "t.csv", rows))
    assert list(st.values()) == [[4000, 2000], [6000]]
    md = rs.stats_markdown(str(tmp_path / "t.csv"), "T", "cmd")
    # avg, median (upper middle of an even count), min in us
    assert "| tie::combine_kernel | 512,1,1 | 256 | 2 | 3.00 | 4.00 | 2.00 |" in md


def counter_rows(kernel, counter, values):
    return [{"Kernel_Name": kernel, "Counter_Name": counter, "Counter_Value": str(v)} for v in values]


def test_traffic_scales_by_the_copy_and_counts_forwards(tmp_path):
    copy = "void at::native::copy_kernel(...)"
    # the copy of 1 MiB reads 512 KiB and writes 1024 KiB by the counters:
    # FETCH_SIZE x 2, WRITE_SIZE x 1 (the largest copy dispatch counts)
    cf = write_csv(tmp_path / "cf.csv", counter_rows(copy, "FETCH_SIZE", [3, 512]))
    cw = write_csv(tmp_path / "cw.csv", counter_rows(copy, "WRITE_SIZE", [5, 1024]))
    gu = "tie::mfma_experts_kernel<12, false, 32>(...)"
    cb = "tie::combine_fix_kernel<12, 12, 14>(...)"
    fetch = write_csv(tmp_path / "f.csv", counter_rows(gu, "FETCH_SIZE", [100, 100]) +
                      counter_rows(cb, "FETCH_SIZE", [10, 10]))
    write = write_csv(tmp_path / "w.csv", counter_rows(gu, "WRITE_SIZE", [1, 1]) +
                      counter_rows(cb, "WRITE_SIZE", [4, 4]))
    res, scales = rs.traffic(fetch, write, cf, cw, 1 << 20)
    assert scales["fetch_scale"] == pytest.approx(2.0)
    assert scales["write_scale"] == pytest.approx(1.0)
    # two forwards (two combine dispatches): per forward 100 KiB x 2 fetched, 1 KiB written
    assert res["mfma_gate_up"]["fetch_bytes"] == 200 * 1024
    assert res["mfma_gate_up"]["write_bytes"] == 1024
    assert res["mfma_gate_up"]["bytes"] == 201 * 1024
    assert res["combine"]["forwards"] == 2


def test_traffic_needs_a_forward_marker(tmp_path):
    copy = "copy_kernel"
    cf = write_csv(tmp_path / "cf.csv", counter_rows(copy, "FETCH_SIZE", [1]))
    cw = write_csv(tmp_path / "cw.csv", counter_rows(copy, "WRITE_SIZE", [1]))
    f = write_csv(tmp_path / "f.csv", counter_rows("tie::router_logits_kernel(...)", "FETCH_SIZE", [1]))
    w = write_csv(tmp_path / "w.csv", counter_rows("tie::router_logits_kernel(...)", "WRITE_SIZE", [1]))
    with pytest.raises(ValueError):
        rs.traffic(f, w, cf, cw, 1024)
