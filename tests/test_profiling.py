"""Host logic of flyai_amd.profiling on synthetic rocprofv3 CSV files (no GPU)."""
import csv
import os

from flyai_amd import profiling


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def _counter_dir(tmp, name, counter, kernel_vals, copy_vals):
    d = os.path.join(tmp, name)
    os.makedirs(d)
    rows, disp = [], 0
    for v in kernel_vals:
        disp += 1
        # two instance rows per dispatch: the summary must add them
        rows += [[disp, "void flyai::moe_mxfp4_kernel<true, 2>(int)", counter, v / 2],
                 [disp, "void flyai::moe_mxfp4_kernel<true, 2>(int)", counter, v / 2]]
    for v in copy_vals:
        disp += 1
        rows.append([disp, "__amd_rocclr_copyBuffer", counter, v])
    _write(os.path.join(d, "c1_counter_collection.csv"),
           ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"], rows)
    return d


def test_traffic_scales_by_copy_reading(tmp_path):
    fetch = _counter_dir(str(tmp_path), "f", "FETCH_SIZE", [999.0, 400.0, 400.0], [128.0, 128.0, 128.0])
    write = _counter_dir(str(tmp_path), "w", "WRITE_SIZE", [50.0, 10.0, 10.0], [256.0] * 3)
    r = profiling.traffic(fetch, write, "moe_mxfp4_kernel<true", reps=2, copy_mib=0.25)
    # copy of 256 KiB reads as 128 KiB -> factor 2; the last two kernel dispatches read 400 KiB each
    assert abs(r["read"]["factor"] - 2.0) < 1e-12
    assert r["read"]["bytes"] == 800.0 * 1024
    assert r["write"]["factor"] == 1.0 and r["write"]["bytes"] == 10.0 * 1024
    assert r["hbm_bytes_per_launch"] == 810 * 1024


def test_short_name_keeps_template_drops_params():
    assert profiling.short_name("void flyai::moe_mxfp4_kernel<true, 2>(unsigned short const*, int)") == \
        "moe_mxfp4_kernel<true, 2>"
    n = profiling.short_name("void at::native::(anonymous namespace)::k<float, (a)1>(int)")
    assert n == "at::native::k<float, (a)1>"


def test_kernel_table_and_last_dispatches(tmp_path):
    d = str(tmp_path)
    _write(os.path.join(d, "c1_kernel_stats.csv"),
           ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"],
           [["a(int)", 2, 3000, 1500, 75, 1000, 2000, 1], ["b(int)", 1, 1000, 1000, 25, 1000, 1000, 0]])
    _write(os.path.join(d, "c1_kernel_trace.csv"),
           ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"],
           [[1, "a(int)", 0, 1000], [2, "b(int)", 1000, 2000], [3, "a(int)", 2000, 4000]])
    lines, total = profiling.kernel_table(d)
    assert total == 4000 and lines[2].startswith("| `a` | 2 | 1.50")
    assert profiling.last_dispatches(d, "a", 1) == [(3, 2000)]


def test_counter_table_groups_by_kernel_and_grid(tmp_path):
    d = str(tmp_path)
    trace = os.path.join(d, "trace")
    os.makedirs(trace)
    _write(os.path.join(trace, "c1_kernel_trace.csv"),
           ["Dispatch_Id", "Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp",
            "End_Timestamp"],
           [[1, "attn(int)", 64, 1, 1, 0, 2000], [2, "attn(int)", 128, 1, 1, 0, 4000],
            [3, "attn(int)", 64, 1, 1, 0, 4000]])
    pmc = os.path.join(d, "pmc")
    os.makedirs(pmc)
    hdr = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    rows = [[1, "attn(int)", 64, "FETCH_SIZE", 50.0], [1, "attn(int)", 64, "FETCH_SIZE", 50.0],
            [1, "attn(int)", 64, "TA_TA_BUSY_sum", 1000.0], [1, "attn(int)", 64, "GRBM_GUI_ACTIVE", 10.0],
            [1, "attn(int)", 64, "GRBM_GUI_ACTIVE", 5.0],
            [2, "attn(int)", 128, "FETCH_SIZE", 300.0], [2, "attn(int)", 128, "SQ_INSTS_VALU_MFMA_MOPS_BF16", 2.0],
            [3, "__amd_rocclr_copyBuffer", 4096, "FETCH_SIZE", 512.0]]
    _write(os.path.join(pmc, "c1_counter_collection.csv"), hdr, rows)
    ents = profiling.counter_table([pmc], trace, ["attn"], copy_mib=1, n_cu=200)
    by = {e["grid"]: e for e in ents}
    # a 1 MiB copy reads as 512 KiB -> 2 bytes per counter byte; instance rows of a dispatch add up
    assert by[64]["FETCH_SIZE_bytes"] == 100.0 * 2 * 1024
    assert by[64]["calls"] == 2 and by[64]["avg_us"] == 3.0
    # busy cycles over n_cu x the dispatch's GRBM_GUI_ACTIVE (max over its instances)
    assert by[64]["TA_TA_BUSY_sum_frac"] == 1000.0 / (200 * 10.0)
    assert by[128]["mfma_TFLOPs"] == 2.0 * 512 / 4e-6 / 1e12
    md = profiling.counter_markdown(ents, "t", ["cmd"])
    assert md[0] == "# t" and any(line.startswith("| `attn` | 64 |") for line in md)
