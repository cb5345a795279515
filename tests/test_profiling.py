"""tcc_amd.profiling: rocprofv3 csv reductions behind the profiles/ files
(synthetic csv files; no GPU)."""
import csv
import json

from tcc_amd import profiling


def test_kernel_key_strips_arguments_and_namespaces():
    k = profiling.kernel_key("void tcc::(anonymous namespace)::gather_kernel<4, (tcc::(anonymous namespace)::Src)2, "
                             "true>(tcc::(anonymous namespace)::GatherArgs)")
    assert k == "gather_kernel<4, (Src)2, true>"
    assert profiling.kernel_key("tcc::(anonymous namespace)::hub_reduce_kernel(tcc::(anonymous namespace)::TileArgs, "
                                "unsigned int)") == "hub_reduce_kernel"
    assert profiling.kernel_key("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"
    assert profiling.kernel_key("tcc::(anonymous namespace)::calibration_copy_kernel(unsigned int __vector(4)*, "
                                "unsigned long)") == "calibration_copy_kernel"


def _counters(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (name, counter, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value})


def _stats(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"])
        w.writeheader()
        for name, calls, avg_ns in rows:
            w.writerow({"Name": name, "Calls": calls, "TotalDurationNs": calls * avg_ns, "AverageNs": avg_ns,
                        "Percentage": 0})


def test_traffic_scales_by_the_copy_and_divides_by_launches(tmp_path):
    g = "void tcc::(anonymous namespace)::gather_kernel<4>(tcc::(anonymous namespace)::GatherArgs)"
    h = "void tcc::(anonymous namespace)::hub_tiles_kernel<4, 2>(tcc::(anonymous namespace)::TileArgs)"
    other = "tcc::(anonymous namespace)::degree_kernel(unsigned int const*)"
    copy = "tcc::(anonymous namespace)::calibration_copy_kernel(unsigned int __vector(4)*, unsigned int const __vector(4)*, unsigned long)"
    # the 1 GiB copy reads FETCH_SIZE 512 Ki (factor 2) and WRITE_SIZE 1 Gi KiB... (factor 1)
    _counters(tmp_path / "f.csv", [(copy, "FETCH_SIZE", 524288), (g, "FETCH_SIZE", 100), (g, "FETCH_SIZE", 300),
                                   (h, "FETCH_SIZE", 50), (h, "FETCH_SIZE", 50), (other, "FETCH_SIZE", 1e9)])
    _counters(tmp_path / "w.csv", [(copy, "WRITE_SIZE", 1048576), (g, "WRITE_SIZE", 10), (g, "WRITE_SIZE", 10),
                                   (h, "WRITE_SIZE", 4), (h, "WRITE_SIZE", 4), (other, "WRITE_SIZE", 1e9)])
    _counters(tmp_path / "hm.csv", [(g, "TCC_HIT_sum", 3), (g, "TCC_MISS_sum", 1)])
    _stats(tmp_path / "s.csv", [(g, 2, 2_000_000), (h, 2, 1_000_000), (other, 1, 5_000_000)])
    out = tmp_path / "t.json"
    profiling.main(["traffic", "--config", "3", "--fetch", str(tmp_path / "f.csv"), "--write", str(tmp_path / "w.csv"),
                    "--hits", str(tmp_path / "hm.csv"), "--stats", str(tmp_path / "s.csv"),
                    "--kernels", "gather_kernel|hub_", "--launches", "2", "--command", "cmd", "--out", str(out)])
    d = json.loads(out.read_text())
    gather = (400 * 2 + 20 * 1) * 1024 / 2
    hub = (100 * 2 + 8 * 1) * 1024 / 2
    assert d["per_kernel"]["gather_kernel<4>"]["hbm_bytes_per_step"] == round(gather)
    assert d["per_kernel"]["hub_tiles_kernel<4, 2>"]["hbm_bytes_per_step"] == round(hub)
    assert d["hbm_bytes_per_launch"] == round(gather + hub)
    assert d["per_kernel"]["gather_kernel<4>"]["l2_hit_rate"] == 0.75
    assert "degree_kernel" not in d["per_kernel"]
    assert d["copy_calibration"]["fetch_scale"] == 2.0 and d["copy_calibration"]["write_scale"] == 1.0
    assert d["step_kernel_ms_rocprof"] == 3.0  # 2 ms + 1 ms, one dispatch each per step
    assert "tcc_amd/csrc/hub_tiles.hip" in d["sources"] and d["command"] == "cmd"


def test_stats_table(tmp_path):
    _stats(tmp_path / "s.csv", [("void tcc::a_kernel(int)", 4, 1_500_000), ("void tcc::b_kernel(int)", 1, 500_000)])
    out = tmp_path / "s.md"
    profiling.main(["stats", "--csv", str(tmp_path / "s.csv"), "--title", "T", "--command", "python bench.py",
                    "--out", str(out)])
    text = out.read_text()
    assert "python bench.py" in text
    assert "| `a_kernel` | 4 | 1.5000 | 6.00 | 92.3 |" in text


def test_counters_table_mfma_busy(tmp_path):
    k = "void tcc::(anonymous namespace)::dense_tn_kernel<4>(tcc::(anonymous namespace)::TnArgs)"
    # 2 dispatches; GRBM_GUI_ACTIVE summed over 8 XCDs: 8 * 1000 cycles; busy 1024 SIMDs * 500
    _counters(tmp_path / "c.csv", [(k, "GRBM_GUI_ACTIVE", 8000), (k, "GRBM_GUI_ACTIVE", 8000),
                                   (k, "SQ_VALU_MFMA_BUSY_CYCLES", 512000), (k, "SQ_VALU_MFMA_BUSY_CYCLES", 512000),
                                   (k, "SQ_WAIT_INST_ANY", 30), (k, "SQ_WAIT_INST_ANY", 30),
                                   (k, "SQ_WAVE_CYCLES", 120), (k, "SQ_WAVE_CYCLES", 120)])
    out = tmp_path / "c.md"
    profiling.main(["counters", "--csv", str(tmp_path / "c.csv"), "--kernels", "dense_tn", "--title", "T",
                    "--command", "cmd", "--out", str(out)])
    row = [ln for ln in out.read_text().splitlines() if ln.startswith("| `dense_tn_kernel<4>`")][0]
    assert row.endswith("| 0.500 | 0.250 |") and "| 2 |" in row


def test_kernel_sources_follow_definitions_and_includes():
    srcs = profiling.kernel_sources(["gather_kernel<4, (Src)2, true>", "hub_reduce_kernel"])
    assert "tcc_amd/csrc/bcsr_spmm.hip" in srcs and "tcc_amd/csrc/hub_tiles.hip" in srcs
    assert "tcc_amd/csrc/common.hpp" in srcs  # included by both
    assert "tcc_amd/csrc/swtcf_convert.hip" not in srcs  # defines none of them
    sha = profiling.sources_sha(["tile_emit_kernel<unsigned int>"])
    assert list(sha) == profiling.kernel_sources(["tile_emit_kernel"])
    assert "tcc_amd/csrc/swtcf_convert.hip" in sha and "tcc_amd/csrc/hub_tiles.hip" not in sha


def _trace(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for name, start, end in rows:
            w.writerow({"Kind": "KERNEL_DISPATCH", "Kernel_Name": name, "Start_Timestamp": start,
                        "End_Timestamp": end})


def test_step_period_from_the_anchor_kernel(tmp_path):
    """Steps whose kernels overlap on two streams: the period is anchor start
    to anchor start (the steps' wall time), not the sum of the durations; the
    rows come in any order."""
    pack = "void tcc::(anonymous namespace)::tf32_pack_kernel(float const*, unsigned int)"
    full = "void tcc::(anonymous namespace)::gather_kernel<4, (tcc::(anonymous namespace)::Src)4, false>(int)"
    last = "void tcc::(anonymous namespace)::gather_kernel<2, (tcc::(anonymous namespace)::Src)4, false>(int)"
    rows = []
    for i, t0 in enumerate((1_000_000, 5_000_000, 9_500_000)):
        rows += [(pack, t0, t0 + 200_000), (full, t0 + 300_000, t0 + 3_800_000), (last, t0 + 300_000, t0 + 2_300_000)]
    rows.reverse()
    _trace(tmp_path / "k.csv", rows)
    assert profiling.step_periods(str(tmp_path / "k.csv"), "^tf32_pack_kernel$") == [4.0, 4.5]
    _stats(tmp_path / "s.csv", [(pack, 3, 200_000), (full, 3, 3_500_000), (last, 3, 2_000_000)])
    out = tmp_path / "p.md"
    profiling.main(["stats", "--csv", str(tmp_path / "s.csv"), "--title", "t",
                    "--command", "rocprofv3 --kernel-trace --stats --output-format csv -d /tmp/s -o run -- python x.py",
                    "--kernels", "gather_kernel|tf32_pack", "--launches", "3", "--trace", str(tmp_path / "k.csv"),
                    "--anchor", "^tf32_pack_kernel$", "--out", str(out)])
    text = out.read_text()
    assert "median **4.2500 ms**, min 4.0000, max 4.5000" in text
    assert "--csv /tmp/s/run_kernel_stats.csv" in text and "--trace /tmp/s/run_kernel_trace.csv" in text
    assert "| **per step** | | | **5.7000** |" in text  # overlapping durations add up past the period
