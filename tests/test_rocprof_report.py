"""The measurement harness behind profiles/ (helm_amd/rocprof_report.py) on
synthetic rocprofv3 CSVs: kernel names, per-kernel durations, the HBM byte
scale measured from calibration copies, counter ratios, and the run script."""
import csv
import json

import pytest

from helm_amd import rocprof_report as R

TRACE_COLS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id",
              "Kernel_Id", "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp",
              "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count",
              "Workgroup_Size_X", "Workgroup_Size_Y", "Workgroup_Size_Z", "Grid_Size_X",
              "Grid_Size_Y", "Grid_Size_Z"]
CTR_COLS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
            "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
            "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
            "Counter_Value", "Start_Timestamp", "End_Timestamp"]
DEC = "void helm::decode_mfma_kernel<helm::bf16_t, helm::PoolSrc, 0, 4>(helm::AttnParams, X)"
MRG = "void helm::merge_splits_d128_kernel<helm::bf16_t>(helm::AttnParams)"
COPY = "__amd_rocclr_copyBuffer"


def _trace(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, TRACE_COLS)
        w.writeheader()
        for i, (name, start_ns, dur_ns) in enumerate(rows):
            w.writerow({"Kind": "KERNEL_DISPATCH", "Dispatch_Id": i + 1, "Kernel_Name": name,
                        "Start_Timestamp": start_ns, "End_Timestamp": start_ns + dur_ns,
                        "LDS_Block_Size": 39936, "Scratch_Size": 0, "VGPR_Count": 168,
                        "Accum_VGPR_Count": 0, "SGPR_Count": 100, "Workgroup_Size_X": 256,
                        "Workgroup_Size_Y": 1, "Workgroup_Size_Z": 1, "Grid_Size_X": 8192,
                        "Grid_Size_Y": 8, "Grid_Size_Z": 1})


def _ctr(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, CTR_COLS)
        w.writeheader()
        for i, (name, counter, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Grid_Size": 1,
                        "Counter_Name": counter, "Counter_Value": value})


def test_short_names():
    assert R.short_name(DEC) == "decode_mfma_kernel<bf16, PoolSrc, 0, 4>"
    assert R.short_name(MRG) == "merge_splits_d128_kernel<bf16>"
    assert R.short_name("(anonymous namespace)::stream_copy_kernel(unsigned int*, long)") == \
        "stream_copy_kernel"
    long = "at::native::k<" + "x" * 200 + ">(int)"
    assert R.short_name(long) == "at::native::k<...>"


def test_kernel_stats_and_headline_times(tmp_path):
    d = tmp_path / "headline"
    d.mkdir()
    rows = [(DEC, 1000 * i, 22000 + 100 * (i % 3)) for i in range(9)] + \
           [(MRG, 1000 * i, 4000) for i in range(9)]
    _trace(d / "run_kernel_trace.csv", rows)
    st = R.kernel_stats(R.kernel_trace([str(d)]))
    key = ("decode_mfma_kernel<bf16, PoolSrc, 0, 4>", "8192 x 8 x 1")
    assert st[key]["dispatches"] == 9
    assert st[key]["mean_us"] == pytest.approx(22.1)
    assert st[key]["median_us"] == pytest.approx(22.1)
    t = R.headline_times(st)
    assert t["decode_kernel_avg_us"] == 22.1 and t["merge_kernel_avg_us"] == 4.0
    assert t["call_kernels_us"] == 26.1
    md = R.kernels_md(st, "T", ["cmd"])
    assert "| `decode_mfma_kernel<bf16, PoolSrc, 0, 4>` | 8192 x 8 x 1 | 9 | 22.10 |" in md


def test_traffic_scales_from_the_calibration_copies(tmp_path):
    """The counters read half the copy's KiB for FETCH_SIZE and all of them
    for WRITE_SIZE; small copies of the same run do not set the scale."""
    gib = 1 << 30
    f, w = tmp_path / "fetch", tmp_path / "write"
    f.mkdir()
    w.mkdir()
    _ctr(f / "f_counter_collection.csv",
         [(COPY, "FETCH_SIZE", 64.0)] +                       # a small copy
         [(COPY, "FETCH_SIZE", gib / 2048)] * 3 +             # three 1 GiB copies
         [(DEC, "FETCH_SIZE", 65000.0), (DEC, "FETCH_SIZE", 65002.0),
          (MRG, "FETCH_SIZE", 300.0)])
    _ctr(w / "w_counter_collection.csv",
         [(COPY, "WRITE_SIZE", 64.0)] + [(COPY, "WRITE_SIZE", gib / 1024)] * 3 +
         [(DEC, "WRITE_SIZE", 520.0), (MRG, "WRITE_SIZE", 8.0)])
    t = R.traffic([str(f)], [str(w)], 134242304, r"^decode_mfma", r"^merge_splits")
    assert t["fetch_scale"] == pytest.approx(2.0)
    assert t["write_scale"] == pytest.approx(1.0)
    assert t["decode_fetch_bytes"] == pytest.approx(65001.0 * 1024 * 2)
    assert t["decode_write_bytes"] == pytest.approx(520.0 * 1024)
    assert t["hbm_bytes_per_launch"] == pytest.approx(
        (65001.0 * 2 + 520.0 + 300.0 * 2 + 8.0) * 1024)
    with pytest.raises(ValueError):
        R.traffic([str(w)], [str(w)], 1, r"^decode_mfma", r"^merge_splits")


CHK = "void helm::chunk32_mfma_kernel<helm::bf16_t, helm::DescSrc, 4, 8>(helm::AttnParams, X)"
MRW = "void helm::merge_rows_d128_kernel<helm::bf16_t>(helm::AttnParams)"


@pytest.mark.parametrize("with_chunk", [True, False])
def test_prefill_traffic_summary_from_the_same_passes(tmp_path, with_chunk):
    """The traffic passes that include the prefill leg also give the chunk
    kernel's bytes (scaled like the decode kernel's) and its ratio to the K,
    V and query bytes; passes without the prefill leg write no such file."""
    gib = 1 << 30
    runs = tmp_path / "runs"
    f, w = runs / "fetch", runs / "write"
    f.mkdir(parents=True)
    w.mkdir()
    chunk_f = [(CHK, "FETCH_SIZE", 74000.0), (MRW, "FETCH_SIZE", 16700.0)] if with_chunk else []
    chunk_w = [(CHK, "WRITE_SIZE", 33284.0), (MRW, "WRITE_SIZE", 4096.0)] if with_chunk else []
    _ctr(f / "run_counter_collection.csv",
         [(COPY, "FETCH_SIZE", gib / 2048)] * 3 +
         [(DEC, "FETCH_SIZE", 65000.0), (MRG, "FETCH_SIZE", 300.0)] + chunk_f)
    _ctr(w / "run_counter_collection.csv",
         [(COPY, "WRITE_SIZE", gib / 1024)] * 3 +
         [(DEC, "WRITE_SIZE", 520.0), (MRG, "WRITE_SIZE", 8.0)] + chunk_w)
    out = tmp_path / "out"
    written = [str(x) for x in R.write_all(str(runs), str(out))]
    name = "prefill_chunk32_qwen3-8b-512x32k_traffic.md"
    assert any(x.endswith("paged_decode_qwen3-8b-32k_traffic.md") for x in written)
    assert any(x.endswith(name) for x in written) == with_chunk
    if with_chunk:
        md = (out / name).read_text()
        assert f"{74000 * 1024 * 2:,} B read, {33284 * 1024:,} B written" in md
        assert f"x{74000 * 1024 * 2 / R.PREFILL_READ_BYTES:.4f}" in md
        assert R.PREFILL_READ_BYTES == 32768 * 4096 + 512 * 32 * 256


def test_counter_ratios(tmp_path):
    rows = [("void helm::chunk32_mfma_kernel<helm::bf16_t, helm::DescSrc, 4, 8>(A, B)", c, v)
            for c, v in (("SQ_INSTS_MFMA", 1000.0), ("SQ_INSTS_VALU", 5500.0),
                         ("SQ_INSTS_SALU", 4800.0), ("SQ_VALU_MFMA_BUSY_CYCLES", 1024 * 42.0),
                         ("GRBM_GUI_ACTIVE", 800.0), ("SQ_WAVE_CYCLES", 100.0),
                         ("SQ_ACTIVE_INST_ANY", 39.0))]
    _ctr(tmp_path / "a_counter_collection.csv", rows)
    md = R.counters_md(R.counter_means(R.counter_rows([str(tmp_path)])), ".", "T", [])
    assert "VALU per MFMA 5.50" in md and "SALU per MFMA 4.80" in md
    assert "matrix pipe busy 0.420" in md          # 42 cycles per SIMD of 100 per XCD
    assert "issuing 0.390" in md


def test_run_script_and_bench_summary(tmp_path):
    lines = R.run_commands("rocprof_runs")
    body = "\n".join(lines)
    assert lines[0] == "#!/bin/bash" and "cd /tmp && export TMPDIR=/tmp" in body
    for name in R.RUNS:
        assert f"-d $R/rocprof_runs/{name} " in body
    # every counter pass under a SIGKILL time limit, the program after --
    for ln in lines:
        if "--pmc" in ln:
            assert ln.startswith("timeout -s KILL ") and " -- python3 -u " in ln
    line = {"roofline": {"per_call": {"us": 26.6}, "avg_launch_us": 24.0},
            "workgroup_stamps": {"how": "h", "workgroups": 256, "captures": 2,
                                 "start_us": {"min": 0, "mean": 0.1, "max": 0.2, "std": 0.1},
                                 "loop_end_us": {"min": 18, "mean": 20, "max": 21, "std": 1},
                                 "end_us": {"min": 18.4, "mean": 20.4, "max": 21.4, "std": 1},
                                 "loop_end_spread_us_per_capture": [3, 2.5],
                                 "last_end_us_per_capture": [21.4, 21.3],
                                 "loop_end_mean_per_xcd_us": {"0": 20},
                                 "loop_end_mean_per_kv_head_us": {"0": 20},
                                 "lateness_correlation_between_calls": 0.4},
            "read_pass_floor": {"how": "h", "kv_bytes": 134217728, "tail_bytes": 532480,
                                "iters": 10, "workgroups_256": {"read_us": 21.5,
                                                                "read_GBs": 6242.7,
                                                                "read_then_tail_us": 24.5}}}
    p = tmp_path / "bench.json"
    p.write_text("[bench] noise\n" + json.dumps(line) + "\n")
    out = R.bench_summaries(str(p), str(tmp_path), "python3 bench.py --stamps")
    assert len(out) == 2
    assert "| 256 | 21.5 | 6242.7 | 24.5 |" in open(out[1]).read()


def test_copy_runs_group_large_copies_by_stream(tmp_path):
    """Consecutive large host-to-device copies on one stream form a run; its
    median copy time and start-to-start cycle; small and device-to-host
    copies do not count."""
    cols = ["Kind", "Direction", "Stream_Id", "Source_Agent_Id", "Destination_Agent_Id",
            "Correlation_Id", "Start_Timestamp", "End_Timestamp"]
    rows = []
    t = 0
    for stream, n, dur, cyc in (("1", 3, 1_170_000, 1_210_000), ("0", 4, 1_177_000, 1_300_000),
                                ("2", 3, 1_185_000, 1_250_000)):
        for _ in range(n):
            rows.append(("MEMORY_COPY", "MEMORY_COPY_HOST_TO_DEVICE", stream, t, t + dur))
            rows.append(("MEMORY_COPY", "MEMORY_COPY_HOST_TO_DEVICE", stream, t + 10, t + 4000))
            rows.append(("MEMORY_COPY", "MEMORY_COPY_DEVICE_TO_HOST", stream, t + 20, t + 900_000))
            t += cyc
        t += 20_000_000
    with open(tmp_path / "run_memory_copy_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, cols)
        w.writeheader()
        for i, (kind, d, s, a, b) in enumerate(rows):
            w.writerow({"Kind": kind, "Direction": d, "Stream_Id": s, "Correlation_Id": i,
                        "Start_Timestamp": a, "End_Timestamp": b})
    runs = R.copy_runs([str(tmp_path)])
    assert [(r["stream"], r["copies"]) for r in runs] == [("1", 3), ("0", 4), ("2", 3)]
    assert runs[1]["copy_us_median"] == 1177.0 and runs[1]["cycle_us_median"] == 1300.0
    assert runs[2]["cycle_us_median"] == 1250.0 and runs[0]["start_ms"] == 0.0
