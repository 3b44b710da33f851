"""CPU tests of bench.py's measurement plumbing: the rocprofv3 CSV summaries
that the committed profiles are made with, the readers of those profiles that
fill the bench line's roofline, and the single-GPU guard. The CSVs are
synthetic, in rocprofv3's column layout, with known answers."""

import csv
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

BWD = "void wkv7::(anonymous namespace)::wkv7_bwd_chunk_kernel<false>(wkv7::(anonymous namespace)::BwdChunkParams)"
FWD = "void wkv7::(anonymous namespace)::wkv7_fwd_chunk_kernel<true>(wkv7::(anonymous namespace)::FwdChunkParams)"
ABS = "void at::native::vectorized_elementwise_kernel<4, at::native::AbsFunctor<float>, std::array<char*, 2ul> >"


def write_csv(path, header, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(header)
        w.writerows(rows)


def counter_rows(name, dispatch, counter, per_row):
    """One dispatch's rows (one per XCD), as rocprofv3 --pmc writes them."""
    return [[dispatch, dispatch, "Agent 1", 1, 1, 1, 256, 7, name, 512, 0, 0, 256, 0, 64,
             counter, v, 0, 1] for v in per_row]


PMC_HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
              "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
              "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
              "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def test_pmc_summary_sums_rows_averages_dispatches_and_scales_by_the_probe(tmp_path, capsys):
    probe_kib = bench.COPY_PROBE_BYTES / 1024
    rows = []
    # two backward dispatches, 8 rows each: 8 x 100 and 8 x 150 KiB -> mean 1000 KiB
    rows += counter_rows(BWD, 3, "FETCH_SIZE", [100.0] * 8)
    rows += counter_rows(BWD, 5, "FETCH_SIZE", [150.0] * 8)
    # an earlier probe-kernel dispatch that is not the probe, then the probe
    # itself reading half its bytes (as FETCH_SIZE does on this part)
    rows += counter_rows(ABS, 1, "FETCH_SIZE", [1.0] * 8)
    rows += counter_rows(ABS, 9, "FETCH_SIZE", [probe_kib / 2 / 8] * 8)
    rows += counter_rows(BWD, 3, "SQ_INSTS_VALU_MFMA_MOPS_BF16", [10.0] * 8)
    rows += counter_rows(BWD, 5, "SQ_INSTS_VALU_MFMA_MOPS_BF16", [10.0] * 8)
    write_csv(str(tmp_path / "p" / "run_counter_collection.csv"), PMC_HEADER, rows)
    bench.pmc_summary([str(tmp_path / "p")])
    out = capsys.readouterr().out
    # scale = 2 (probe read half), bytes = 1000 KiB x 1024 x 2
    assert f"traffic_bytes wkv7_bwd_chunk_kernel: {1000 * 1024 * 2}" in out
    assert "| wkv7_bwd_chunk_kernel | FETCH_SIZE | 1000 | 2.0 |" in out
    # MOPS count units of 512 FLOPs: 80 per dispatch
    assert f"mfma_flop_issued wkv7_bwd_chunk_kernel: {80 * 512}" in out


def test_stats_summary_table_counts_dispatches_per_step_and_takes_the_trace_median(tmp_path, capsys):
    stats_header = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs",
                    "StdDev"]
    write_csv(str(tmp_path / "s" / "run_kernel_stats.csv"), stats_header,
              [[BWD, 4, 4.0e6, 1.0e6, 60.0, 0.8e6, 1.4e6, 0.0],
               [FWD, 4, 2.0e6, 0.5e6, 30.0, 0.5e6, 0.5e6, 0.0],
               ["__amd_rocclr_copyBuffer", 2, 2.0e4, 1.0e4, 10.0, 1.0e4, 1.0e4, 0.0]])
    trace_header = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id",
                    "Kernel_Id", "Kernel_Name", "Correlation_Id", "Start_Timestamp",
                    "End_Timestamp"]
    trace = []
    for i, d in enumerate((1.4e6, 0.8e6, 0.9e6, 0.9e6)):     # backward durations, median 0.9 ms
        trace.append(["KERNEL_DISPATCH", "Agent 1", 1, 0, 1, i, 7, BWD, i, 1000, 1000 + int(d)])
    for i in range(4):
        trace.append(["KERNEL_DISPATCH", "Agent 1", 1, 0, 1, 10 + i, 8, FWD, 10 + i, 0, 500000])
    write_csv(str(tmp_path / "s" / "run_kernel_trace.csv"), trace_header, trace)
    bench.stats_summary(str(tmp_path / "s"), "cfg1", 2)
    out = capsys.readouterr().out
    lines = [l for l in out.splitlines() if l.startswith("| `")]
    assert lines[0] == "| `wkv7_bwd_chunk_kernel<false>` | 2 | 1000.0 | 900.0 | 800.0 | 1400.0 | 2.000 |"
    assert lines[1].startswith("| `wkv7_fwd_chunk_kernel<true>` | 2 | 500.0 | 500.0 |")
    assert len(lines) == 2   # runtime copies are not this library's kernels


def test_committed_profiles_feed_the_bench_line():
    """What the bench line reads from profiles/ parses, and is consistent with
    the algorithmic bytes and per-wave instruction counts the profiles state."""
    bwd_alg = 1_048_576 * 2_944
    traffic = bench.recorded_traffic("wkv7_bwd_chunk_kernel")
    assert traffic is not None and 0.98 < traffic / bwd_alg < 1.05
    assert bench.recorded_traffic("wkv7_infer_kernel", bench.TRAFFIC_FILE_DECODE) is not None
    assert bench.recorded_traffic("wkv7_infer_bf16_kernel", bench.TRAFFIC_FILE_DECODE) is not None
    mops = bench.recorded_counter("mfma_flop_issued", "wkv7_bwd_chunk_kernel", bench.COUNTER_FILE)
    valu = bench.recorded_counter("valu_insts", "wkv7_bwd_chunk_kernel", bench.COUNTER_FILE)
    assert mops is not None and valu is not None
    # per wave and chunk: 2048 waves x 256 chunks
    assert 300 < valu / (2048 * 256) < 600
    # issued bf16 work is a few times the fp32 algorithmic FLOPs (split products)
    assert 2.0 < mops / (bench.FLOP_BWD * 1_048_576) < 6.0


def test_neighbour_bytes_and_categories():
    alg = bench.neighbor_bytes(bench.CONFIGS["cfg4"])
    nb, what = alg["shift_mix_forward_kernel<false, true, 6>"]
    # B x T x C: x read as fp32, six bf16 mixes written
    assert nb == 16 * 512 * 768 * (4 + 6 * 2)
    assert bench.kernel_category("void wkv7::(anonymous namespace)::wkv7_fwd_chunk_kernel<true>(x)") \
        == "WKV7 (this library)"
    assert bench.kernel_category("Cijk_Alik_Bljk_BBS_BH_Bias") == "GEMM (hipBLASLt)"


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
