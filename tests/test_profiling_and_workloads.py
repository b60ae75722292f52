"""CPU checks of the rocprofv3 summarizer (`aspec_amd.profiling`) and of the reference's B = 7
workload fixture.

* Kernel names shorten to the kernel's own name with its template arguments; dispatches group by
  (name, grid size), so the teacher and dgrad GEMMs (one solution, two grids) are told apart; the
  idle time before a dispatch is its start minus the latest end of every earlier dispatch.
* Traffic: the copy kernel's FETCH_SIZE / WRITE_SIZE readings give the byte scale.
* The B = 7 workload: its visible pairs per head equal the reference's own accounting
  Sum_blocks B (u + B) (tools/performance/bench_dspark_b7_attention.py:173-176) over the fixture's
  document-local anchors, 358,904,588 (20.58 TFLOP for fwd + bwd at GQA 32/8 x 128), and the
  packed row has the study's 43008 query rows and 174080 key rows.
"""

import csv

import numpy as np

from aspec_amd import profiling as P
from aspec_amd import workloads as W
from oracle import metadata as M

GEMM = "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname1_gfx950"


def test_short_names():
    assert P.short_name("void aspec::(anonymous namespace)::attn_fwd_kernel<4>(aspec::(anonymous "
                        "namespace)::AttnArgs)") == "attn_fwd_kernel<4>"
    assert P.short_name("void aspec::(anonymous namespace)::loss_fwd_persistent<8, false, true, "
                        "true>(aspec::LossArgs)") == "loss_fwd_persistent<8, false, true, true>"
    assert P.short_name(GEMM) == GEMM
    assert P.short_name("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"


def _trace(path, rows):
    fields = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y",
              "Grid_Size_Z"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for name, grid, start, end in rows:
            w.writerow({"Kind": "KERNEL_DISPATCH", "Kernel_Name": name, "Start_Timestamp": start,
                        "End_Timestamp": end, "Grid_Size_X": grid, "Grid_Size_Y": 1, "Grid_Size_Z": 1})


def test_trace_groups_regions_and_gaps(tmp_path):
    path = tmp_path / "k.csv"
    _trace(path, [(GEMM, 512000, 0, 700_000),                       # teacher
                  ("void aspec::attn_fwd_kernel<4>(x)", 524288, 650_000, 950_000),
                  (GEMM, 131072, 1_050_000, 2_250_000),             # dgrad, 100 us after the latest end
                  (GEMM, 131072, 2_255_000, 3_455_000)])            # dgrad, 5 us gap
    d = P.load_dispatches(path)
    stats = P.kernel_stats(d)
    assert stats[P.group_key(GEMM, 131072)]["calls"] == 2
    assert abs(stats[P.group_key(GEMM, 131072)]["avg_us"] - 1200.0) < 1e-9
    regions = P.region_stats(d)
    assert regions["teacher_gemm"]["calls"] == 1 and regions["head_gemm_dgrad"]["calls"] == 2
    assert abs(regions["attn_fwd"]["avg_us"] - 300.0) < 1e-9
    gaps = P.idle_gaps(d, "shortname1", 131072)
    assert np.allclose(gaps, [100.0, 5.0])
    # an overlapping dispatch has no idle time before it
    assert P.idle_gaps(d, "attn_fwd") == [0.0]
    text = P.trace_markdown(d, ["shortname1@131072"])
    assert "1 above 10 us" in text


def _counters(path, rows, counter):
    fields = ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for name, grid, value in rows:
            w.writerow({"Kernel_Name": name, "Grid_Size": grid, "Counter_Name": counter, "Counter_Value": value})


def test_traffic_calibration(tmp_path):
    mib = 512
    _counters(tmp_path / "cf.csv", [("__amd_rocclr_copyBuffer", 1, mib * 512.0), ("fill", 1, 3.0)], "FETCH_SIZE")
    _counters(tmp_path / "cw.csv", [("__amd_rocclr_copyBuffer", 1, mib * 1024.0)], "WRITE_SIZE")
    _counters(tmp_path / "f.csv", [(GEMM, 131072, 1000.0), (GEMM, 131072, 3000.0), (GEMM, 512000, 10.0)], "FETCH_SIZE")
    _counters(tmp_path / "w.csv", [(GEMM, 131072, 50.0), (GEMM, 131072, 50.0)], "WRITE_SIZE")
    out = P.traffic(tmp_path / "f.csv", tmp_path / "w.csv", tmp_path / "cf.csv", tmp_path / "cw.csv", mib)
    assert out["calibration"]["fetch_factor"] == 2.0 and out["calibration"]["write_factor"] == 1.0
    dgrad = out["regions"]["head_gemm_dgrad"]
    assert dgrad["read_bytes"] == 2000.0 * 1024 * 2 and dgrad["write_bytes"] == 50.0 * 1024
    assert out["regions"]["teacher_gemm"]["write_bytes"] is None


def test_reference_b7_workload_matches_the_reference_accounting():
    import json

    data = json.loads(W.B7_FIXTURE.read_text())
    block = data["block"]
    closed_form = sum(int(((np.asarray(a, np.int64) + block) * block).sum()) for a in data["anchor_positions"])
    assert closed_form == 358_904_588
    w = W.reference_b7()
    assert (w.num_queries, w.num_keys, w.context_length) == (43008, 174080, 131072)
    assert w.block_size == 7 and w.num_blocks == 6144
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length)
    pairs = int((ends[2] - ends[1]).sum() + (ends[4] - ends[3]).sum())
    assert pairs == closed_form
    assert round(14 * 32 * 128 * pairs / 1e12, 2) == 20.58
    pub = W.reference_b7_published()
    assert round(pub["ms"]["cudnn_joint"]["fb"]["median_ms"], 2) == 18.12
    assert pub["timing_contract"]["windows"] == 11 and pub["timing_contract"]["retained"] == 9
