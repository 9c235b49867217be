"""The profile summaries bench.py writes into profiles/ (rocprofv3 csv -> tables and json), on
synthetic counter files with known answers: byte calibration against the copy kernel, the
autotuner's candidate tilings left out of a stage's bytes, per-dispatch sums over counter
instances, and the MFMA busy / clock / LDS ratios. CPU only."""

import csv
import json

import pytest

import bench

GEMM = "void sfenc::gemm_kernel<1, 0, 2, 8, 0>(sfenc::GemmArgs)"
GEMM_4W = "void sfenc::gemm_kernel<1, 0, 2, 4, 0>(sfenc::GemmArgs)"
ROWS = "void sfenc::gemm_kernel<1, 0, 1, 8, 1>(sfenc::GemmArgs)"
COPY = "void at::native::neg_kernel(float)"
DECODE = "void (anonymous namespace)::decode_lines_kernel<1, true, 4, 4>((anonymous namespace)::LineArgs)"
COMPACT = "void (anonymous namespace)::compact_row_kernel<2>(char const*, long, long)"

FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
          "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
          "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def write_pmc(d, dispatches):
    """dispatches: [(dispatch_id, kernel, ns, {counter: [instance values]}[, grid[, workgroup size]])] ->
    rocprofv3 csv files."""
    d.mkdir(parents=True, exist_ok=True)
    with open(d / "bench_agent_info.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, ["Name", "Num_Xcc", "Simd_Count", "Cu_Count", "Max_Engine_Clk_Fcompute"])
        w.writeheader()
        w.writerow({"Name": "CPU", "Num_Xcc": 0, "Simd_Count": 0, "Cu_Count": 0, "Max_Engine_Clk_Fcompute": 0})
        w.writerow({"Name": "gfx950", "Num_Xcc": 8, "Simd_Count": 1024, "Cu_Count": 256,
                    "Max_Engine_Clk_Fcompute": 2400})
    with open(d / "bench_counter_collection.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, FIELDS)
        w.writeheader()
        for did, name, ns, counters, *grid in dispatches:
            for c, vals in counters.items():
                for v in vals:  # one row per counter instance (XCD / SE), summed per dispatch
                    w.writerow({**{f: 0 for f in FIELDS}, "Dispatch_Id": did, "Kernel_Name": name, "Counter_Name": c,
                                "Counter_Value": v, "Start_Timestamp": 1000, "End_Timestamp": 1000 + ns,
                                "Grid_Size": grid[0] if grid else 0,
                                "Workgroup_Size": grid[1] if len(grid) > 1 else 0})


def test_kernel_stage_tells_dense_from_row_candidate_gemms():
    assert bench.kernel_stage(GEMM) == "encode"
    assert bench.kernel_stage(GEMM_4W) == "encode"
    assert bench.kernel_stage(ROWS) == "encode_rows"
    assert bench.kernel_stage("void sfenc::gemm_kernel<2, 0, 2, 8, 2, false>(sfenc::GemmArgs)") == "encode_rows"
    assert bench.kernel_stage("void sfenc::gemm_kernel<1, 0, 2, 8, 0, false>(sfenc::GemmArgs)") == "encode"
    assert bench.kernel_stage("void sfenc::gemm_kernel<2, 0, 2, 8, 0, true>(sfenc::GemmArgs)") == "encode"
    assert bench.kernel_stage(DECODE) == "decode"
    assert bench.kernel_stage(COMPACT) == "compact"
    assert bench.kernel_stage("void unrelated_kernel()") is None


def test_pmc_dispatches_sums_counter_instances(tmp_path):
    write_pmc(tmp_path, [(7, GEMM, 5000, {"SQ_WAVE_CYCLES": [10, 20, 30], "GRBM_GUI_ACTIVE": [4] * 8})])
    disp, gpu = bench._pmc_dispatches(str(tmp_path))
    (d,) = disp.values()
    assert d["SQ_WAVE_CYCLES"] == 60 and d["GRBM_GUI_ACTIVE"] == 32
    assert d["ns"] == 5000 and d["name"] == GEMM and d["id"] == 7
    assert gpu["Name"] == "gfx950"


def test_traffic_summary_calibrates_on_the_copy_kernel_and_keeps_the_last_tiling(tmp_path, monkeypatch):
    """The copy kernel over 1 MiB reads as 2 MiB of FETCH and 1 MiB of WRITE (factors 0.5 and 1);
    the autotuner's 4-wave candidate ran first, the kept 8-wave tiling last: only the latter's
    bytes (and the compaction's) count."""
    monkeypatch.setattr(bench, "TRAFFIC_FILE", tmp_path / "traffic.json")
    kib = 1024.0  # counters are in KiB
    write_pmc(tmp_path / "fetch", [
        (1, COPY, 100, {"FETCH_SIZE": [2 * kib]}),
        (2, GEMM_4W, 100, {"FETCH_SIZE": [999 * kib]}),
        (3, GEMM, 100, {"FETCH_SIZE": [300 * kib, 100 * kib]}),
        (4, COMPACT, 100, {"FETCH_SIZE": [50 * kib]}),
    ])
    write_pmc(tmp_path / "write", [
        (1, COPY, 100, {"WRITE_SIZE": [1 * kib]}),
        (2, GEMM_4W, 100, {"WRITE_SIZE": [999 * kib]}),
        (3, GEMM, 100, {"WRITE_SIZE": [64 * kib]}),
        (4, COMPACT, 100, {"WRITE_SIZE": [2 * kib]}),
    ])
    bench.traffic_summary(str(tmp_path), 1, "C3")
    out = json.loads((tmp_path / "traffic.json").read_text())["C3"]
    mib = 1 << 20
    assert out["_calibration"]["fetch_factor"] == 0.5 and out["_calibration"]["write_factor"] == 1.0
    assert out["_split"]["encode"] == {"fetch": 200 * mib, "write": 64 * mib}
    assert out["encode"] == 264 * mib
    assert out["compact"] == 25 * mib + 2 * mib


def test_traffic_summary_keeps_launch_shapes_apart(tmp_path, monkeypatch):
    """One GEMM kernel at two grids (C4: the floor encode of 4096 features, then the dense
    encode of all of them): the stage holds the shape that ran last, the other shape gets its
    own entry, and neither is an average of both."""
    monkeypatch.setattr(bench, "TRAFFIC_FILE", tmp_path / "traffic.json")
    kib = 1024.0
    small, big = 512 * 512, 16384 * 512
    write_pmc(tmp_path / "fetch", [
        (1, COPY, 100, {"FETCH_SIZE": [1 * kib]}, 1),
        (2, GEMM, 100, {"FETCH_SIZE": [10 * kib]}, small),
        (3, GEMM, 100, {"FETCH_SIZE": [12 * kib]}, small),
        (4, GEMM, 100, {"FETCH_SIZE": [700 * kib]}, big),
    ])
    write_pmc(tmp_path / "write", [
        (1, COPY, 100, {"WRITE_SIZE": [1 * kib]}, 1),
        (2, GEMM, 100, {"WRITE_SIZE": [2 * kib]}, small),
        (3, GEMM, 100, {"WRITE_SIZE": [2 * kib]}, small),
        (4, GEMM, 100, {"WRITE_SIZE": [300 * kib]}, big),
    ])
    bench.traffic_summary(str(tmp_path), 1, "C4")
    out = json.loads((tmp_path / "traffic.json").read_text())["C4"]
    mib = 1 << 20
    assert out["encode"] == 1000 * mib
    assert out[f"encode@grid{small}"] == 13 * mib


def test_traffic_summary_tells_candidates_from_other_shapes_by_the_outputs_covered(tmp_path, monkeypatch, capsys):
    """The 4-wave candidate (256-thread workgroups) of the kept 8-wave tiling (512) has half its
    grid yet covers the same outputs: an autotune candidate, not another shape; the 256x128
    tiling (gemm2_kernel) at the same grid as the kept one covers the same outputs too."""
    monkeypatch.setattr(bench, "TRAFFIC_FILE", tmp_path / "traffic.json")
    kib = 1024.0
    gemm2 = "void sfenc::gemm2_kernel<1, 0, 2>(sfenc::GemmArgs)"
    tiles = 16384
    for sub, c in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")):
        write_pmc(tmp_path / sub, [
            (1, COPY, 100, {c: [1 * kib]}, 1, 256),
            (2, GEMM_4W, 100, {c: [900 * kib]}, tiles * 256, 256),
            (3, gemm2, 100, {c: [800 * kib]}, 2 * tiles * 256, 256),
            (4, GEMM, 100, {c: [700 * kib]}, tiles * 512, 512),
        ])
    bench.traffic_summary(str(tmp_path), 1, "C3")
    out = json.loads((tmp_path / "traffic.json").read_text())["C3"]
    assert [k for k in out if k.startswith("encode")] == ["encode"]
    assert out["encode"] == 700 * (1 << 20) * 2  # fetch x 1 + write x 1 (calibration factors 1)
    table = capsys.readouterr().out
    assert table.count("(autotune candidate)") == 2 and "other shape" not in table


def test_stats_summary_one_row_per_kernel_and_grid(tmp_path, capsys):
    fields = ["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y",
              "Grid_Size_Z"]
    with open(tmp_path / "x_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fields)
        w.writeheader()
        for i, (g, ns) in enumerate([(512, 200_000), (512, 240_000), (8192, 7_000_000), (8192, 7_200_000)]):
            w.writerow({"Kind": "KERNEL_DISPATCH", "Dispatch_Id": i, "Kernel_Name": GEMM, "Start_Timestamp": 0,
                        "End_Timestamp": ns, "Grid_Size_X": g, "Grid_Size_Y": 1, "Grid_Size_Z": 1})
    bench.stats_summary(str(tmp_path))
    out = capsys.readouterr().out
    assert "| `sfenc::gemm_kernel<1, 0, 2, 8, 0>` | 8192 | 2 | 7100.0 | 7000.0 | 7200.0 |" in out
    assert "| `sfenc::gemm_kernel<1, 0, 2, 8, 0>` | 512 | 2 | 220.0 | 200.0 | 240.0 |" in out


def test_mfma_summary_busy_clock_and_flops(tmp_path, monkeypatch):
    """busy = SQ_VALU_MFMA_BUSY_CYCLES / (GPU cycles x SIMDs); GPU cycles = GRBM_GUI_ACTIVE
    summed over the 8 XCDs / 8; clock = cycles / duration; flops = MOPS x 512."""
    monkeypatch.setattr(bench, "MFMA_FILE", tmp_path / "mfma.json")
    ns, cycles = 4_000_000, 6_600_000  # 4 ms at 1.65 GHz
    write_pmc(tmp_path, [(1, GEMM, ns, {"SQ_VALU_MFMA_BUSY_CYCLES": [0.68 * cycles * 1024],
                                         "SQ_INSTS_VALU_MFMA_MOPS_BF16": [4.9478e12 / 512],
                                         "GRBM_GUI_ACTIVE": [cycles] * 8})])
    bench.mfma_summary(str(tmp_path), "C3")
    rec = json.loads((tmp_path / "mfma.json").read_text())["C3"]
    assert rec["mfma_busy"] == pytest.approx(0.68, abs=1e-4)
    assert rec["clock_ghz"] == pytest.approx(1.65, abs=1e-3)
    assert rec["tflops"] == pytest.approx(4.9478e12 / 4e-3 / 1e12, abs=0.1)
    assert rec["mfma_flops"] == pytest.approx(4.9478e12)


def test_sq_and_lds_summaries(tmp_path, capsys):
    cycles = 1_000_000  # per XCD
    cu_cycles = cycles * 256
    write_pmc(tmp_path, [
        (1, GEMM, 4_000_000, {"SQ_WAVE_CYCLES": [1000.0], "SQ_BUSY_CYCLES": [1.0], "SQ_WAIT_ANY": [360.0],
                              "SQ_WAIT_INST_ANY": [420.0], "SQ_INSTS_LDS": [1.6e8], "SQ_LDS_BANK_CONFLICT": [0.0],
                              "SQ_INSTS_VMEM": [4e7], "GRBM_GUI_ACTIVE": [cycles] * 8}),
        (2, DECODE, 360_000, {"SQ_LDS_IDX_ACTIVE": [0.25 * cu_cycles], "SQ_LDS_BANK_CONFLICT": [0.0],
                              "SQ_LDS_DATA_FIFO_FULL": [0.005 * cu_cycles], "SQ_LDS_CMD_FIFO_FULL": [0.0],
                              "SQ_INSTS_LDS_LOAD_BANDWIDTH": [0.0], "SQ_INSTS_LDS_STORE_BANDWIDTH": [0.0],
                              "GRBM_GUI_ACTIVE": [cycles] * 8}),
        (3, GEMM, 4_000_000, {"SQ_LDS_IDX_ACTIVE": [0.284 * cu_cycles], "SQ_LDS_BANK_CONFLICT": [0.033 * 0.284 * cu_cycles],
                              "SQ_LDS_DATA_FIFO_FULL": [0.0], "SQ_LDS_CMD_FIFO_FULL": [0.001 * cu_cycles],
                              "SQ_INSTS_LDS_LOAD_BANDWIDTH": [67.5 / 64 * cu_cycles],
                              "SQ_INSTS_LDS_STORE_BANDWIDTH": [1.2 / 64 * cu_cycles],
                              "GRBM_GUI_ACTIVE": [cycles] * 8}),
    ])
    bench.sq_summary(str(tmp_path))
    sq = capsys.readouterr().out
    assert "| `sfenc::gemm_kernel<1, 0, 2, 8, 0>` | 1 | 4000.0 | 36.0% | 42.0% | 1.6e+08 | 0 | 4e+07 |" in sq
    bench.lds_summary(str(tmp_path))
    lds = capsys.readouterr().out
    assert "| `sfenc::gemm_kernel<1, 0, 2, 8, 0>` | 1 | 4000.0 | 28.4% | 67.5 | 1.2 | 0.0% | 0.1% | 3.3% |" in lds
    assert "| `decode_lines_kernel<1, true, 4, 4>` | 1 | 360.0 | 25.0% | 0.0 | 0.0 | 0.5% | 0.0% | 0.0% |" in lds


PERSIST = "void sfenc::gemm_persist_kernel<2, 0, 2, 0, 8>(sfenc::GemmArgs)"
PERSIST_4W = "void sfenc::gemm_persist_kernel<2, 0, 2, 0, 4>(sfenc::GemmArgs)"


def test_persistent_launches_are_split_by_size(tmp_path, monkeypatch, capsys):
    """The persistent encode's grid is the CU count at every problem size: at C4 its floor
    encode (the first features) and its dense encode share a grid and are told apart by their
    bytes; the dense one covers the configuration's T x d_sae outputs, so the 4-wave tilings of
    that problem (one workgroup per tile or persistent) are its autotune candidates, and the
    4-wave persistent launch of the floor encode is the candidate of that shape."""
    monkeypatch.setattr(bench, "TRAFFIC_FILE", tmp_path / "traffic.json")
    kib = 1024.0
    grid = 256 * 512
    tiles = 8192 // 256 * (131072 // 256)
    for sub, c in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")):
        write_pmc(tmp_path / sub, [
            (1, COPY, 100, {c: [1 * kib]}, 1, 256),
            (2, PERSIST, 100, {c: [10 * kib]}, grid, 512),
            (3, GEMM_4W, 100, {c: [900 * kib]}, tiles * 256, 256),
            (4, PERSIST_4W, 100, {c: [9 * kib]}, grid // 2, 256),
            (5, PERSIST_4W, 100, {c: [650 * kib]}, grid // 2, 256),
            (6, PERSIST, 100, {c: [700 * kib]}, grid, 512),
            (7, PERSIST, 100, {c: [11 * kib]}, grid, 512),
            (8, PERSIST, 100, {c: [720 * kib]}, grid, 512),
        ])
    bench.traffic_summary(str(tmp_path), 1, "C4")
    out = json.loads((tmp_path / "traffic.json").read_text())["C4"]
    mib = 1 << 20
    assert out["encode"] == 710 * mib * 2
    assert out[f"encode@grid{grid}"] == round(10.5 * mib * 2)
    table = capsys.readouterr().out
    assert "`sfenc::gemm_persist_kernel<2, 0, 2, 0, 8>#2` | 131072 | kept" in table
    assert "`sfenc::gemm_persist_kernel<2, 0, 2, 0, 8>#1` | 131072 | (other shape" in table
    assert "`sfenc::gemm_persist_kernel<2, 0, 2, 0, 4>#2` | 65536 | (autotune candidate)" in table
    assert "`sfenc::gemm_persist_kernel<2, 0, 2, 0, 4>#1` | 65536 | (autotune candidate)" in table
    assert table.count("(autotune candidate)") == 3


def test_stats_summary_splits_persistent_launches_by_duration(tmp_path, capsys):
    fields = ["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y",
              "Grid_Size_Z"]
    with open(tmp_path / "x_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fields)
        w.writeheader()
        for i, ns in enumerate([200_000, 7_000_000, 240_000, 7_200_000]):
            w.writerow({"Kind": "KERNEL_DISPATCH", "Dispatch_Id": i, "Kernel_Name": PERSIST, "Start_Timestamp": 0,
                        "End_Timestamp": ns, "Grid_Size_X": 131072, "Grid_Size_Y": 1, "Grid_Size_Z": 1})
    bench.stats_summary(str(tmp_path))
    out = capsys.readouterr().out
    assert "| `sfenc::gemm_persist_kernel<2, 0, 2, 0, 8>#2` | 131072 | 2 | 7100.0 | 7000.0 | 7200.0 |" in out
    assert "| `sfenc::gemm_persist_kernel<2, 0, 2, 0, 8>#1` | 131072 | 2 | 220.0 | 200.0 | 240.0 |" in out
    assert bench.kernel_stage(PERSIST) == "encode"
    assert bench.kernel_stage("void sfenc::gemm_persist_kernel<2, 0, 2, 2>(sfenc::GemmArgs)") == "encode_rows"
    assert bench.kernel_stage("void sfenc::gemm_persist_kernel<2, 0, 2, 2, 8>(sfenc::GemmArgs)") == "encode_rows"
    assert bench.kernel_stage("void sfenc::gemm_persist_kernel<1, 1, 1, 0, 4>(sfenc::GemmArgs)") == "encode"
