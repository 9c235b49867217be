"""Benchmark of the SAE hot path on one MI355X: fused encode -> dense->CSR -> sparse decode.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3] [--cpu-seconds S | --no-cpu]

One step = one pass of the path over one batch of the headline workload (C3: JumpReLU
bf16, d_in=2304, d_sae=65536, T=16384 tokens, mean L0 64, synthetic seeded inputs already
resident in HBM): zero row_nnz + fused encode with counting, exclusive scan, the host read
of nnz, compaction, sparse decode. Each kernel is bracketed by HIP events on the stream it
is launched on (torch's current stream) in every timed step.

Prints ONE JSON line. `value` is encode TFLOP/s over the timed steps (the metric's first
term, the dominant kernel). The decode appears twice: `decode_requested_gbps` is the
reference's formula (every gathered W_dec row counted once per use, bench_decode.py:57), not
an HBM rate, while `roofline_decode` divides the counter-measured HBM bytes by the flushed
launch time, so its `frac` is a true share of the 8 TB/s; the compaction rate sits beside
them. `torch_reference` times the torch ops the reference's bench compares against on this
GPU (sae.encode, sae(x), dense decode, to_sparse_csr), for scale. `path_rows` times the same path through the
row-candidate encode (per-row lists instead of the dense features, then lists -> CSR).
`backward` times the training backward of the path (sparse_backward: every parameter's
gradient from dL/dx_hat on the step's CSR) against its algorithmic bytes, and `train_step` a
whole training step without the optimizer (forward, MSE gradient, backward); `cache` the
activation-cache caller encoding a hook on the fly against its compute alone. `cpu_baseline` times
the CPU oracle on this host's cores over a bounded token subset of the same workload.
"""

import argparse
import json
import os
import statistics
import sys
import time
import warnings
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "encode TFLOP/s + decode GB/s (% of roofline), bf16 d_in=2304 d_sae=65536 L0=64"
PEAK_TFLOPS = {torch.bfloat16: 2516.6, torch.float16: 2516.6, torch.float32: 157.3}  # dense MFMA
PEAK_GBPS = 8000.0  # HBM3E
DTYPE_NAME = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _median_time(fn, reps=3):
    fn()  # warmup
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(sae, x, target_s):
    """The CPU restatement of the reference path, timed on this host's cores over a token
    subset of the same workload: encode = oracle.reference.encode (fp32 from the same rounded
    inputs, the reference's SAE.encode), compaction = torch's to_sparse_csr of those features
    (the reference's CPU dense->CSR), decode = torch.addmm(b_dec, f_csr, W_dec) in fp32, and
    the backward as dense fp32 autograd of the same forward on a quarter of the subset. The
    subset is sized so one encode takes about target_s/5 seconds; each figure is the median of
    3 runs after 1 warmup."""
    from saeflow_amd import workloads
    from oracle import reference as oref

    W = sae.W_enc.float().cpu()
    W_dec = sae.W_dec.float().cpu()
    b_enc, b_dec = sae.b_enc.float().cpu(), sae.b_dec.float().cpu()
    thr = None if sae.threshold is None else sae.threshold.float().cpu()
    T, d_in = x.shape
    d_sae = W.shape[1]
    xc = x[: min(T, 4096)].float().cpu()

    def enc(n):
        return oref.encode(xc[:n], W, b_enc, b_dec, thr, sae.activation, sae.k)

    t0 = time.perf_counter()
    enc(128)
    dt = time.perf_counter() - t0
    n = int(max(64, min(xc.shape[0], 128 * (target_s / 5) / max(dt, 1e-3))))
    sec = _median_time(lambda: enc(n))
    f = enc(n)
    warnings.filterwarnings("ignore", message="Sparse CSR tensor support is in beta")
    f_csr = f.to_sparse_csr()
    nnz = f_csr.values().numel()
    sec_c = _median_time(lambda: f.to_sparse_csr())
    sec_d = _median_time(lambda: torch.addmm(b_dec, f_csr, W_dec))
    flops = workloads.encode_flops(n, d_in, d_sae)
    comp_gbps = workloads.compaction_bytes(n, d_sae, nnz, 4) / sec_c / 1e9
    dec_gbps = workloads.decode_bytes(n, d_in, nnz, 4) / sec_d / 1e9

    # The backward on the CPU: dense fp32 torch autograd of the same forward and loss
    # (sum(x_hat * G), the MSE gradient's shape) on the first n_b tokens, with the active set
    # fixed by the sample's features.
    n_b = max(16, n // 4)
    active = f[:n_b] != 0
    G = torch.randn(n_b, d_in, generator=torch.Generator().manual_seed(0))
    leaves = [t.clone().requires_grad_(True) for t in (W, b_enc, W_dec, b_dec)]

    def bwd():
        We, be, Wd, bd = leaves
        for t in leaves:
            t.grad = None
        fb = ((xc[:n_b] - bd) @ We + be) * active
        ((fb @ Wd + bd) * G).sum().backward()

    sec_b = _median_time(bwd)
    del leaves, G, active
    return {"value": round(flops / sec / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{n} of the {T} tokens ({sae.activation} d_in={d_in} d_sae={d_sae}, fp32 on CPU): "
                      f"oracle.reference.encode {n / sec:.1f} tokens/s; median of 3 runs after 1 warmup",
            "tokens_per_s": round(n / sec, 1),
            "compact_gbps": round(comp_gbps, 2), "decode_requested_gbps": round(dec_gbps, 2),
            "backward_tokens_per_s": round(n_b / sec_b, 1),
            "backward_sample": f"{n_b} tokens, dense fp32 torch autograd (all four parameter gradients)",
            "nnz": nnz}


TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"
# kernel-name substrings (rocprofv3 Kernel_Name) -> stage; the copy kernel calibrates the counters
KERNEL_STAGE = {"xprep_kernel": "encode", "gemm_kernel": "encode", "gemm2_kernel": "encode",
                "gemm_persist_kernel": "encode",
                "compact_kernel": "compact", "compact_row_kernel": "compact", "decode_vec_kernel": "decode", "decode_lines_kernel": "decode", "decode_generic_kernel": "decode",
                "scan_tiles_kernel": "scan", "scan_totals_kernel": "scan", "scan_final_kernel": "scan",
                "rows_to_csr_wave_kernel": "rows_to_csr", "rows_to_csr_kernel": "rows_to_csr",
                "backward_units_kernel": "backward", "gpre_kernel": "backward", "csc_count_kernel": "backward",
                "csc_bucket_kernel": "backward", "csc_sort_kernel": "backward",
                "backward_reduce_kernel": "backward", "plan_tiles_kernel": "backward", "plan_totals_kernel": "backward",
                "plan_final_kernel": "backward", "item_table_kernel": "backward",
                "col_count_kernel": "backward", "col_place_kernel": "backward", "col_sort_kernel": "backward",
                "shift_vec_kernel": "backward", "transpose_kernel": "backward", "matvec_kernel": "backward",
                "col_sums_kernel": "backward", "col_sums_final_kernel": "backward", "enc_tile_kernel": "backward",
                "topk_vec_kernel": "topk", "topk_kernel": "topk", "topk_large_kernel": "topk",
                "rows_topk_kernel": "topk"}
COPY_KERNEL = "neg_kernel"
GRID_SEP = "@@grid="  # kernel name + launch grid: the key of one launch shape
# The persistent encode's grid is the CU count whatever the problem, so its launches at
# different problem sizes share a grid: they are told apart by their size (bytes or time).
PERSIST = "gemm_persist_kernel"


def group_tag(kernel, g):
    """Kernel name with size group g marked after its template arguments (before the argument list)."""
    i = kernel.find("(")
    return f"{kernel}#{g}" if i < 0 else f"{kernel[:i]}#{g}{kernel[i:]}"


def size_groups(values):
    """Indices of `values` grouped by magnitude: ascending, a new group wherever a value is
    more than twice the first value of the current group."""
    groups, first = [], None
    for i in sorted(range(len(values)), key=lambda i: values[i]):
        if first is None or values[i] > 2 * first:
            groups.append([])
            first = values[i]
        groups[-1].append(i)
    return groups


def kernel_stage(name):
    """Stage of a profiled kernel name; the 256x256 GEMM's fifth template argument (the
    persistent form's fourth, before its wave count) is its epilogue (0 dense, 1 / 2 row
    candidates)."""
    import re
    if re.search(r"gemm_kernel<\d+, \d+, \d+, \d+, [12](, (true|false))?>", name) or \
            re.search(r"gemm_persist_kernel<\d+, \d+, \d+, [12](, \d+)?>", name):
        return "encode_rows"
    return next((st for k, st in KERNEL_STAGE.items() if k in name), None)


def read_traffic(config, name):
    """HBM bytes per launch of stage `name` of configuration `config`, measured with
    rocprofv3 --pmc (profiles/traffic.json), if committed."""
    try:
        return json.loads(TRAFFIC_FILE.read_text()).get(config, {}).get(name)
    except (ValueError, OSError, AttributeError):
        return None


def copy_calibration(mib):
    """Launches a plain streaming kernel of known size (torch.neg over `mib` MiB of fp32:
    reads mib MiB, writes mib MiB) three times, so a --pmc pass over this process reads what
    FETCH_SIZE / WRITE_SIZE report for a known number of bytes."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def traffic_summary(pmc_dir, copy_mib, config):
    """Turns two rocprofv3 --pmc passes of `bench.py --config CONFIG --calibrate-copy MIB`
    (FETCH_SIZE under <pmc_dir>/fetch, WRITE_SIZE under <pmc_dir>/write, csv output) into HBM
    bytes per launch of each stage, scaled so the copy kernel reads and writes exactly its
    size; stores them under CONFIG in profiles/traffic.json and prints a markdown table."""
    import collections
    import csv
    import glob

    def per_kernel(sub, counter):
        files = glob.glob(os.path.join(pmc_dir, sub, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            raise SystemExit(f"no counter_collection.csv under {pmc_dir}/{sub}")
        disp = collections.defaultdict(float)
        names = {}
        wgs = {}
        for fn in files:
            for r in csv.DictReader(open(fn)):
                if r["Counter_Name"] != counter:
                    continue
                key = (fn, int(r["Dispatch_Id"]))
                disp[key] += float(r["Counter_Value"])
                names[key] = f"{r['Kernel_Name']}{GRID_SEP}{r['Grid_Size']}"  # one entry per launch shape
                wgs[key] = int(r["Workgroup_Size"])
        # persistent launches of one grid: one entry per size group, "#1" the smallest
        for name in {n for n in names.values() if PERSIST in n}:
            keys = [k for k, n in names.items() if n == name]
            groups = size_groups([disp[k] for k in keys])
            if len(groups) > 1:
                kernel, grid = name.split(GRID_SEP)
                for g, idx in enumerate(groups):
                    for i in idx:
                        names[keys[i]] = f"{group_tag(kernel, g + 1)}{GRID_SEP}{grid}"
        for key, n in names.items():
            wg_size[n] = wgs[key]
        agg = collections.defaultdict(list)
        for key, v in disp.items():
            agg[names[key]].append(v * 1024.0)  # KiB -> bytes
            last[names[key]] = max(last.get(names[key], -1), key[1])
        return agg

    last = {}  # kernel name -> its last dispatch id (in either pass)
    wg_size = {}  # kernel name -> its workgroup size
    fetch, write = per_kernel("fetch", "FETCH_SIZE"), per_kernel("write", "WRITE_SIZE")
    copy_bytes = copy_mib * (1 << 20)

    def calib(agg):
        vals = [v for k, vs in agg.items() if COPY_KERNEL in k for v in vs]
        if not vals:
            raise SystemExit(f"no {COPY_KERNEL} dispatch found: run bench.py with --calibrate-copy")
        return copy_bytes / statistics.median(vals)

    f_fetch, f_write = calib(fetch), calib(write)
    # The encode autotuner launches every candidate tiling once per shape before the timed
    # steps: a stage's bytes are those of the GEMM tiling that ran last (the one it kept), plus
    # its other kernels.
    # Entries are (kernel, grid size) pairs, so launches of one kernel at different shapes (C4:
    # the floor encode of the first S features and the dense encode of all of them) are never
    # averaged together. A stage's bytes are those of the (kernel, grid) of each role that ran
    # last; every other GEMM shape of the stage is reported under "<stage>@grid<G>".
    names = [n for n in set(fetch) | set(write) if kernel_stage(n) is not None]
    role = lambda n: (kernel_stage(n), "gemm" if "gemm" in n else n.split(GRID_SEP)[0])  # noqa: E731
    grid_of = lambda n: int(n.split(GRID_SEP)[1])  # noqa: E731

    from saeflow_amd.workloads import CONFIGS
    persist = sorted(n for n in names if PERSIST in n)  # size groups in ascending order
    pbytes = lambda m: statistics.mean(fetch.get(m, [0.0]) + write.get(m, [0.0]))  # noqa: E731

    def shape_of(n):
        # A GEMM launch's shape is the output elements it covers: workgroups x tile (gemm2_kernel
        # 256x128 tiles, gemm_kernel 256x256), so tilings of one problem compare equal whatever
        # their block size; the gathered (persistent) form is a shape of its own. The whole-tile
        # persistent kernel's grid says nothing of its outputs: its launches of a stage (the 8-
        # and 4-wave forms alike) are grouped by bytes (size_groups), the largest group being the
        # configuration's dense encode (T x d_sae outputs), smaller ones shapes of their own.
        # Other kernels: their grid.
        if "gemm" not in n:
            return ("grid", grid_of(n))
        if ", true>(" in n:
            return ("gathered",)
        if PERSIST in n:
            same = [m for m in persist if kernel_stage(m) == kernel_stage(n)]
            groups = size_groups([pbytes(m) for m in same])
            gi = next(i for i, g in enumerate(groups) if n in (same[j] for j in g))
            cfg = CONFIGS.get(config)
            return ("outputs", cfg["T"] * cfg["d_sae"]) if gi == len(groups) - 1 and cfg else ("persistent", gi)
        return ("outputs", grid_of(n) // max(wg_size.get(n, 1), 1) * (256 * 128 if "gemm2_kernel" in n else 256 * 256))

    def latest(group):
        best = {}
        for n in names:
            g = group(n)
            if g not in best or last[n] > last[best[g]]:
                best[g] = n
        return best
    kept = latest(lambda n: (role(n), shape_of(n)))  # the tiling each shape ran last
    main = latest(role)  # the shape each role ran last: the stage's bytes
    stages = collections.defaultdict(lambda: [0.0, 0.0])
    rows = []
    for name in sorted(names, key=lambda n: (kernel_stage(n), n)):
        stage = kernel_stage(name)
        fb = statistics.mean(fetch.get(name, [0.0])) * f_fetch
        wb = statistics.mean(write.get(name, [0.0])) * f_write
        k = kept[(role(name), shape_of(name))]
        if k == name:
            key = stage if main[role(name)] == name else f"{stage}@grid{grid_of(name)}"
            stages[key][0] += fb
            stages[key][1] += wb
            note = "kept" if key == stage else f"(other shape: `{key}`)"
        else:
            note = "(autotune candidate)"
        short = name.split(GRID_SEP)[0].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0][:60]
        rows.append(f"| {stage} | `{short}` | {grid_of(name)} | {note} | "
                    f"{len(fetch.get(name, []))} | {fb / 1e9:.4f} | {wb / 1e9:.4f} |")
    out = {s: int(round(fb + wb)) for s, (fb, wb) in stages.items()}
    out["_split"] = {s: {"fetch": int(round(fb)), "write": int(round(wb))} for s, (fb, wb) in stages.items()}
    out["_calibration"] = {"copy_kernel": COPY_KERNEL, "copy_bytes_each_way": copy_bytes,
                           "fetch_factor": round(f_fetch, 4), "write_factor": round(f_write, 4)}
    TRAFFIC_FILE.parent.mkdir(exist_ok=True)
    try:
        allcfg = json.loads(TRAFFIC_FILE.read_text())
    except (ValueError, OSError):
        allcfg = {}
    allcfg[config] = out
    TRAFFIC_FILE.write_text(json.dumps(allcfg, indent=1, sort_keys=True) + "\n")
    print(f"calibration: {COPY_KERNEL} over {copy_mib} MiB -> fetch factor {f_fetch:.4f}, write factor {f_write:.4f}")
    print("| stage | kernel | grid (work-items) | role | dispatches | FETCH GB/launch | WRITE GB/launch |")
    print("|---|---|---|---|---|---|---|")
    print("\n".join(rows))
    print(json.dumps(out))


MFMA_FILE = ROOT / "profiles" / "mfma.json"
MOPS_COUNTER = {torch.bfloat16: "SQ_INSTS_VALU_MFMA_MOPS_BF16", torch.float16: "SQ_INSTS_VALU_MFMA_MOPS_F16",
                torch.float32: "SQ_INSTS_VALU_MFMA_MOPS_F32"}


def _short_kernel(name):
    name = name.replace("(anonymous namespace)::", "").replace("void ", "")
    if name.startswith("Cijk_") or name.startswith("Custom_Cijk_"):
        return "hipBLASLt " + name.split("_UserArgs")[0][:60]
    return name.split("(")[0]


def _pmc_dispatches(pmc_dir):
    """{dispatch: {counter: value, 'ns': duration, 'name': kernel}} and the GPU agent's info
    from a rocprofv3 --pmc csv directory."""
    import collections
    import csv
    import glob

    files = glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True)
    agents = glob.glob(os.path.join(pmc_dir, "**", "*agent_info.csv"), recursive=True)
    if not files or not agents:
        raise SystemExit(f"no counter_collection.csv / agent_info.csv under {pmc_dir}")
    gpu = next(r for r in csv.DictReader(open(agents[0])) if r.get("Name", "").startswith("gfx"))
    disp = collections.defaultdict(dict)
    for fn in files:
        for r in csv.DictReader(open(fn)):
            key = (fn, int(r["Dispatch_Id"]))
            d = disp[key]
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            d["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            d["name"] = r["Kernel_Name"]
            d["grid"] = int(r.get("Grid_Size") or 0)
            d["id"] = key[1]
    return disp, gpu


def _by_shape(dispatches):
    """Dispatches grouped per (kernel, grid size), and a label per group: the kernel's short name,
    with its grid when the kernel ran at more than one shape. Persistent launches of one grid are
    split by duration (size groups "#1", "#2", ... from the shortest)."""
    import collections
    per = collections.defaultdict(list)
    for d in dispatches:
        per[(d["name"], d.get("grid", 0))].append(d)
    for (name, grid), ds in list(per.items()):
        groups = size_groups([d["ns"] for d in ds]) if PERSIST in name else [range(len(ds))]
        if len(groups) > 1:
            del per[(name, grid)]
            for g, idx in enumerate(groups):
                per[(group_tag(name, g + 1), grid)] = [ds[i] for i in idx]
    grids = collections.Counter(n for n, _ in per)
    label = {k: _short_kernel(k[0]) + (f" [grid {k[1]}]" if grids[k[0]] > 1 else "") for k in per}
    return per, label


def mfma_summary(pmc_dir, config):
    """Turns a rocprofv3 --pmc pass of SQ_VALU_MFMA_BUSY_CYCLES, the MFMA MOPS counter of the
    config's dtype (SQ_INSTS_VALU_MFMA_MOPS_BF16 / _F16 / _F32) and GRBM_GUI_ACTIVE over
    bench.py (csv output under pmc_dir) into, per GEMM kernel (the encode's and hipBLASLt's
    of the comparison leg): the MFMA flops the hardware counted (MOPS x 512) against the
    algorithmic 2*T*d_in*d_sae, the MFMA busy share (busy SIMD-cycles / (GPU cycles x SIMDs))
    and the average GPU clock while the kernel ran (GRBM_GUI_ACTIVE, summed over the XCDs, /
    XCDs / duration). Writes the kept encode kernel's record under CONFIG in profiles/mfma.json
    and prints a markdown table."""

    from saeflow_amd import workloads
    cfg = workloads.CONFIGS[config]
    mops = MOPS_COUNTER[cfg["dtype"]]
    disp, gpu = _pmc_dispatches(pmc_dir)
    n_xcc, n_simd = int(gpu["Num_Xcc"]), int(gpu["Simd_Count"])
    max_ghz = float(gpu["Max_Engine_Clk_Fcompute"]) / 1e3
    per, label = _by_shape(d for d in disp.values()
                           if ("gemm" in d["name"] or "Cijk" in d["name"])
                           and all(c in d for c in ("SQ_VALU_MFMA_BUSY_CYCLES", mops, "GRBM_GUI_ACTIVE")))
    last = {k: max(d["id"] for d in ds) for k, ds in per.items()}
    # the dominant GEMM: the dense encode (the autotuner's pick runs last), or for TopK
    # configs the floor-filtered row-candidate encode; one record per launch shape
    want = "encode_rows" if cfg["activation"] == "topk" else "encode"
    dense = [k for k in per if kernel_stage(k[0]) == want]
    kept = max(dense, key=lambda k: last[k])
    rows, out = [], {}
    for name in sorted(per, key=lambda k: ("Cijk" in k[0], k)):
        ds = per[name]
        ns = statistics.mean(d["ns"] for d in ds)
        cyc = statistics.mean(d["GRBM_GUI_ACTIVE"] for d in ds) / n_xcc
        busy = statistics.mean(d["SQ_VALU_MFMA_BUSY_CYCLES"] for d in ds) / (cyc * n_simd)
        flops = statistics.mean(d[mops] for d in ds) * 512
        ghz = cyc / ns
        rec = {"dispatches": len(ds), "avg_us": round(ns / 1e3, 1), "mfma_flops": flops,
               "mfma_busy": round(busy, 4), "clock_ghz": round(ghz, 3), "tflops": round(flops / ns / 1e3, 1)}
        short = label[name]
        if name == kept:
            out = {"kernel": short, "grid": name[1], **rec, "max_clock_ghz": max_ghz, "xcc": n_xcc, "simds": n_simd}
        tag = " (kept)" if name == kept else (" (row candidates)" if kernel_stage(name[0]) == "encode_rows" else "")
        rows.append(f"| `{short}`{tag} | {len(ds)} | {rec['avg_us']} | {flops:.4e} | "
                    f"{100 * busy:.1f}% | {ghz:.3f} | {rec['tflops']} |")
    MFMA_FILE.parent.mkdir(exist_ok=True)
    try:
        allcfg = json.loads(MFMA_FILE.read_text())
    except (ValueError, OSError):
        allcfg = {}
    allcfg[config] = out
    MFMA_FILE.write_text(json.dumps(allcfg, indent=1, sort_keys=True) + "\n")
    print(f"{n_xcc} XCDs, {n_simd} SIMDs, max engine clock {max_ghz} GHz; flops from {mops} x 512")
    print("| kernel | dispatches | avg us | MFMA flops (MOPS x 512) | MFMA busy | clock GHz | TFLOP/s |")
    print("|---|---|---|---|---|---|---|")
    print("\n".join(rows))
    print(json.dumps(out))


SQ_COUNTERS = ("SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_INSTS_LDS",
               "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_VMEM", "GRBM_GUI_ACTIVE")


def sq_summary(pmc_dir):
    """Turns a rocprofv3 --pmc pass of SQ_COUNTERS over bench.py into a per-kernel table of the
    GEMMs (the encode's tilings and hipBLASLt's), the compaction and the decode: the share of
    wave-cycles spent waiting at s_waitcnt / barriers (SQ_WAIT_ANY) and waiting to issue
    (SQ_WAIT_INST_ANY), LDS and VMEM instructions per launch and LDS bank-conflict cycles."""

    disp, gpu = _pmc_dispatches(pmc_dir)
    keep = ("gemm", "Cijk", "compact_row", "decode_lines", "decode_vec")
    per, label = _by_shape(d for d in disp.values()
                           if any(k in d["name"] for k in keep) and all(c in d for c in SQ_COUNTERS))
    print("| kernel | dispatches | avg us | waves waiting (SQ_WAIT_ANY / SQ_WAVE_CYCLES) | waiting to issue "
          "(SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES) | LDS insts | LDS bank-conflict cycles | VMEM insts |")
    print("|---|---|---|---|---|---|---|---|")
    for name in sorted(per, key=lambda k: ("Cijk" in k[0], k)):
        ds = per[name]
        m = {c: statistics.mean(d[c] for d in ds) for c in SQ_COUNTERS}
        ns = statistics.mean(d["ns"] for d in ds)
        print(f"| `{label[name]}` | {len(ds)} | {ns / 1e3:.1f} | "
              f"{100 * m['SQ_WAIT_ANY'] / m['SQ_WAVE_CYCLES']:.1f}% | "
              f"{100 * m['SQ_WAIT_INST_ANY'] / m['SQ_WAVE_CYCLES']:.1f}% | {m['SQ_INSTS_LDS']:.3g} | "
              f"{m['SQ_LDS_BANK_CONFLICT']:.3g} | {m['SQ_INSTS_VMEM']:.3g} |")


LDS_COUNTERS = ("SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_DATA_FIFO_FULL", "SQ_LDS_CMD_FIFO_FULL",
                "SQ_INSTS_LDS_LOAD_BANDWIDTH", "SQ_INSTS_LDS_STORE_BANDWIDTH", "GRBM_GUI_ACTIVE")


def lds_summary(pmc_dir):
    """Turns a rocprofv3 --pmc pass of LDS_COUNTERS over bench.py into a per-kernel table of
    the GEMMs, the compaction and the decode: cycles the LDS works on indexed (ds_*) operations
    per CU-cycle, bytes read and written by ds_* instructions per CU per clock, cycles the LDS
    data / command queues are full, and bank-conflict cycles per active cycle. LDS DMA writes
    (buffer_load ... lds) are not indexed operations and appear in none of these."""

    disp, gpu = _pmc_dispatches(pmc_dir)
    n_xcc, cus = int(gpu["Num_Xcc"]), int(gpu["Cu_Count"])
    keep = ("gemm", "Cijk", "compact_row", "decode_lines", "decode_vec")
    per, label = _by_shape(d for d in disp.values()
                           if any(k in d["name"] for k in keep) and all(c in d for c in LDS_COUNTERS))
    print("| kernel | dispatches | avg us | LDS busy (SQ_LDS_IDX_ACTIVE / CU-cycles) | ds_* read B/clk/CU | "
          "ds_* write B/clk/CU | data queue full | command queue full | bank-conflict cycles / busy |")
    print("|---|---|---|---|---|---|---|---|---|")
    for name in sorted(per, key=lambda k: ("Cijk" in k[0], k)):
        ds = per[name]
        m = {c: statistics.mean(d[c] for d in ds) for c in LDS_COUNTERS}
        ns = statistics.mean(d["ns"] for d in ds)
        cc = m["GRBM_GUI_ACTIVE"] / n_xcc * cus  # CU-cycles of the dispatch
        print(f"| `{label[name]}` | {len(ds)} | {ns / 1e3:.1f} | {100 * m['SQ_LDS_IDX_ACTIVE'] / cc:.1f}% | "
              f"{64 * m['SQ_INSTS_LDS_LOAD_BANDWIDTH'] / cc:.1f} | {64 * m['SQ_INSTS_LDS_STORE_BANDWIDTH'] / cc:.1f} | "
              f"{100 * m['SQ_LDS_DATA_FIFO_FULL'] / cc:.1f}% | {100 * m['SQ_LDS_CMD_FIFO_FULL'] / cc:.1f}% | "
              f"{100 * m['SQ_LDS_BANK_CONFLICT'] / max(1.0, m['SQ_LDS_IDX_ACTIVE']):.1f}% |")


MIX_PASSES = {
    "p1": "SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_INSTS_VALU SQ_INSTS_SALU GRBM_GUI_ACTIVE",
    "p2": "SQ_INSTS_VMEM SQ_INSTS_LDS SQ_INSTS_SMEM SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_WAIT_INST_LDS "
          "SQ_ACTIVE_INST_VALU GRBM_GUI_ACTIVE",
    "p3": "SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_SCA SQ_ACTIVE_INST_MISC SQ_INST_CYCLES_VMEM_RD "
          "SQ_LDS_BANK_CONFLICT SQ_INSTS_BRANCH GRBM_GUI_ACTIVE",
}


def gemms_only(config):
    """The encode GEMM of `config` alone, for counter passes: the fused encode with the kept
    8-wave 256x256 tiling on the feature-contiguous W_enc and on the same values d_in-contiguous,
    then hipBLASLt's plain GEMM (torch.mm) of the shape in both layouts; five launches each."""
    from saeflow_amd import workloads
    from saeflow_amd.kernels import fused_encode
    sae, x, meta = workloads.make(config, device="cuda")
    T, d_in, d_sae, dtype = meta["T"], meta["d_in"], meta["d_sae"], meta["dtype"]
    if sae.activation == "topk":
        raise SystemExit("--gemms-only runs the relu / jumprelu encode")
    Wk = sae.W_enc.t().contiguous().t()
    bk = 32 if dtype == torch.float32 else 64
    cfg = {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": bk, "GROUP_M": 1, "NUM_WAVES": 8, "GROUP_N": 8}
    row_nnz = torch.zeros(T, device="cuda", dtype=torch.int32)
    for W in (sae.W_enc, Wk):
        for _ in range(5):
            fused_encode(x, W, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz, config=cfg)
    out = torch.empty(T, d_sae, device="cuda", dtype=dtype)
    for b in (sae.W_enc, Wk):
        for _ in range(5):
            torch.mm(x, b, out=out)
    torch.cuda.synchronize()
    print(f"{config}: 4 GEMMs x 5 launches done")


def mix_summary(pmc_dir):
    """Turns three rocprofv3 --pmc passes (MIX_PASSES, under <pmc_dir>/p1..p3) of
    `bench.py --gemms-only` into the instruction mix of each GEMM per 32x32x16-equivalent
    MFMA (32768 flops: hipBLASLt's 16x16x32 MFMAs count half): MFMA busy share, waves waiting
    (s_waitcnt / barrier) and waiting to issue, LDS / VALU / SALU / VMEM / SMEM / branch
    instructions and LDS wait cycles per MFMA, and LDS bank-conflict cycles per LDS
    instruction. Medians over each kernel's dispatches."""
    import collections
    rows = collections.defaultdict(lambda: collections.defaultdict(list))
    n_xcc = 8
    for sub in ("p1", "p2", "p3"):
        disp, gpu = _pmc_dispatches(os.path.join(pmc_dir, sub))
        n_xcc = int(gpu["Num_Xcc"])
        n_simd = int(gpu["Simd_Count"])
        for d in disp.values():
            if "gemm" in d["name"] or "Cijk" in d["name"]:
                for c, v in d.items():
                    if c not in ("name", "id"):
                        rows[(d["name"], d.get("grid", 0))][c].append(v)
    print("| kernel | us | MFMA busy | waves waiting | waiting to issue | MFMA insts (32x32x16 eq.) | LDS / MFMA | "
          "VALU / MFMA | SALU / MFMA | VMEM / MFMA | SMEM / MFMA | branch / MFMA | LDS wait cycles / MFMA | "
          "LDS bank-conflict cycles / LDS inst | waves |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|")
    for key in sorted(rows, key=lambda k: ("Cijk" in k[0], k)):
        m = {c: statistics.median(v) for c, v in rows[key].items()}
        need = ("SQ_INSTS_MFMA", "SQ_WAVE_CYCLES", "SQ_INSTS_LDS", "SQ_INSTS_BRANCH", "GRBM_GUI_ACTIVE")
        if not all(c in m for c in need):
            continue
        mfma = m["SQ_INSTS_MFMA"] * (0.5 if "Cijk" in key[0] else 1.0)  # hipBLASLt: 16x16x32 MFMAs
        cyc = m["GRBM_GUI_ACTIVE"] / n_xcc
        busy = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * n_simd)
        wc = m["SQ_WAVE_CYCLES"]
        print(f"| `{_short_kernel(key[0])[:70]}` | {m['ns'] / 1e3:.0f} | {100 * busy:.1f}% | "
              f"{100 * m['SQ_WAIT_ANY'] / wc:.1f}% | {100 * m['SQ_WAIT_INST_ANY'] / wc:.1f}% | {mfma:.3g} | "
              f"{m['SQ_INSTS_LDS'] / mfma:.3f} | {m['SQ_INSTS_VALU'] / mfma:.3f} | {m['SQ_INSTS_SALU'] / mfma:.3f} | "
              f"{m['SQ_INSTS_VMEM'] / mfma:.3f} | {m['SQ_INSTS_SMEM'] / mfma:.4f} | {m['SQ_INSTS_BRANCH'] / mfma:.4f} | "
              f"{m['SQ_WAIT_INST_LDS'] / mfma:.2f} | {m['SQ_LDS_BANK_CONFLICT'] / m['SQ_INSTS_LDS']:.3f} | "
              f"{m['SQ_WAVES']:.0f} |")


def stats_summary(kt_dir, top=24):
    """Turns the kernel_trace.csv of a rocprofv3 --kernel-trace --stats run into a markdown
    table of the launches by total time, one row per kernel and grid size (a kernel launched
    at several shapes gets one row per shape, never one average over them): calls, average /
    min / max microseconds, share of the GPU time."""
    import collections
    import csv
    import glob

    files = glob.glob(os.path.join(kt_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_trace.csv under {kt_dir}")
    groups = collections.defaultdict(list)
    for r in csv.DictReader(open(files[0])):
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        groups[(r["Kernel_Name"], grid)].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    # persistent launches of one grid: one row per size group ("#1" the shortest)
    for (name, grid), ns in list(groups.items()):
        sg = size_groups(ns) if PERSIST in name else []
        if len(sg) > 1:
            del groups[(name, grid)]
            for g, idx in enumerate(sg):
                groups[(group_tag(name, g + 1), grid)] = [ns[i] for i in idx]
    total = sum(sum(v) for v in groups.values()) or 1
    print("| kernel | grid (work-items) | calls | avg us | min us | max us | % of GPU time |")
    print("|---|---|---|---|---|---|---|")
    for (name, grid), ns in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]:
        print(f"| `{_short_kernel(name)[:90]}` | {grid} | {len(ns)} | {statistics.mean(ns) / 1e3:.1f} | "
              f"{min(ns) / 1e3:.1f} | {max(ns) / 1e3:.1f} | {100 * sum(ns) / total:.2f} |")


def read_mfma(config):
    """MFMA busy share and clock of the kept encode GEMM of `config` from a committed --pmc summary."""
    try:
        return json.loads(MFMA_FILE.read_text()).get(config)
    except (ValueError, OSError, AttributeError):
        return None


def cache_leg(sae, d_in, dtype, n_seqs=2048, seq_len=256, batch=32, per_shard=8):
    """The activation-cache caller (saeflow_amd/cache.py) on the bench's SAE: a one-layer
    stand-in model emits [batch, seq, d_in] activations at one hook (b_dec + N(0, 1)-like rows,
    as the synthetic x), cache_activations encodes them on the fly (encode_sparse), copies the
    CSR to pinned host memory on its side stream and writes each shard (fsync + rename) from
    its writer thread. Timed end to end after an identical warm-up call (steady state: the
    pinned host buffers are allocated by then), against the model forward + encode_sparse
    alone over the same batches."""
    import shutil
    import tempfile

    import saeflow_amd
    from saeflow_amd.cache import cache_activations

    hook = "blocks.0.hook_resid_post"

    class Standin:
        def __init__(self):
            g = torch.Generator(device="cuda").manual_seed(3)
            self.embed = torch.randn(1024, d_in, device="cuda", generator=g).to(dtype)
            self.w = (torch.randn(d_in, d_in, device="cuda", generator=g) / d_in ** 0.5).to(dtype)

        def parameters(self):
            return iter([self.embed])

        def run_with_cache(self, tokens, names_filter=None, stop_at_layer=None, return_type="logits"):
            act = sae.b_dec + self.embed[tokens] @ self.w
            return None, {hook: act}

    model = Standin()
    tokens = torch.randint(0, 1024, (n_seqs, seq_len), generator=torch.Generator().manual_seed(4))
    root = Path(tempfile.mkdtemp(prefix="saeflow_cache_bench_"))
    try:
        kw = dict(batch_size=batch, batches_per_shard=per_shard, dtype=dtype, encoders={hook: sae})
        cache_activations(model, tokens, [hook], root / "warm", **kw)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cache_activations(model, tokens, [hook], root / "run", **kw)
        cached_s = time.perf_counter() - t0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pinned = tokens.pin_memory()  # the batches go up as cache_activations uploads them
        for b0 in range(0, n_seqs, batch):
            _, acts = model.run_with_cache(pinned[b0:b0 + batch].cuda(non_blocking=True), names_filter=[hook])
            saeflow_amd.encode_sparse(sae, acts[hook].reshape(-1, d_in))
        torch.cuda.synchronize()
        compute_s = time.perf_counter() - t0
    finally:
        shutil.rmtree(root, ignore_errors=True)
    rows = n_seqs * seq_len
    return {"tokens_per_s": round(rows / cached_s, 1), "compute_only_tokens_per_s": round(rows / compute_s, 1),
            "hidden_frac": round(compute_s / cached_s, 4),
            "sample": f"{n_seqs} x {seq_len} tokens, batches of {batch} sequences, {per_shard} batches a shard",
            "what": "cache_activations with the SAE encoding one hook on the fly (CSR shards written and "
                    "fsynced), against the stand-in model forward + encode_sparse alone"}


FLUSH_BYTES = 1 << 30  # written before each flushed launch: 4x the 256 MB MALL


def _ev():
    return torch.cuda.Event(enable_timing=True)


def flushed_ms(fn, flush, reps):
    """Median duration of single launches of fn with cold caches: a 1 GiB buffer is written
    before each launch (the reference's do_bench clears the L2 the same way,
    bench/common.py:91-96) and HIP events on the launch stream bracket the launch alone."""
    stream = torch.cuda.current_stream()
    fn()
    pairs = []
    for _ in range(reps):
        flush.zero_()
        a, b = _ev(), _ev()
        a.record(stream)
        fn()
        b.record(stream)
        pairs.append((a, b))
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in pairs)


def back_to_back_ms(fn, reps):
    """Average duration of fn over `reps` launches queued back to back after one warm-up."""
    stream = torch.cuda.current_stream()
    fn()
    a, b = _ev(), _ev()
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def decode_roofline(config, indices, T, d_in, nnz, esize, ms):
    """The decode kernel against HBM: `achieved` is the counter-measured HBM bytes per launch
    (profiles/traffic.json) over the flushed launch time, so frac <= 1; beside it the
    requested bytes (the reference's formula, bench/bench_decode.py:57, which counts a
    W_dec row once per use) and the compulsory floor (each distinct W_dec row once, the CSR,
    x_hat), each as a rate over the same time. The line-slab kernel serves most gathers from
    L2 (each XCD holds one 128-B column slab of W_dec at a time), so its measured bytes sit
    well under the requested ones: `traffic_over_floor` is how far they are from the floor,
    `floor_ms_at_peak` the time the floor alone takes at the HBM peak."""
    from saeflow_amd import workloads
    requested = workloads.decode_bytes(T, d_in, nnz, esize)
    uniq = int(torch.unique(indices).numel())
    floor = uniq * d_in * esize + nnz * (4 + esize) + T * d_in * esize + (T + 1) * 8
    traffic = read_traffic(config, "decode")
    basis = traffic if traffic else requested
    rate = basis / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(rate, 1), "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": round(rate / PEAK_GBPS, 4), "traffic": traffic,
            "achieved_from": "measured HBM bytes" if traffic else "requested bytes (no counter profile)",
            "kernel_ms": round(ms, 4), "requested_bytes": requested,
            "requested_gbps": round(requested / (ms * 1e-3) / 1e9, 1),
            "requested_frac": round(requested / (ms * 1e-3) / 1e9 / PEAK_GBPS, 4),
            "floor_bytes": floor, "unique_rows": uniq,
            "floor_gbps": round(floor / (ms * 1e-3) / 1e9, 1),
            "traffic_over_floor": round(traffic / floor, 2) if traffic else None,
            "floor_ms_at_peak": round(floor / (PEAK_GBPS * 1e9) * 1e3, 4),
            "timing": "median of single launches, 1 GiB written before each"}


def blas_reference(T, d_in, d_sae, dtype, reps=10):
    """The library GEMM of the encode's shape for scale (torch.mm -> hipBLASLt): no bias,
    activation, counting or prologue. Both layouts of W: feature-contiguous [d_in, d_sae] (the
    SAE layout) and K-contiguous [d_sae, d_in] transposed. Median of single launches."""
    g = torch.Generator(device="cuda").manual_seed(0)
    a = torch.randn(T, d_in, device="cuda", generator=g).to(dtype)
    w = (torch.randn(d_in, d_sae, device="cuda", generator=g) / d_in ** 0.5).to(dtype)
    wt = w.t().contiguous()
    out = torch.empty(T, d_sae, device="cuda", dtype=dtype)
    flops = 2 * T * d_in * d_sae
    res = {}
    for name, b in (("feature_contiguous", w), ("k_contiguous", wt.t())):
        for _ in range(3):
            torch.mm(a, b, out=out)
        torch.cuda.synchronize()
        pairs = []
        for _ in range(reps):
            e0, e1 = _ev(), _ev()
            e0.record()
            torch.mm(a, b, out=out)
            e1.record()
            pairs.append((e0, e1))
        torch.cuda.synchronize()
        ms = statistics.median(x.elapsed_time(y) for x, y in pairs)
        res[name] = {"ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
    del a, w, wt, out
    res["what"] = "torch.mm (hipBLASLt) of x [T, d_in] and W in both layouts: the plain GEMM, for scale"
    return res


def _torch_encode(sae, x):
    """The reference SAE's encode in plain torch ops on the GPU (reference.py:36-46): the
    library baseline the reference's bench times beside its kernels (bench_encode.py:66-70)."""
    pre = (x - sae.b_dec) @ sae.W_enc + sae.b_enc
    if sae.activation == "relu":
        return torch.relu(pre)
    if sae.activation == "jumprelu":
        return torch.relu(pre) * (pre > sae.threshold)
    top = pre.topk(sae.k, dim=-1)
    return torch.zeros_like(pre).scatter_(-1, top.indices, torch.relu(top.values))


def torch_reference(sae, x, meta, csr, flush, reps=5):
    """Same-box library baselines, for scale, as the reference's own bench times them: torch
    sae.encode and sae(x) (bench_encode.py:66-96; forward in the reference's effective FLOPs,
    4 * T * d_in * d_sae), the dense sae.decode, and the dense -> CSR conversion
    f.to_sparse_csr() (bench_decode.py:78-93). The CSR addmm baseline (bench_decode.py:61-64)
    is not run (see below). Each a median
    of single launches with 1 GiB written before each, beside this library's op on the same
    inputs; a torch op that ROCm does not support for the dtype is reported as skipped."""
    import saeflow_amd
    from saeflow_amd import workloads
    from saeflow_amd.kernels import dense_to_csr, sparse_decode

    T, d_in, d_sae, dtype = meta["T"], meta["d_in"], meta["d_sae"], meta["dtype"]
    esize = torch.finfo(dtype).bits // 8
    indptr, indices, values = csr
    nnz = indices.numel()
    res = {}

    def timed(fn):
        try:
            return round(flushed_ms(fn, flush, reps), 4)
        except (RuntimeError, NotImplementedError) as err:
            return f"skipped: {str(err).splitlines()[0][:120]}"

    def entry(torch_ms, ours_ms, work, unit):
        e = {"torch_ms": torch_ms, "saeflow_amd_ms": ours_ms}
        for k, ms in (("torch", torch_ms), ("saeflow_amd", ours_ms)):
            if isinstance(ms, float):
                e[f"{k}_{unit}"] = round(work / (ms * 1e-3) / (1e12 if unit == "tflops" else 1e9), 1)
        return e

    enc_flops = workloads.encode_flops(T, d_in, d_sae)
    res["encode"] = entry(timed(lambda: _torch_encode(sae, x)), timed(lambda: saeflow_amd.encode(sae, x)),
                          enc_flops, "tflops")
    res["forward"] = entry(timed(lambda: _torch_encode(sae, x) @ sae.W_dec + sae.b_dec),
                           timed(lambda: saeflow_amd.forward(sae, x)), 2 * enc_flops, "tflops")
    res["forward"]["flops"] = "effective: 4 * T * d_in * d_sae (bench_encode.py:89)"
    dec_bytes = workloads.decode_bytes(T, d_in, nnz, esize)
    f = torch.zeros(T, d_sae, device="cuda", dtype=dtype)
    f[torch.repeat_interleave(torch.arange(T, device="cuda"), torch.diff(indptr)), indices.long()] = values
    ours_dec = timed(lambda: sparse_decode(indptr, indices, values, sae.W_dec, sae.b_dec))
    res["decode_dense"] = entry(timed(lambda: f @ sae.W_dec + sae.b_dec), ours_dec, dec_bytes, "gbps")
    res["decode_dense"]["bytes"] = "requested: the reference's formula (bench_decode.py:57)"
    # torch.addmm(bias, csr_tensor, W_dec) (bench_decode.py:61-64) is not called: with bf16
    # values it ended the process on this ROCm build (an exception thrown through the sparse
    # library, "terminate called after throwing an instance of 'char const*'"), which no
    # Python handler can catch, so no dtype of it is risked here
    res["decode_csr"] = "not run: torch's CSR addmm aborted the process on ROCm with bf16 values"
    comp_bytes = workloads.compaction_bytes(T, d_sae, nnz, esize)
    res["to_csr"] = entry(timed(lambda: f.to_sparse_csr()), timed(lambda: dense_to_csr(f)), comp_bytes, "gbps")
    res["to_csr"]["what"] = "dense -> CSR with the counts computed (dense_to_csr(f) without row_nnz, one host read each)"
    del f
    res["what"] = "torch ops of the reference's own bench on this GPU, for scale"
    return res


def bench_path(args, sae, x, meta, flush):
    """relu / jumprelu configs: zero row_nnz + fused encode with counting, scan + the host
    read of nnz, compaction, decode, timed per step with events around each stage; then the
    kernels alone (flushed), the row-candidate path, the backward and a training step."""
    import saeflow_amd
    from saeflow_amd import workloads
    from saeflow_amd.kernels import (best_config, compact, encode_rows, exclusive_scan, fused_encode, rows_to_csr,
                                     sparse_backward, sparse_decode)
    from saeflow_amd.ops import ROW_CAP

    T, d_in, d_sae, dtype = meta["T"], meta["d_in"], meta["d_sae"], meta["dtype"]
    esize = torch.finfo(dtype).bits // 8
    stream = torch.cuda.current_stream()

    def step(rec):
        e = [_ev() for _ in range(6)]
        e[0].record(stream)
        row_nnz = torch.zeros(T, device="cuda", dtype=torch.int32)
        e[1].record(stream)
        f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz)
        e[2].record(stream)
        indptr = exclusive_scan(row_nnz)
        nnz = int(indptr[-1])  # the one host sync (decode.py:88)
        e[3].record(stream)
        indices, values = compact(f, indptr, nnz)
        e[4].record(stream)
        out = sparse_decode(indptr, indices, values, sae.W_dec, sae.b_dec)
        e[5].record(stream)
        if rec is not None:
            rec.append((e, nnz))
        return f, indptr, indices, values, out

    for _ in range(args.warmup):
        step(None)
    torch.cuda.synchronize()
    recs = []
    t_start, t_end = _ev(), _ev()
    t_start.record(stream)
    for _ in range(args.steps):
        last = step(recs)
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    enc_tiling = best_config()  # the autotuner's pick for this shape (timed during warmup)

    # Kernel-only launch durations with cold caches: the compaction follows the step's host
    # sync, so its stage time above also holds the launch gap.
    f_l, indptr_l, indices_l, values_l, _ = last
    nnz_l = indices_l.numel()
    reps = max(5, args.steps)
    comp_kernel_ms = flushed_ms(lambda: compact(f_l, indptr_l, nnz_l), flush, reps)
    dec_kernel_ms = flushed_ms(lambda: sparse_decode(indptr_l, indices_l, values_l, sae.W_dec, sae.b_dec), flush,
                               reps)
    dec_b2b_ms = back_to_back_ms(lambda: sparse_decode(indptr_l, indices_l, values_l, sae.W_dec, sae.b_dec), reps)
    del last, f_l
    torch_ref = None if args.no_blas else torch_reference(sae, x, meta, (indptr_l, indices_l, values_l), flush)

    # The row-candidate path of encode_sparse (no dense features): the fused encode appends each
    # row's nonzeros to a per-row list, the scan + host read, lists -> CSR, then decode. Same
    # CSR as the dense path.
    def encode_rows_call():
        return encode_rows(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, cap=ROW_CAP)

    def rows_step():
        cnt, idx, val = encode_rows_call()
        indptr = exclusive_scan(cnt)
        n = int(indptr[-1])
        ind, vals = rows_to_csr(cnt, idx, val, indptr, n)
        return sparse_decode(indptr, ind, vals, sae.W_dec, sae.b_dec), n

    _, rows_nnz = rows_step()
    assert rows_nnz == nnz_l, "row-candidate path found a different nnz"
    rows_enc_ms = back_to_back_ms(encode_rows_call, reps=max(3, args.steps // 2))
    rows_step_ms = back_to_back_ms(rows_step, reps=max(3, args.steps // 2))

    # The backward of the path (training): gradients of every parameter from dL/dx_hat on the
    # same CSR, without an input gradient (the common SAE-training case).
    bwd_ms = train_ms = None
    if not args.no_backward:
        g_xhat = torch.randn(T, d_in, device="cuda", dtype=dtype)
        csr_b = (indptr_l, indices_l, values_l)
        bwd_ms = back_to_back_ms(lambda: sparse_backward(x, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, csr_b,
                                                         g_xhat, need_grad_x=False), reps=max(3, args.steps // 2))
        del g_xhat, csr_b

        # One SAE training step through the sparse path, without the optimizer: encode_sparse
        # (row-candidate encode), decode, dL/dx_hat of the mean squared reconstruction error,
        # and every parameter's gradient.
        def train_step():
            csr = saeflow_amd.encode_sparse(sae, x)
            x_hat = saeflow_amd.decode_sparse(sae, csr)
            g = (x_hat - x) * (2.0 / T)
            return sparse_backward(x, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, csr, g, need_grad_x=False)

        train_ms = back_to_back_ms(train_step, reps=max(3, args.steps // 2))

    def stage(i, j):
        return [e[i].elapsed_time(e[j]) for e, _ in recs]

    enc_ms, scan_ms, comp_ms, dec_ms = stage(1, 2), stage(2, 3), stage(3, 4), stage(4, 5)
    nnz = recs[-1][1]
    assert all(n == nnz for _, n in recs), "nnz changed between identical steps"
    K = args.steps
    enc_flops = workloads.encode_flops(T, d_in, d_sae)
    comp_bytes = workloads.compaction_bytes(T, d_sae, nnz, esize)
    dec_bytes = workloads.decode_bytes(T, d_in, nnz, esize)
    enc_avg, comp_avg, dec_avg = sum(enc_ms) / K, sum(comp_ms) / K, sum(dec_ms) / K
    enc_tf = enc_flops / (enc_avg * 1e-3) / 1e12
    comp_gbps = comp_bytes / (comp_avg * 1e-3) / 1e9
    dec_gbps = dec_bytes / (dec_avg * 1e-3) / 1e9
    comp_k_gbps = comp_bytes / (comp_kernel_ms * 1e-3) / 1e9
    peak_tf = PEAK_TFLOPS[dtype]
    bwd_bytes = workloads.backward_bytes(T, d_in, d_sae, nnz, esize)

    return {
        "value": round(enc_tf, 2),
        "ms_per_step": round(total_ms / K, 4),
        "l0_measured": round(nnz / T, 2),
        "decode_requested_gbps": round(dec_gbps, 1),
        "tokens_per_s": round(T / (total_ms / K * 1e-3), 1),
        "stages": {
            "encode": {"ms": round(enc_avg, 4), "tflops": round(enc_tf, 2), "frac": round(enc_tf / peak_tf, 4),
                       "ms_min": round(min(enc_ms), 4), "tiling": enc_tiling},
            "scan_and_sync": {"ms": round(sum(scan_ms) / K, 4)},
            "compact": {"ms": round(comp_avg, 4), "gbps": round(comp_gbps, 1),
                        "frac": round(comp_gbps / PEAK_GBPS, 4), "bytes": comp_bytes,
                        "kernel_ms": round(comp_kernel_ms, 4)},
            "decode": {"ms": round(dec_avg, 4), "requested_gbps": round(dec_gbps, 1), "requested_bytes": dec_bytes,
                       "nnz": nnz,
                       "kernel_ms": round(dec_kernel_ms, 4), "kernel_ms_back_to_back": round(dec_b2b_ms, 4)},
            "encode_rows": {"ms": round(rows_enc_ms, 4),
                            "tflops": round(enc_flops / (rows_enc_ms * 1e-3) / 1e12, 2),
                            "frac": round(enc_flops / (rows_enc_ms * 1e-3) / 1e12 / peak_tf, 4)},
        },
        "path_rows": {"ms_per_step": round(rows_step_ms, 4), "tokens_per_s": round(T / (rows_step_ms * 1e-3), 1),
                      "stages": "encode_rows + scan + nnz read + rows_to_csr + decode"},
        "backward": None if bwd_ms is None else {
            "ms": round(bwd_ms, 4), "bytes": bwd_bytes, "gbps": round(bwd_bytes / (bwd_ms * 1e-3) / 1e9, 1),
            "frac": round(bwd_bytes / (bwd_ms * 1e-3) / 1e9 / PEAK_GBPS, 4),
            "traffic": read_traffic(args.config, "backward"),
            "what": "sparse_backward: dW_enc, db_enc, dW_dec, db_dec from dL/dx_hat on the step's CSR (no dx)"},
        "train_step": None if train_ms is None else {
            "ms": round(train_ms, 4), "tokens_per_s": round(T / (train_ms * 1e-3), 1),
            "what": "encode_sparse + decode_sparse + MSE gradient + sparse_backward (no optimizer)"},
        "roofline": {"bound": "mfma", "achieved": round(enc_tf, 2), "peak": peak_tf, "unit": "TFLOP/s",
                     "frac": round(enc_tf / peak_tf, 4), "traffic": read_traffic(args.config, "encode")},
        "roofline_decode": decode_roofline(args.config, indices_l, T, d_in, nnz, esize, dec_kernel_ms),
        "torch_reference": torch_ref,
        "roofline_compact": {"bound": "hbm", "achieved": round(comp_k_gbps, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                             "frac": round(comp_k_gbps / PEAK_GBPS, 4), "traffic": read_traffic(args.config, "compact"),
                             "kernel_ms": round(comp_kernel_ms, 4),
                             "timing": "median of single launches, 1 GiB written before each"},
    }


def bench_topk(args, sae, x, meta, flush):
    """TopK configs: the TopK encode of ops._topk (on wide dictionaries: a dense encode of the
    first S features and its top-k as a floor, the floor-filtered row-candidate encode, the
    list select and the device-side redo of overflowed rows, with no host read) and the
    decode of the fixed-width rows (indptr = arange(0, M*k+1, k), ops.py:35-36; no
    compaction exists)."""
    from saeflow_amd import ops, workloads
    from saeflow_amd.kernels import encode_rows, fused_encode, sparse_decode, topk_rows

    T, d_in, d_sae, dtype, k = meta["T"], meta["d_in"], meta["d_sae"], meta["dtype"], meta["k"]
    esize = torch.finfo(dtype).bits // 8
    stream = torch.cuda.current_stream()
    indptr = torch.arange(0, T * k + 1, k, device="cuda", dtype=torch.int64)

    def step(rec):
        e = [_ev() for _ in range(3)]
        e[0].record(stream)
        values, indices = ops._topk(sae, x)
        e[1].record(stream)
        out = sparse_decode(indptr, indices.view(-1), values.view(-1), sae.W_dec, sae.b_dec)
        e[2].record(stream)
        if rec is not None:
            rec.append(e)
        return values, indices, out

    for _ in range(args.warmup):
        step(None)
    torch.cuda.synchronize()
    recs = []
    t_start, t_end = _ev(), _ev()
    t_start.record(stream)
    for _ in range(args.steps):
        last = step(recs)
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    values_l, indices_l, _ = last
    K = args.steps
    enc_avg = sum(e[0].elapsed_time(e[1]) for e in recs) / K
    dec_avg = sum(e[1].elapsed_time(e[2]) for e in recs) / K
    nnz = T * k
    reps = max(5, args.steps)
    dec_kernel_ms = flushed_ms(lambda: sparse_decode(indptr, indices_l.view(-1), values_l.view(-1), sae.W_dec,
                                                     sae.b_dec), flush, reps)

    # the pieces of the TopK encode, each alone (back to back): the floor's dense encode of the
    # first S features, its select, the floor-filtered GEMM into row lists, the list select;
    # and the dense alternative (fused_encode + topk_rows over all features)
    S = ops._floor_slice(d_sae, k)
    W_sub, be_sub = sae.W_enc[:, :S], sae.b_enc[:S]
    f_sub = fused_encode(x, W_sub, be_sub, sae.b_dec, activation="relu")
    floor = topk_rows(f_sub, k)[0][:, k - 1].float()
    pieces = {
        "floor_encode_ms": back_to_back_ms(lambda: fused_encode(x, W_sub, be_sub, sae.b_dec, activation="relu"), 5),
        "floor_select_ms": back_to_back_ms(lambda: topk_rows(f_sub, k), 5),
    }
    del f_sub
    lists = encode_rows(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu", cap=ops.TOPK_CAP, row_floor=floor)
    pieces["filtered_gemm_ms"] = back_to_back_ms(
        lambda: encode_rows(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu", cap=ops.TOPK_CAP,
                            row_floor=floor), 5)
    pieces["list_select_ms"] = back_to_back_ms(lambda: ops.rows_topk(*lists, k, d_sae), 5)
    pieces["longest_list"] = int(lists[0].max())
    sel = ops.rows_topk(*lists, k, d_sae)

    def redo():  # the overflow redo as _topk_rows runs it (no row overflows at this config)
        rows, n_over = ops.overflow_rows(lists[0], ops.TOPK_CAP)
        f = ops.encode_gather(x, sae.W_enc, sae.b_enc, sae.b_dec, rows, n_over, out_rows=T)
        ops.topk_gather(f, k, n_over, rows, *sel)
    pieces["overflow_redo_ms"] = back_to_back_ms(redo, 5)
    del sel
    del lists
    pieces["dense_alternative_ms"] = back_to_back_ms(lambda: ops._topk_dense(sae, x), 3)
    enc_flops = workloads.encode_flops(T, d_in, d_sae)
    pieces["filtered_gemm_tflops"] = round(enc_flops / (pieces["filtered_gemm_ms"] * 1e-3) / 1e12, 1)
    for key in list(pieces):
        if key.endswith("_ms"):
            pieces[key] = round(pieces[key], 4)
    enc_tf = enc_flops / (enc_avg * 1e-3) / 1e12
    peak_tf = PEAK_TFLOPS[dtype]
    dec_bytes = workloads.decode_bytes(T, d_in, nnz, esize)
    return {
        "value": round(enc_tf, 2),
        "ms_per_step": round(total_ms / K, 4),
        "l0_measured": k,
        "decode_requested_gbps": round(dec_bytes / (dec_avg * 1e-3) / 1e9, 1),
        "tokens_per_s": round(T / (total_ms / K * 1e-3), 1),
        "stages": {
            "encode_topk": {"ms": round(enc_avg, 4), "tflops": round(enc_tf, 2), "frac": round(enc_tf / peak_tf, 4),
                            "pieces": pieces, "floor_features": S},
            "decode": {"ms": round(dec_avg, 4), "requested_bytes": dec_bytes, "nnz": nnz,
                       "kernel_ms": round(dec_kernel_ms, 4)},
        },
        "torch_reference": None if args.no_blas else torch_reference(
            sae, x, meta, (indptr, indices_l.view(-1), values_l.view(-1)), flush),
        "roofline": {"bound": "mfma", "achieved": round(enc_tf, 2), "peak": peak_tf, "unit": "TFLOP/s",
                     "frac": round(enc_tf / peak_tf, 4), "traffic": read_traffic(args.config, "encode_rows")},
        "roofline_decode": decode_roofline(args.config, indices_l, T, d_in, nnz, esize, dec_kernel_ms),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C3")
    ap.add_argument("--tokens", type=int, default=None, help="override T (default: the config's)")
    ap.add_argument("--cpu-seconds", type=float, default=16.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first launch a plain copy kernel over MIB MiB (for --pmc byte calibration)")
    ap.add_argument("--mfma-from", metavar="DIR",
                    help="summarise a rocprofv3 --pmc pass of SQ_VALU_MFMA_BUSY_CYCLES, "
                         "SQ_INSTS_VALU_MFMA_MOPS_BF16 and GRBM_GUI_ACTIVE under DIR into profiles/mfma.json (CPU only)")
    ap.add_argument("--sq-from", metavar="DIR",
                    help="summarise a rocprofv3 --pmc pass of the SQ_COUNTERS (waits, LDS, VMEM) under DIR (CPU only)")
    ap.add_argument("--lds-from", metavar="DIR",
                    help="summarise a rocprofv3 --pmc pass of the LDS_COUNTERS under DIR (CPU only)")
    ap.add_argument("--stats-from", metavar="DIR",
                    help="summarise the kernel_stats.csv of a rocprofv3 --kernel-trace --stats run under DIR "
                         "(CPU only)")
    ap.add_argument("--gemms-only", action="store_true",
                    help="run only the encode GEMM of --config in both W layouts and hipBLASLt's, for counter passes")
    ap.add_argument("--mix-from", metavar="DIR",
                    help="summarise the three MIX_PASSES --pmc passes of --gemms-only under DIR/p1..p3 (CPU only)")
    ap.add_argument("--no-backward", action="store_true", help="skip the backward (training) leg")
    ap.add_argument("--no-cache", action="store_true", help="skip the activation-cache caller leg")
    ap.add_argument("--no-blas", action="store_true", help="skip the hipBLASLt GEMM comparison leg")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="summarise rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE passes under DIR/fetch, DIR/write "
                         "into profiles/traffic.json under --config (CPU only; needs --calibrate-copy MIB of the "
                         "profiled run)")
    args = ap.parse_args()
    if args.traffic_from:
        traffic_summary(args.traffic_from, args.calibrate_copy or 1024, args.config)
        return
    if args.mfma_from:
        mfma_summary(args.mfma_from, args.config)
        return
    if args.sq_from:
        sq_summary(args.sq_from)
        return
    if args.lds_from:
        lds_summary(args.lds_from)
        return
    if args.stats_from:
        stats_summary(args.stats_from)
        return
    if args.mix_from:
        mix_summary(args.mix_from)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the SAE path's multi-GPU sharding is a design note, not a measured run", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)

    from saeflow_amd import workloads

    torch.cuda.set_device(0)
    if args.gemms_only:
        gemms_only(args.config)
        return
    if args.calibrate_copy:
        copy_calibration(args.calibrate_copy)
    sae, x, meta = workloads.make(args.config, T=args.tokens, device="cuda")
    T, d_in, d_sae, dtype = meta["T"], meta["d_in"], meta["d_sae"], meta["dtype"]
    flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
    topk = meta["activation"] == "topk"
    legs = (bench_topk if topk else bench_path)(args, sae, x, meta, flush)
    del flush
    enc_tf = legs["value"]
    result = {
        "metric": METRIC,
        "value": enc_tf,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": legs.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAME[dtype],
        "data": "synthetic (seeded: W_enc~N(0,1/d_in), " + ("b_enc=-2.8" if topk or meta["activation"] == "relu"
                                                           else "log-normal JumpReLU thresholds") + ", x=b_dec+N(0,1))",
        "config": {"workload": f"{args.config}: {meta['activation']} {DTYPE_NAME[dtype]} d_in={d_in} "
                               f"d_sae={d_sae} T={T} " + (f"k={meta['k']}" if topk else f"L0={meta['l0_target']}"),
                   "tokens": T, "d_in": d_in, "d_sae": d_sae, "activation": meta["activation"],
                   "l0_measured": legs.pop("l0_measured"), "parallelism": "single GPU"},
    }
    legs.pop("value")
    result.update(legs)
    result["device"] = torch.cuda.get_device_name(0)
    if not args.no_blas:
        result["blas_reference"] = blas_reference(T, d_in, d_sae, dtype)
    if not args.no_cache and not topk:
        result["cache"] = cache_leg(sae, d_in, dtype)
    counters = read_mfma(args.config)
    if counters:
        result["roofline"]["mfma_counters"] = {k: counters[k] for k in ("mfma_busy", "clock_ghz", "max_clock_ghz")}
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(sae, x, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
