#!/usr/bin/env python3
"""Benchmark: cascade verify attention at Qwen3-8B shape on one MI355X.

Workload (one "step" = one verify step of the target model): all 36 layers of
cascade verify attention, Qwen3-8B shape (32 query / 8 kv heads, head_dim 128,
bf16), prefix 4096 tokens paged at 16 with a random page permutation, and the
D2SD candidate tree of generation/d3_generator.py:116-180 (DFlash block 16 +
top-4 DTA branches of block 32; N unique nodes).  Each layer has its own KV
pool (604 MB in total, beyond the 256 MB Infinity Cache).  The 36 layer calls
(attention launch + merge launch each) are captured in one hipGraph and
replayed.

Prints ONE JSON line.  value = microseconds per layer-call (lower is better).

HBM traffic of the attention launch (roofline.traffic) comes from two
rocprofv3 counter runs over this same workload:

    python bench.py --measure-traffic     # writes profiles/verify_attn_cfg2_traffic.txt

which starts `rocprofv3 --pmc FETCH_SIZE` and then `--pmc WRITE_SIZE` as child
processes on `bench.py --traffic-workload` (the 36 attention launches plus a
plain 256 MiB device copy of known size).  Each counter is scaled by
known_bytes / counter for the copy kernel.  A default run reads that file.

MFMA utilisation of the attention launch (SQ_VALU_MFMA_BUSY_CYCLES, MFMA
instruction and MOPS counts, GRBM_GUI_ACTIVE, kernel trace) comes from

    python bench.py --measure-mfma        # writes profiles/verify_attn_cfg2_mfma.txt
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "d2-sd_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "cascade-verify attn µs/layer + HBM GB/s (% roofline), Qwen3-8B shape, 1 GPU"
TRAFFIC_FILE = ROOT / "profiles" / "verify_attn_cfg2_traffic.txt"
COPY_BYTES = 256 << 20
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_graph(graph, reps: int, torch) -> float:
    """Average milliseconds per replay of `graph` (HIP events on the stream the
    replays are launched on)."""
    s = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(reps):
        graph.replay(s)
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def cpu_threads() -> dict:
    """Host threads for the CPU baseline: os.cpu_count() (the baseline
    recipe: torch on every host core), bounded by the process's CPU affinity
    and by OMP_NUM_THREADS when the environment sets it (a host may grant a
    share of its cores)."""
    count = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = count
    threads = min(count, affinity)
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    return {"os_cpu_count": count, "affinity": affinity, "omp_num_threads": omp, "threads": threads}


def cpu_baseline(mp, reps: int, torch, sample: str) -> dict:
    """The oracle's fp32 torch-sdpa form of request 0 of one layer on the host
    cores (3 warm-ups, median of `reps`)."""
    from oracle import cascade_oracle as orc
    prob = mp.problem
    th = cpu_threads()
    torch.set_num_threads(th["threads"])
    lt = mp.layers[0]
    req = prob.requests[0]
    L = req.prefix_len
    if prob.page_size > 0:
        pages = mp.page_table[mp.page_indptr[0]:mp.page_indptr[1]].cpu().tolist()
        kp = orc.gather_paged(lt.k_prefix.cpu(), pages, L).float()
        vp = orc.gather_paged(lt.v_prefix.cpu(), pages, L).float()
    else:
        s0 = mp.prefix_tok_indptr[0]
        kp = lt.k_prefix.cpu()[:, s0:s0 + L].transpose(0, 1).float()
        vp = lt.v_prefix.cpu()[:, s0:s0 + L].transpose(0, 1).float()
    a, b = prob.qo_indptr[0], prob.qo_indptr[1]
    q, ks, vs = lt.q[a:b].cpu().float(), lt.k_suffix[a:b].cpu().float(), lt.v_suffix[a:b].cpu().float()
    m = torch.as_tensor(req.tree.ancestor_mask())
    sm = prob.head_dim ** -0.5

    def once():
        return orc.cascade_tree_ref(q, ks, vs, kp, vp, m, sm, prob.window_left, None, dtype=torch.float32,
                                    use_sdpa=True)

    for _ in range(3):
        once()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    us = statistics.median(times) * 1e6
    nq = b - a
    return {"value": us, "unit": "us/layer", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{sample}: one layer, {nq} queries, prefix {L} + tree; fp32 torch scaled_dot_product_attention "
                      f"+ logsumexp on the host, median of {reps} after 3 warm-ups",
            "queries_per_s": nq / (us * 1e-6), "cpu_model": cpu_model(), **th}


CAL_BYTES = 1 << 30   # fill / sum calibration buffers: 32x the 32 MiB of L2 over all XCDs


def traffic_workload(args) -> int:
    """The workload the counter runs profile, per round: a 1 GiB fill
    (write-only calibration), a 1 GiB sum of another buffer (read-only
    calibration), a COPY_BYTES device copy, then the attention launch of every
    layer; three rounds."""
    import torch
    import d2sd
    from d2sd import workloads as wl
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    wbuf = torch.empty(CAL_BYTES // 4, dtype=torch.float32, device=dev)
    rbuf = torch.ones(CAL_BYTES // 4, dtype=torch.float32, device=dev)
    prob = _traffic_problem(wl, args)
    mp = wl.materialize(prob, dev)
    attn = d2sd.CascadeVerifyAttention(dev)
    wl.plan_for(attn, mp)
    T, hq, d = prob.total_q, prob.num_qo_heads, prob.head_dim
    o = torch.empty(T, hq, d, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(T, hq, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    for _ in range(3):
        wbuf.fill_(1.5)
        rbuf.sum()
        dst.copy_(src)
        for lt in mp.layers:
            attn.run_attention(lt.q, lt.k_suffix, lt.v_suffix, lt.k_prefix, lt.v_prefix, out=o, lse=lse)
        torch.cuda.synchronize()
    print(f"traffic workload done: {attn.info.num_slots} partial slots, {attn.info.num_items} items", flush=True)
    return 0


def _traffic_problem(wl, args):
    """The workload of the traffic passes: config 2 (36 layers, one KV pool
    each) or config 3 (8 requests of 8K-32K keys: one 670 MB pool already
    passes the 256 MB MALL)."""
    if args.traffic_config == "config3":
        return wl.config3(args.seed)
    return wl.config2(args.seed, layers=args.layers)


def _traffic_file(args) -> Path:
    return ROOT / "profiles" / ("verify_attn_cfg3_traffic.txt" if args.traffic_config == "config3"
                                else "verify_attn_cfg2_traffic.txt")


def _kernel_class(name: str):
    if "verify_attn_kernel" in name:
        return "attention"
    if "copyBuffer" in name:
        return "copy"
    if "FillFunctor" in name:
        return "fill"
    if "reduce_kernel" in name:
        return "sum"
    return None


def _counter_means(csv_path: Path, counter: str) -> dict:
    import csv
    sums, counts = {}, {}
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            key = _kernel_class(row["Kernel_Name"])
            if key is None:
                continue
            sums[key] = sums.get(key, 0.0) + float(row["Counter_Value"])
            counts[key] = counts.get(key, 0) + 1
    return {k: sums[k] / counts[k] for k in sums}


def _pmc_pass(counters, outdir: Path, args, kernel_trace: bool = False):
    """One rocprofv3 counter pass over the traffic workload (a child process);
    returns the directory it wrote, or None after printing the failure."""
    import subprocess
    # each pass in its own process under a hard time limit: a counter set the
    # hardware cannot collect makes rocprofv3 stop responding
    cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", *counters]
    if kernel_trace:
        cmd.append("--kernel-trace")
    cmd += ["--kernel-include-regex", TRAFFIC_KERNELS,
            "-d", str(outdir), "-o", "run", "--output-format", "csv", "--",
            sys.executable, str(Path(__file__).resolve()), "--traffic-workload",
            "--layers", str(args.layers), "--seed", str(args.seed), "--traffic-config", args.traffic_config]
    log("running " + " ".join(cmd))
    r = subprocess.run(cmd, capture_output=True, text=True)
    _PMC_STDOUT.append(r.stdout)
    if r.returncode != 0:
        print(r.stdout[-2000:], r.stderr[-2000:], file=sys.stderr)
        return None
    return outdir


_PMC_STDOUT: list = []


TRAFFIC_KERNELS = "verify_attn_kernel|copyBuffer|FillFunctor|reduce_kernel"


def _attention_mean_ns(trace_csv: Path) -> float:
    import csv
    durs = []
    with open(trace_csv) as f:
        for row in csv.DictReader(f):
            if "verify_attn_kernel" in row["Kernel_Name"]:
                durs.append(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    return statistics.mean(durs)


MFMA_FILE = ROOT / "profiles" / "verify_attn_cfg2_mfma.txt"
SHADER_ENGINES = 32  # MI355X: 8 XCDs x 4 shader engines (rocminfo)
MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_BF16",
                 "SQ_BUSY_CYCLES", "GRBM_GUI_ACTIVE")


def measure_mfma(args) -> int:
    """MFMA utilisation of the attention launch: one rocprofv3 pass with the
    SQ MFMA counters and the kernel trace over the traffic workload; writes
    MFMA_FILE.  MOPS counts units of 512 flops; one v_mfma_f32_32x32x16_bf16
    is 32*32*16*2 = 32768 flops = 64 MOPS."""
    import tempfile
    from d2sd import workloads as wl
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as tmp:
        out = _pmc_pass(MFMA_COUNTERS, Path(tmp) / "mfma", args, kernel_trace=True)
        if out is None:
            return 1
        files = list(out.rglob("*counter_collection.csv"))
        traces = list(out.rglob("*kernel_trace.csv"))
        if not files or not traces:
            print("rocprofv3 wrote no counter_collection.csv / kernel_trace.csv", file=sys.stderr)
            return 1
        c = {name: _counter_means(files[0], name)["attention"] for name in MFMA_COUNTERS}
        dur_ns = _attention_mean_ns(traces[0])
    prob = wl.config2(args.seed, layers=args.layers)
    _, af = wl.attention_launch_bytes_flops(prob)
    cus, simds = 256, 4
    exec_flops = c["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512.0
    busy, grbm_xcd = c["SQ_VALU_MFMA_BUSY_CYCLES"], c["GRBM_GUI_ACTIVE"] / 8.0
    lines = [
        "# MFMA utilisation of the cascade verify attention launch, config 2 (Qwen3-8B, L=4096 paged, 36 layers)",
        f"# command: python bench.py --measure-mfma --layers {args.layers} --seed {args.seed}",
        "#   = rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + " --kernel-trace",
        f"#     --kernel-include-regex '{TRAFFIC_KERNELS}' --output-format csv -- python bench.py --traffic-workload",
        "# counters: mean per attention dispatch; duration: mean kernel-trace duration of the same dispatches",
    ]
    lines += [f"{k}: {v:.0f}" for k, v in c.items()]
    lines += [
        f"attention_duration_ns: {dur_ns:.0f}",
        f"mops_per_mfma_instruction: {c['SQ_INSTS_VALU_MFMA_MOPS_BF16'] / max(c['SQ_INSTS_VALU_MFMA_BF16'], 1):.2f}",
        f"executed_mfma_flops_per_launch: {exec_flops:.0f}",
        f"algorithmic_flops_per_launch: {af:.0f}",
        f"executed_over_algorithmic: {exec_flops / af:.3f}",
        f"executed_tflops: {exec_flops / dur_ns / 1e3:.1f}",
        f"executed_frac_of_2500_tflops: {exec_flops / dur_ns / 1e3 / MFMA_BF16_PEAK_TFLOPS:.3f}",
        f"mfma_busy_cycles_per_instruction: {c['SQ_VALU_MFMA_BUSY_CYCLES'] / max(c['SQ_INSTS_VALU_MFMA_BF16'], 1):.2f}",
        # the csv value of GRBM_GUI_ACTIVE is the sum over the 8 XCD instances;
        # rocprof's MfmaUtil expression divides by one instance (its max)
        f"grbm_gui_active_per_xcd: {grbm_xcd:.0f}",
        f"mfma_util_rocprof_expr: {busy / (grbm_xcd * cus * simds):.4f}",
        f"mfma_util_over_trace_duration_at_2400MHz: {busy / (dur_ns * 2.4 * cus * simds):.4f}",
        # SQ_BUSY_CYCLES sums the busy cycles of the 32 shader engines
        # (rocminfo: 8 XCDs x 4); per engine over the traced duration it is
        # the clock the launch actually ran at
        f"sq_busy_cycles_per_shader_engine: {c['SQ_BUSY_CYCLES'] / SHADER_ENGINES:.0f}",
        f"effective_clock_ghz: {c['SQ_BUSY_CYCLES'] / SHADER_ENGINES / dur_ns:.3f}",
        f"mfma_peak_at_effective_clock_tflops: {cus * simds * 1024 * c['SQ_BUSY_CYCLES'] / SHADER_ENGINES / dur_ns / 1e3:.0f}",
        f"executed_frac_of_peak_at_effective_clock: "
        f"{exec_flops / (cus * simds * 1024.0 * c['SQ_BUSY_CYCLES'] / SHADER_ENGINES):.3f}",
    ]
    MFMA_FILE.parent.mkdir(exist_ok=True)
    MFMA_FILE.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


TRAFFIC_PASSES = (
    ("FETCH_SIZE",),
    ("WRITE_SIZE",),
    ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum"),
    ("TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum", "TCC_EA0_RDREQ_DRAM_sum", "TCC_EA0_WRREQ_DRAM_sum"),
)


MIX_FILE = ROOT / "profiles" / "verify_attn_cfg2_instmix.txt"
MIX_PASSES = (
    ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_SALU", "SQ_INSTS_VALU_TRANS_F32",
     "SQ_ACTIVE_INST_VALU", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_WAIT_INST_LDS"),
    ("SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_ANY", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_BUSY_CYCLES",
     "SQ_INSTS_VALU_CVT", "SQ_THREAD_CYCLES_VALU", "SQ_INSTS_SMEM"),
    ("SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_LDS_LOAD_BANDWIDTH", "SQ_ACTIVE_INST_VALU2",
     "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES"),
    ("LdsLatency",),
)
CUS, SIMDS = 256, 1024


def measure_mix(args) -> int:
    """Instruction mix of the attention launch: two rocprofv3 passes of SQ
    counters over the traffic workload; writes MIX_FILE.  Per wave-tile
    figures divide by the launch's prefix wave-tiles (items x waves x 64-key
    tiles of their ranges; the suffix items' few tiles are left out)."""
    import tempfile
    from d2sd import workloads as wl
    res = {}
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as tmp:
        for i, counters in enumerate(MIX_PASSES):
            out = _pmc_pass(counters, Path(tmp) / f"mix{i}", args)
            if out is None:
                return 1
            files = list(out.rglob("*counter_collection.csv"))
            if not files:
                print("no counter_collection.csv from rocprofv3", file=sys.stderr)
                return 1
            for c in counters:
                res[c] = _counter_means(files[0], c)["attention"]
    prob = wl.config2(args.seed, layers=args.layers)
    hkv, T, L = prob.num_kv_heads, prob.total_q, prob.requests[0].prefix_len
    qtiles = (T * prob.num_qo_heads // hkv + 127) // 128
    wave_tiles = hkv * qtiles * (L // 64) * 4
    valu = res["SQ_INSTS_VALU"] - res["SQ_INSTS_MFMA"]
    lines = [
        "# Instruction mix of the cascade verify attention launch, config 2 (Qwen3-8B, L=4096 paged, 36 layers)",
        f"# command: python bench.py --measure-mix --layers {args.layers} --seed {args.seed}",
        f"#   = {len(MIX_PASSES)} passes, each: timeout -s KILL 120 rocprofv3 --pmc <counters>",
        f"#     --kernel-include-regex '{TRAFFIC_KERNELS}' --output-format csv -- python bench.py --traffic-workload",
        "#   passes: " + " | ".join(" ".join(c) for c in MIX_PASSES),
        "# mean per attention dispatch",
    ]
    lines += [f"{k}: {v:.0f}" for k, v in res.items()]
    lines += [
        "",
        f"prefix_wave_tiles (8 kv heads x {qtiles} q-tiles x {L // 64} tiles x 4 waves): {wave_tiles}",
        f"mfma_per_wave_tile: {res['SQ_INSTS_MFMA'] / wave_tiles:.1f}",
        f"valu_non_mfma_per_wave_tile: {valu / wave_tiles:.1f}  (includes the per-item prologue and epilogue)",
        f"trans_per_wave_tile: {res['SQ_INSTS_VALU_TRANS_F32'] / wave_tiles:.1f}",
        f"lds_per_wave_tile: {res['SQ_INSTS_LDS'] / wave_tiles:.1f}",
        f"salu_per_wave_tile: {res['SQ_INSTS_SALU'] / wave_tiles:.1f}",
        f"valu_per_mfma: {valu / res['SQ_INSTS_MFMA']:.2f}",
        "",
        "# per SIMD (1024) or CU (256) over the launch: SQ_BUSY_CYCLES summed over the",
        f"# {SHADER_ENGINES} shader engines / {SHADER_ENGINES} = the launch's cycles",
        f"launch_cycles: {res['SQ_BUSY_CYCLES'] / SHADER_ENGINES:.0f}",
        f"valu_issue_cycles_per_simd (SQ_ACTIVE_INST_VALU quad-cycles x 4): "
        f"{res['SQ_ACTIVE_INST_VALU'] * 4 / SIMDS:.0f}",
        f"mfma_busy_cycles_per_simd: {res['SQ_VALU_MFMA_BUSY_CYCLES'] / SIMDS:.0f}",
        f"valu_mfma_coexec_cycles_per_simd: {res['SQ_VALU_MFMA_COEXEC_CYCLES'] / SIMDS:.0f}",
        f"lds_active_cycles_per_cu: {res['SQ_LDS_IDX_ACTIVE'] / CUS:.0f}",
        f"lds_active_frac: {res['SQ_LDS_IDX_ACTIVE'] / CUS / (res['SQ_BUSY_CYCLES'] / SHADER_ENGINES):.3f}",
        f"lds_read_bytes_per_active_cycle_per_cu: "
        f"{res['SQ_INSTS_LDS_LOAD_BANDWIDTH'] * 64 / res['SQ_LDS_IDX_ACTIVE']:.0f}",
        f"lds_latency_cycles (LdsLatency): {res['LdsLatency']:.1f}",
    ]
    MIX_FILE.parent.mkdir(exist_ok=True)
    MIX_FILE.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


def measure_traffic(args) -> int:
    """HBM traffic of the attention launch: four counter passes of the
    traffic workload (FETCH_SIZE; WRITE_SIZE; the L2-to-fabric read requests
    by size; write requests), each a child process; writes the summary
    under profiles/ (verify_attn_cfg2_traffic.txt or ..._cfg3_traffic.txt).

    Calibration: the 1 GiB fill writes and the 1 GiB sum reads known bytes
    with no reuse, so measured / known is what the counters see of a
    streaming kernel spread over all XCDs; the attention launch's figures are
    divided by it.  Itemisation: its reads are the unique prefix and suffix
    K/V, Q, the page table, the tree mask and the plan records, plus re-reads
    of K/V chunks by the q-tiles that share them; its writes are the partial
    slots (bf16 [rows, D] + fp32 [rows] each)."""
    import re
    import tempfile
    from d2sd import workloads as wl
    res, slots_seen = {}, []
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as tmp:
        for i, counters in enumerate(TRAFFIC_PASSES):
            out = _pmc_pass(counters, Path(tmp) / f"pass{i}", args)
            if out is None:
                return 1
            m = re.search(r"traffic workload done: (\d+) partial slots, (\d+) items", _PMC_STDOUT[-1])
            slots_seen.append((int(m.group(1)), int(m.group(2))))
            files = list(out.rglob("*counter_collection.csv"))
            if not files:
                print("no counter_collection.csv from rocprofv3", file=sys.stderr)
                return 1
            for c in counters:
                res[c] = _counter_means(files[0], c)
    prob = _traffic_problem(wl, args)
    hq, hkv, d, T = prob.num_qo_heads, prob.num_kv_heads, prob.head_dim, prob.total_q
    P = prob.page_size
    ab, _ = wl.attention_launch_bytes_flops(prob)
    slots, nitems = slots_seen[0]
    rows = 128
    items = {
        "prefix_kv_unique": sum(2 * r.prefix_len * hkv * d * 2 for r in prob.requests),
        "suffix_kv": 2 * T * hkv * d * 2,
        "q": T * hq * d * 2,
        "page_table": sum(4 * ((r.prefix_len + P - 1) // P) for r in prob.requests),
        "tree_mask": sum(r.n * ((r.n + 63) // 64) * 8 for r in prob.requests),
        "plan_items": nitems * 64,
    }
    w_items = {"partial_slots": slots * (rows * d * 2 + rows * 4)}

    def hist_reads(k):
        return (32 * res["TCC_EA0_RDREQ_32B_sum"][k] + 64 * res["TCC_EA0_RDREQ_64B_sum"][k]
                + 128 * res["TCC_EA0_RDREQ_128B_sum"][k])

    def hist_writes(k):
        return (32 * (res["TCC_EA0_WRREQ_sum"][k] - res["TCC_EA0_WRREQ_64B_sum"][k])
                + 64 * res["TCC_EA0_WRREQ_64B_sum"][k])

    read_cov = hist_reads("sum") / CAL_BYTES
    write_cov = hist_writes("fill") / CAL_BYTES
    fetch_cov = res["FETCH_SIZE"]["sum"] * 1024 / CAL_BYTES
    wsize_cov = res["WRITE_SIZE"]["fill"] * 1024 / CAL_BYTES
    a_reads = hist_reads("attention") / read_cov
    a_writes = hist_writes("attention") / write_cov
    lines = [
        f"# HBM traffic of the cascade verify attention launch, {prob.name}",
        f"# command: python bench.py --measure-traffic --traffic-config {args.traffic_config} --layers {args.layers} "
        f"--seed {args.seed}",
        "#   = four passes, each: timeout -s KILL 120 rocprofv3 --pmc <counters>",
        f"#     --kernel-include-regex '{TRAFFIC_KERNELS}' --output-format csv -- python bench.py --traffic-workload",
        "#   passes: " + " | ".join(" ".join(c) for c in TRAFFIC_PASSES),
        "# per dispatch means; fill = 1 GiB written, sum = 1 GiB read, copy = 256 MiB read + written",
        "",
        "## raw counters (requests; FETCH_SIZE / WRITE_SIZE in KiB)",
    ]
    for c in ("FETCH_SIZE", "WRITE_SIZE", "TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum",
              "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum", "TCC_EA0_RDREQ_DRAM_sum",
              "TCC_EA0_WRREQ_DRAM_sum"):
        lines.append(f"{c}: " + ", ".join(f"{k} {res[c].get(k, float('nan')):.1f}"
                                         for k in ("fill", "sum", "copy", "attention")))
    lines += [
        "",
        "## calibration (what the counters see of known bytes)",
        f"read_request_bytes_over_known (sum kernel): {read_cov:.4f}",
        f"write_request_bytes_over_known (fill kernel): {write_cov:.4f}",
        f"FETCH_SIZE_over_known (sum kernel): {fetch_cov:.4f}",
        f"WRITE_SIZE_over_known (fill kernel): {wsize_cov:.4f}",
        f"copy_reads_calibrated_over_known: {hist_reads('copy') / read_cov / COPY_BYTES:.4f}",
        f"copy_writes_calibrated_over_known: {hist_writes('copy') / write_cov / COPY_BYTES:.4f}",
        "",
        "## attention launch, calibrated bytes per launch",
        f"reads: {a_reads:.0f}",
        f"writes: {a_writes:.0f}",
        "",
        "## itemised (bytes per launch)",
    ]
    lines += [f"read {k}: {v}" for k, v in items.items()]
    unique = sum(items.values())
    lines += [
        f"read unique total: {unique}  (algorithmic bytes of the launch: {ab})",
        f"read beyond unique (K/V chunks re-read by q-tiles sharing them): {a_reads - unique:.0f} "
        f"= {(a_reads - unique) / items['prefix_kv_unique']:.3f} x prefix K/V",
        f"write partial_slots: {w_items['partial_slots']}  ({slots} slots x ({rows} rows x {d} x 2 + {rows} x 4))",
        f"writes measured / itemised: {a_writes / w_items['partial_slots']:.3f}",
        "",
        f"traffic_bytes_per_launch: {a_reads + a_writes:.0f}",
    ]
    out_file = _traffic_file(args)
    out_file.parent.mkdir(exist_ok=True)
    out_file.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


def measure_commit(args) -> int:
    """Accepted-branch KV commit (d2sd.PagedKVCommit, generation/d3_generator.py:
    227-232) at Qwen3-8B shape: 36 layers, prefix 4096 paged at 16, the first
    acceptance_length tokens of row 1 of the d3 verify tree.  Beside it, the
    reference's own form on the same GPU: per layer torch.cat of the
    [1, Hkv, L, D] cache with the accepted window (keys and values), which
    copies the whole cache.  Prints one JSON line."""
    import numpy as np
    import torch
    import d2sd
    from d2sd import tree as dtree

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    layers, P, hkv, d, L, acc = args.layers, 16, 8, 128, 4096, args.accepted
    tr = dtree.d3_verify_tree(np.random.default_rng(args.seed).uniform(size=15))
    rows = tr.num_nodes
    acc = min(acc, tr.node_index.shape[1])
    nodes = torch.as_tensor(tr.node_index[1][:acc], dtype=torch.int32, device=dev)
    pages = (L + acc + P - 1) // P
    g = torch.Generator(device=dev).manual_seed(args.seed)
    kp = [torch.randn(pages + 8, hkv, P, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    vp = [torch.randn(pages + 8, hkv, P, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    kn = [torch.randn(rows, hkv, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    vn = [torch.randn(rows, hkv, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    table = torch.randperm(pages + 8, generator=g, device=dev)[:pages].to(torch.int32)
    commit = d2sd.PagedKVCommit(kp, vp, kn, vn)
    commit.commit(table, L, nodes)
    torch.cuda.synchronize()
    # many commits in one graph, so that the host's graph launches do not
    # pace the GPU (a single-kernel graph replays slower than its kernel runs)
    per_graph = 32
    gc = d2sd.HipGraph()
    with gc.capture():
        for _ in range(per_graph):
            commit.commit(table, L, nodes)
    us = time_graph(gc, max(3, args.kernel_reps // 4), torch) * 1e3 / per_graph
    # reference form: DynamicCache layer tensors [1, Hkv, L, D], grown by torch.cat
    kc = [torch.randn(1, hkv, L, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    vc = [torch.randn(1, hkv, L, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    kw = [torch.randn(1, hkv, acc, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    vw = [torch.randn(1, hkv, acc, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    for _ in range(3):
        out = [(torch.cat([kc[i], kw[i]], dim=2), torch.cat([vc[i], vw[i]], dim=2)) for i in range(layers)]
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = max(5, args.kernel_reps // 5)
    e0.record()
    for _ in range(reps):
        out = [(torch.cat([kc[i], kw[i]], dim=2), torch.cat([vc[i], vw[i]], dim=2)) for i in range(layers)]
    e1.record()
    torch.cuda.synchronize()
    ref_us = e0.elapsed_time(e1) / reps * 1e3
    del out
    moved = 2 * layers * acc * hkv * d * 2 * 2  # K and V rows, read + written
    print(json.dumps({
        "metric": "accepted-branch KV commit µs/step (36 layers, Qwen3-8B shape)",
        "value": us, "unit": "us", "higher_is_better": False, "accepted_tokens": acc,
        "bytes_moved": moved, "achieved_gbps": moved / (us * 1e-6) / 1e9,
        "hbm_frac": moved / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
        "reference_torch_cat_us": ref_us,
        "reference_torch_cat_bytes": 2 * layers * 2 * (2 * L + acc) * hkv * d,
        "speedup_vs_reference": ref_us / us,
        "config": {"workload": "config 2 verify step commit", "layers": layers, "prefix": L, "page_size": P},
    }))
    return 0


def measure_accept(args) -> int:
    """Greedy acceptance walk (d2sd.GreedyAccept, generation/d3_generator.py:
    204-225 at temperature 0) at Qwen3-8B shape: the d3 verify tree's unique
    nodes' logits [N, 151936] bf16, drafts following the target for a few
    positions.  Beside it, the reference's own loop on the same GPU tensors
    (host-driven: nonzero(), argmax, sum() per accepted token).  One JSON line."""
    import numpy as np
    import torch
    import d2sd
    from d2sd import tree as dtree

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    vocab = 151936
    tr = dtree.d3_verify_tree(np.random.default_rng(args.seed).uniform(size=15))
    N, lb = tr.num_nodes, tr.node_index.shape[1]
    g = torch.Generator(device=dev).manual_seed(args.seed)
    logits = torch.randn(N, vocab, generator=g, device=dev, dtype=torch.bfloat16)
    node_index = torch.as_tensor(tr.node_index, dtype=torch.int32, device=dev)
    am = logits.argmax(-1)
    drafts = torch.randint(0, vocab, tuple(node_index.shape), generator=g, device=dev)
    keep = [9, 14, 3, 20, 1]
    for r in range(node_index.shape[0]):
        for pos in range(1, keep[r]):
            drafts[r, pos] = am[node_index[r, pos - 1]]
    acc = d2sd.GreedyAccept(N, vocab, lb, dev)
    acc(logits, node_index, drafts)
    torch.cuda.synchronize()
    per_graph = 32
    ga = d2sd.HipGraph()
    with ga.capture():
        for _ in range(per_graph):
            acc(logits, node_index, drafts)
    us = time_graph(ga, max(3, args.kernel_reps // 4), torch) * 1e3 / per_graph
    n = int(acc.result[0])
    # the reference loop (d3_generator.py:204-225), rows' logits gathered once
    out_logits = logits[node_index.long()]
    def ref_loop():
        valid_blocks = torch.ones(out_logits.shape[0], device=dev)
        acceptance_length = 0
        accept = []
        while True:
            valid_block = (valid_blocks > 0).nonzero(as_tuple=True)[0][0]
            tok = torch.argmax(out_logits[valid_block, acceptance_length, :].unsqueeze(0), dim=-1)
            acceptance_length += 1
            accept.append(tok)
            if acceptance_length == lb:
                break
            valid_blocks = torch.where(drafts[:, acceptance_length] == tok, valid_blocks, 0)
            if valid_blocks.sum() == 0.:
                break
        return acceptance_length
    for _ in range(3):
        n_ref = ref_loop()
    torch.cuda.synchronize()
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        n_ref = ref_loop()
    torch.cuda.synchronize()
    ref_us = (time.perf_counter() - t0) / reps * 1e6
    moved = N * vocab * 2
    print(json.dumps({
        "metric": "greedy acceptance walk µs/step (d3 tree, Qwen3 vocab)",
        "value": us, "unit": "us", "higher_is_better": False, "nodes": N, "vocab": vocab,
        "acceptance_length": n, "reference_acceptance_length": n_ref,
        "bytes_read": moved, "achieved_gbps": moved / (us * 1e-6) / 1e9,
        "hbm_frac": moved / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
        "reference_host_loop_us": ref_us, "speedup_vs_reference": ref_us / us,
        "config": {"workload": "config 2 verify step acceptance", "rows": int(node_index.shape[0]), "row_len": lb},
    }))
    return 0


def measure_qk_rope(args) -> int:
    """QK RMSNorm + RoPE (d2sd.qk_norm_rope, generation/verification.py:113-123)
    for the 36 layers of a Qwen3-8B verify step over the d3 tree's nodes, in
    one graph; beside it the reference's form on the same GPU (transformers
    Qwen3RMSNorm for q / k, the transposes, rotate_half RoPE).  One JSON line."""
    import numpy as np
    import torch
    import d2sd
    from d2sd import tree as dtree
    from transformers.models.qwen3 import modeling_qwen3 as mq

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    layers, hq, hkv, d = args.layers, 32, 8, 128
    T = dtree.d3_verify_tree(np.random.default_rng(args.seed).uniform(size=15)).num_nodes
    g = torch.Generator(device=dev).manual_seed(args.seed)
    qkv = [torch.randn(T, hq + 2 * hkv, d, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    wq = [(torch.rand(d, generator=g, device=dev) + 0.5).to(torch.bfloat16) for _ in range(layers)]
    wk = [(torch.rand(d, generator=g, device=dev) + 0.5).to(torch.bfloat16) for _ in range(layers)]
    pos = torch.arange(T, device=dev) + 4096
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, device=dev).float() / d))
    ang = pos[:, None].float() * inv[None]
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    def ours():
        for l in range(layers):
            d2sd.qk_norm_rope(qkv[l][:, :hq], qkv[l][:, hq:hq + hkv], wq[l], wk[l], cos, sin, 1e-6)
    ours()
    torch.cuda.synchronize()
    gr = d2sd.HipGraph()
    with gr.capture():
        ours()
    us = time_graph(gr, max(5, args.kernel_reps), torch) * 1e3
    qn, kn = mq.Qwen3RMSNorm(d, eps=1e-6).to(dev, torch.bfloat16), mq.Qwen3RMSNorm(d, eps=1e-6).to(dev, torch.bfloat16)
    def reference():
        outs = []
        for l in range(layers):
            q = qkv[l][None, :, :hq]                           # [1, T, Hq, D] as q.view(bsz, seq, H, D)
            k = qkv[l][None, :, hq:hq + hkv]
            q, k = qn(q).transpose(1, 2), kn(k).transpose(1, 2)
            q, k = mq.apply_rotary_pos_emb(q, k, cos[None], sin[None])
            outs.append((q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()))
        return outs
    with torch.no_grad():
        for _ in range(3):
            reference()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        e0.record()
        for _ in range(reps):
            reference()
        e1.record()
        torch.cuda.synchronize()
    ref_us = e0.elapsed_time(e1) / reps * 1e3
    moved = layers * (2 * T * (hq + hkv) * d * 2 + 2 * T * d * 2)
    print(json.dumps({
        "metric": "QK RMSNorm + RoPE µs/step (36 layers, Qwen3-8B shape, d3 tree nodes)",
        "value": us, "unit": "us", "higher_is_better": False, "tokens": T,
        "bytes_moved": moved, "achieved_gbps": moved / (us * 1e-6) / 1e9,
        "hbm_frac": moved / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
        "reference_torch_us": ref_us, "speedup_vs_reference": ref_us / us,
        "config": {"workload": "config 2 verify step QK norm + RoPE", "layers": layers},
    }))
    return 0


# the other workloads of the verify path (parity cases of the tests), each
# timed as a hipGraph of `layers` calls over distinct KV pools
OTHER_WORKLOADS = {
    "northstar": lambda wl, seed: (wl.northstar(seed), 36),  # 16.8 MB of KV per layer, 36 pools
    # KV pools per workload: together well past the 256 MB Infinity Cache, so
    # each call's prefix comes from HBM
    "config1": lambda wl, seed: (wl.config1(seed), 96),      # 4.2 MB of KV per pool: 403 MB
    "config3": lambda wl, seed: (wl.config3(seed), 2),       # ~670 MB of KV per pool
    "config4_full": lambda wl, seed: (wl.config4(seed), 24),  # 16.8 MB per pool: 403 MB
    "config4_sliding": lambda wl, seed: (wl.config4(seed, sliding=True), 24),
    "config5": lambda wl, seed: (wl.config5(seed), 2),       # ~540 MB of fp8 KV per call
}


SYSTEM_WORKLOADS = ("dropin", "dta", "step")


def _events_us(fn, reps: int, torch) -> float:
    """Mean µs per call of fn() over reps calls, HIP events on the current
    stream around the whole loop (eager: host dispatch included where it is
    slower than the GPU)."""
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(reps):
        fn()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def measure_dta(args) -> int:
    """The DTA draft's cascade (model/dflash.py:96-133) at Qwen3-8B heads: 4
    rows of 16 noise tokens, a DynamicCache draft layer of 4096 tokens and 17
    projected context tokens, one distinct cache per layer (36) so nothing
    stays in L2.  Three forms per layer: the reference's call site over the
    drop-ins (torch.cat of [cache | context], the NHD copies, single_prefill,
    the causal=False runner), eager; one plan whose shared level is the
    concatenation made by torch.cat each call; one plan reading the two
    segments in place (no concatenation).  The plan forms replay one hipGraph
    of all layers."""
    import numpy as np
    import torch
    import d2sd

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    bsz, ql, hq, hkv, d, lc, cap, ctx, nl = 4, 16, 32, 8, 128, 4096, 4096 + 256, 17, args.layers
    gen = torch.Generator(device=dev).manual_seed(args.seed + 2)

    def rnd(*shape):
        return torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)

    # per layer: q [bsz, Hq, q_len, D], the k/v projection [bsz, Hkv, ctx + q_len, D]
    # (dflash.py:87), the draft cache layer [1, Hkv, cap, D] holding lc tokens
    layers = [dict(q=rnd(bsz, hq, ql, d), k=rnd(bsz, hkv, ctx + ql, d), v=rnd(bsz, hkv, ctx + ql, d),
                   kc=rnd(1, hkv, cap, d), vc=rnd(1, hkv, cap, d)) for _ in range(nl)]
    scale = d ** -0.5
    n = bsz * ql
    runner = d2sd.CascadeGraphRunner(ql, hq, hkv, d, torch.bfloat16, dev, scale, causal=False)

    def call_site(x):
        k_sh = torch.cat([x["kc"][0, :, :lc], x["k"][0, :, :ctx]], dim=1)
        v_sh = torch.cat([x["vc"][0, :, :lc], x["v"][0, :, :ctx]], dim=1)
        q_fi = x["q"].transpose(1, 2)
        out, lse = d2sd.single_prefill_with_kv_cache(q_fi.reshape(n, hq, d), k_sh.transpose(0, 1).contiguous(),
                                                     v_sh.transpose(0, 1).contiguous(), causal=False,
                                                     return_lse=True, sm_scale=scale)
        runner.run(q_fi, x["k"][:, :, ctx:].transpose(1, 2).contiguous(),
                   x["v"][:, :, ctx:].transpose(1, 2).contiguous(), out.view(bsz, ql, hq, d), lse.view(bsz, ql, hq))
        return out

    mask = np.zeros((n, n), dtype=bool)
    for b in range(bsz):
        mask[b * ql:(b + 1) * ql, b * ql:(b + 1) * ql] = True
    two = d2sd.CascadeVerifyAttention(dev).plan([0, n], [lc + ctx], hq, hkv, d, tree_masks=[mask], page_size=0,
                                                kv_layout="HND", prefix_split=[lc])
    one = d2sd.CascadeVerifyAttention(dev).plan([0, n], [lc + ctx], hq, hkv, d, tree_masks=[mask], page_size=0,
                                                kv_layout="HND")
    # plan inputs made once: queries / noise K,V in the node layout
    prep = [dict(q=x["q"].transpose(1, 2).reshape(n, hq, d).contiguous(),
                 kn=x["k"][:, :, ctx:].transpose(1, 2).reshape(n, hkv, d).contiguous(),
                 vn=x["v"][:, :, ctx:].transpose(1, 2).reshape(n, hkv, d).contiguous(),
                 kcat=torch.empty(hkv, lc + ctx, d, dtype=torch.bfloat16, device=dev),
                 vcat=torch.empty(hkv, lc + ctx, d, dtype=torch.bfloat16, device=dev),
                 o=torch.empty(n, hq, d, dtype=torch.bfloat16, device=dev),
                 lse=torch.empty(n, hq, dtype=torch.float32, device=dev)) for x in layers]

    def run_two():
        for x, y in zip(layers, prep):
            two.run(y["q"], y["kn"], y["vn"], (x["kc"], x["k"][0, :, :ctx]), (x["vc"], x["v"][0, :, :ctx]),
                    out=y["o"], lse=y["lse"])

    def run_cat():
        for x, y in zip(layers, prep):
            torch.cat([x["kc"][0, :, :lc], x["k"][0, :, :ctx]], dim=1, out=y["kcat"])
            torch.cat([x["vc"][0, :, :lc], x["v"][0, :, :ctx]], dim=1, out=y["vcat"])
            one.run(y["q"], y["kn"], y["vn"], y["kcat"], y["vcat"], out=y["o"], lse=y["lse"])

    reps = max(5, args.kernel_reps // 5)
    for _ in range(3):
        for x in layers:
            call_site(x)
    site_us = _events_us(lambda: [call_site(x) for x in layers], reps, torch) / nl
    graphs = {}
    for key, fn in (("two", run_two), ("cat", run_cat)):
        fn()
        torch.cuda.synchronize()
        g = d2sd.HipGraph()
        with g.capture():
            fn()
        for _ in range(3):
            g.replay()
        graphs[key] = _events_us(g.replay, reps, torch) / nl
    print(json.dumps({
        "workload": "dta_draft_qwen3_8b_cache4096_ctx17_rows4x16", "value": graphs["two"], "unit": "us/layer",
        "higher_is_better": False, "rows": bsz, "row_len": ql, "queries": n, "cache_len": lc, "context_len": ctx,
        "layers": nl, "two_segment_us": graphs["two"], "concat_then_run_us": graphs["cat"],
        "reference_call_site_us": site_us,
        "note": "value: one plan reading [draft cache | context] in place, hipGraph of all layers; "
                "concat_then_run: the same plan shape over torch.cat's concatenation made each call (graph); "
                "reference_call_site: dflash.py:103-133 eager over the drop-ins (cat, NHD copies, "
                "single_prefill, causal=False runner)",
    }), flush=True)
    return 0


def measure_dropin(args) -> int:
    """The reference's own per-layer call site after `import d2sd as
    flashinfer` (generation/verification.py:137-165): at config 2's shape (the
    d3 tree's 5 rows x 32 positions, Qwen3-8B heads, DynamicCache prefix
    [Hkv, 4096, D] per layer), the transpose copies of the call site, then
    d2sd.single_prefill_with_kv_cache over all rows' queries and the
    CascadeGraphRunner's local attention + merge.  Eager, as the reference runs
    it; 36 layers of distinct KV so nothing stays in L2."""
    import numpy as np
    import torch
    import d2sd
    from d2sd import tree as dtree

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    conf = np.random.default_rng(args.seed).uniform(0.0, 1.0, size=15)
    tr = dtree.d3_verify_tree(conf, block_size=16, block_size_2=32, topk=4)
    bsz, lb, hq, hkv, d, L, nl = tr.num_rows, tr.row_len, 32, 8, 128, 4096, args.layers
    gen = torch.Generator(device=dev).manual_seed(args.seed + 1)

    def rnd(*shape):
        return torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)

    layers = [dict(q=rnd(bsz, hq, lb, d), k_new=rnd(bsz, hkv, lb, d), v_new=rnd(bsz, hkv, lb, d),
                   k=rnd(hkv, L, d), v=rnd(hkv, L, d)) for _ in range(nl)]
    scale = d ** -0.5
    runner = d2sd.CascadeGraphRunner(lb, hq, hkv, d, torch.bfloat16, dev, scale, causal=True)

    def call_site(x):
        k_fi = x["k"].transpose(0, 1).contiguous()
        v_fi = x["v"].transpose(0, 1).contiguous()
        q_fi = x["q"].transpose(1, 2)
        q_all = q_fi.reshape(bsz * lb, hq, d)
        out, lse = d2sd.single_prefill_with_kv_cache(q_all, k_fi, v_fi, causal=False, return_lse=True,
                                                     sm_scale=scale)
        out = out.view(bsz, lb, hq, d)
        lse = lse.view(bsz, lb, hq)
        runner.run(q_fi.contiguous(), x["k_new"].transpose(1, 2).contiguous(),
                   x["v_new"].transpose(1, 2).contiguous(), out, lse)
        return out

    # prepared inputs: the single-prefill and the runner alone
    prep = [dict(q_all=x["q"].transpose(1, 2).reshape(bsz * lb, hq, d), k_fi=x["k"].transpose(0, 1).contiguous(),
                 v_fi=x["v"].transpose(0, 1).contiguous(), q_fi=x["q"].transpose(1, 2).contiguous(),
                 k_new=x["k_new"].transpose(1, 2).contiguous(), v_new=x["v_new"].transpose(1, 2).contiguous())
            for x in layers]
    outs = [d2sd.single_prefill_with_kv_cache(x["q_all"], x["k_fi"], x["v_fi"], causal=False, return_lse=True,
                                              sm_scale=scale) for x in prep]
    torch.cuda.synchronize()

    def all_layers(fn, xs):
        def go():
            for x in xs:
                fn(x)
        return go

    for _ in range(3):
        all_layers(call_site, layers)()
    reps = max(5, args.kernel_reps // 5)
    site_us = _events_us(all_layers(call_site, layers), reps, torch) / nl
    prefill_us = _events_us(all_layers(lambda x: d2sd.single_prefill_with_kv_cache(
        x["q_all"], x["k_fi"], x["v_fi"], causal=False, return_lse=True, sm_scale=scale), prep), reps, torch) / nl
    runner_us = _events_us(lambda: [runner.run(x["q_fi"], x["k_new"], x["v_new"], o.view(bsz, lb, hq, d),
                                               l.view(bsz, lb, hq)) for x, (o, l) in zip(prep, outs)],
                           reps, torch) / nl
    print(json.dumps({
        "workload": "dropin_cfg2_rows_qwen3_8b_L4096_contiguous", "value": site_us, "unit": "us/layer",
        "higher_is_better": False, "rows": bsz, "row_len": lb, "queries": bsz * lb, "layers": nl,
        "call_site_us": site_us, "single_prefill_us": prefill_us, "runner_us": runner_us,
        "note": "eager, as verification.py:137-165 runs it: the call site's transpose copies, "
                "d2sd.single_prefill_with_kv_cache (cascade kernels, a cached plan per 512-key bucket; outputs "
                "and workspace from torch's caching allocator), CascadeGraphRunner.run (one fused local-attention "
                "+ merge launch on the caller's tensors)",
    }), flush=True)
    return 0


def measure_step(args) -> int:
    """One whole verify step captured in one HipGraph and replayed as the cache
    grows: candidate tree built on the device from the draft confidences
    (d3_generator.py:116-180), 36 layers of dynamic-prefix cascade attention
    (verification.py:127-176), the acceptance walk over [nodes, 151936] bf16
    logits (d3_generator.py:204-225) and the commit of the accepted branch into
    the paged cache of every layer (d3_generator.py:227-232).  Synthetic
    logits and drafts, so about one token is accepted per step."""
    import numpy as np
    import torch
    import d2sd
    from d2sd import tree as dtree

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    hq, hkv, d, P, nl, vocab, L0 = 32, 8, 128, 16, args.layers, 151936, 4096
    builder = dtree.D3TreeBuilder(16, 32, 4, dev)
    cap, rows, lb = builder.capacity, builder.rows_cap, builder.block_size_2
    Lmax = L0 + 512
    npages = (Lmax + P - 1) // P
    gen = torch.Generator(device=dev).manual_seed(args.seed + 1)

    def rnd(*shape):
        return torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)

    kp = [rnd(npages, hkv, P, d) for _ in range(nl)]
    vp = [rnd(npages, hkv, P, d) for _ in range(nl)]
    table = torch.randperm(npages, generator=gen, device=dev).to(torch.int32)
    q = [rnd(cap, hq, d) for _ in range(nl)]
    ks = [rnd(cap, hkv, d) for _ in range(nl)]
    vs = [rnd(cap, hkv, d) for _ in range(nl)]
    out = [torch.empty(cap, hq, d, dtype=torch.bfloat16, device=dev) for _ in range(nl)]
    lse = [torch.empty(cap, hq, dtype=torch.float32, device=dev) for _ in range(nl)]
    logits = rnd(cap, vocab)
    drafts = torch.randint(0, vocab, (rows, lb), generator=gen, device=dev)
    conf = torch.from_numpy(np.random.default_rng(args.seed).uniform(0.0, 1.0, size=15)).to(torch.bfloat16).to(dev)

    t0 = time.perf_counter()
    attn = d2sd.CascadeVerifyAttention(dev).plan(
        [0, cap], [Lmax], hq, hkv, d, tree_masks=[np.eye(cap, dtype=bool)], page_size=P, page_indptr=[0, npages],
        page_table=table, kv_layout="HND", dynamic_prefix=True)
    plan_ms = (time.perf_counter() - t0) * 1e3
    attn.set_prefix_len([L0])
    acc = d2sd.TreeAccept(cap, vocab, lb, dev, temperature=args.temperature, seed=args.seed)
    commit = d2sd.PagedKVCommit(kp, vp, ks, vs)

    def tree_part():
        builder.build(conf, tree_mask=attn.tree_mask_dev)

    def attn_part():
        for i in range(nl):
            attn.run(q[i], ks[i], vs[i], kp[i], vp[i], out=out[i], lse=lse[i])

    def accept_part():
        return acc(logits, builder.node_index, drafts)

    def whole():
        tree_part()
        attn_part()
        _, nodes, res = accept_part()
        commit.commit(table, attn.prefix_len_dev[0:1], nodes, num_accepted=lb, num_accepted_dev=res, advance=True)

    graphs = {}
    for key, fn in (("step", whole), ("tree", tree_part), ("attention", attn_part), ("accept", accept_part)):
        tree_part()
        torch.cuda.synchronize()
        graphs[key] = d2sd.HipGraph()
        with graphs[key].capture():
            fn()
    reps = max(10, args.steps // 2)
    for _ in range(args.warmup):
        graphs["step"].replay()
    attn.set_prefix_len([L0])
    torch.cuda.synchronize()
    step_us = _events_us(graphs["step"].replay, reps, torch)
    grown = int(attn.prefix_len_dev[0]) - L0
    attn.set_prefix_len([L0])
    parts = {k: _events_us(graphs[k].replay, reps, torch) for k in ("tree", "attention", "accept")}
    print(json.dumps({
        "workload": "verify_step_cfg2_qwen3_8b_L4096_paged16_36layers_vocab151936", "value": step_us,
        "unit": "us/step", "higher_is_better": False, "layers": nl, "tree_capacity": cap,
        "temperature": args.temperature, "replays": reps, "prefix_growth_tokens": grown,
        "attention_us_per_layer": parts["attention"] / nl, "tree_build_us": parts["tree"],
        "accept_us": parts["accept"],
        "commit_and_rest_us": step_us - parts["tree"] - parts["attention"] - parts["accept"],
        "plan_ms_dynamic_prefix": plan_ms,
        "note": "one hipGraph per step, no host work between steps: the prefix length lives on the device and "
                "the commit advances it; attention planned once for prefix <= %d (a plan for the largest tree)"
                % Lmax,
    }), flush=True)
    return 0


def measure_workload(args) -> int:
    """One JSON line per named workload: µs per verify-attention call (attention
    + merge launch), and the attention launch alone against its roofline
    (HBM or MFMA, whichever bounds its algorithmic bytes / flops)."""
    import torch
    import d2sd
    from d2sd import workloads as wl

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    for name in args.workload.split(","):
        if name == "dropin":
            measure_dropin(args)
            continue
        if name == "dta":
            measure_dta(args)
            continue
        if name == "step":
            measure_step(args)
            continue
        prob, nl = OTHER_WORKLOADS[name](wl, args.seed)
        log(f"materialising {prob.name} ({nl} KV pools)")
        mp = wl.materialize(prob, dev, layers=nl)
        attn = d2sd.CascadeVerifyAttention(dev)
        wl.plan_for(attn, mp)
        info = attn.info
        T, hq, d = prob.total_q, prob.num_qo_heads, prob.head_dim
        outs = [(torch.empty(T, hq, d, dtype=torch.bfloat16, device=dev),
                 torch.empty(T, hq, dtype=torch.float32, device=dev)) for _ in mp.layers]

        def calls(fn):
            for lt, (o, l) in zip(mp.layers, outs):
                fn(lt.q, lt.k_suffix, lt.v_suffix, lt.k_prefix, lt.v_prefix, out=o, lse=l)

        calls(attn.run)
        torch.cuda.synchronize()
        graphs = {}
        for key, fn in (("call", attn.run), ("attention", attn.run_attention)):
            graphs[key] = d2sd.HipGraph()
            with graphs[key].capture():
                calls(fn)
        for _ in range(3):
            graphs["call"].replay()
        reps = max(5, args.kernel_reps // 2)
        call_us = time_graph(graphs["call"], reps, torch) * 1e3 / nl
        attn_us = time_graph(graphs["attention"], reps, torch) * 1e3 / nl
        ab, af = wl.attention_launch_bytes_flops(prob)
        vb, vf = wl.verify_bytes_flops(prob)
        pb, pf = wl.prefix_bytes_flops(prob)
        t_hbm, t_mfma = ab / (HBM_PEAK_GBPS * 1e9), af / (MFMA_BF16_PEAK_TFLOPS * 1e12)
        bound = "mfma" if t_mfma > t_hbm else "hbm"
        hbm = ab / (attn_us * 1e-6) / 1e9
        tfl = af / (attn_us * 1e-6) / 1e12
        print(json.dumps({
            "workload": prob.name, "value": call_us, "unit": "us/call", "higher_is_better": False,
            "queries": T, "requests": len(prob.requests), "kv_pools": nl,
            "dtype": "fp8_e4m3fn kv / bf16" if prob.kv_dtype == torch.float8_e4m3fn else "bf16",
            "attention_us": attn_us, "merge_us": call_us - attn_us,
            "attention_bytes": ab, "attention_flops": af, "bound": bound,
            "hbm_gbps": hbm, "hbm_frac": hbm / HBM_PEAK_GBPS,
            "mfma_tflops": tfl, "mfma_frac": tfl / MFMA_BF16_PEAK_TFLOPS,
            "roofline_floor_us": max(t_hbm, t_mfma) * 1e6,
            "frac": max(t_hbm, t_mfma) / (attn_us * 1e-6),
            "call_bytes": vb, "call_flops": vf, "queries_per_s": T / (call_us * 1e-6),
            # the prefix level's algorithmic bytes / flops over the attention
            # launch, which also runs the suffix level: a lower bound on the
            # prefix level's own fractions
            "prefix_level": {"bytes": pb, "flops": pf, "hbm_frac_lower_bound": pb / (attn_us * 1e-6) / 1e9 /
                             HBM_PEAK_GBPS, "mfma_frac_lower_bound": pf / (attn_us * 1e-6) / 1e12 /
                             MFMA_BF16_PEAK_TFLOPS, "hbm_ceiling": min(1.0, (pb / (HBM_PEAK_GBPS * 1e9)) /
                                                                       max(pb / (HBM_PEAK_GBPS * 1e9),
                                                                           pf / (MFMA_BF16_PEAK_TFLOPS * 1e12)))},
            "plan": {"workgroups": info.num_items, "waves": info.waves_per_block,
                     "splits": info.max_splits_used, "merges": info.num_merges},
            **({"cpu_baseline": cpu_baseline(mp, max(args.cpu_reps, 20), torch, prob.name)}
               if name == "config1" and not args.no_cpu_baseline else {}),
        }), flush=True)
        del graphs, mp, attn, outs
        torch.cuda.empty_cache()
    return 0


def read_traffic():
    """traffic_bytes_per_launch from TRAFFIC_FILE, or None."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed graph replays (verify steps)")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-reps", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--measure-traffic", action="store_true",
                    help="run the two rocprofv3 counter passes and write the traffic summary")
    ap.add_argument("--traffic-workload", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--traffic-config", default="config2", choices=("config2", "config3"),
                    help="workload of --measure-traffic (its summary: profiles/verify_attn_<cfg>_traffic.txt)")
    ap.add_argument("--measure-mix", action="store_true",
                    help="run two rocprofv3 passes of SQ instruction counters and write the instruction-mix summary")
    ap.add_argument("--measure-mfma", action="store_true",
                    help="run one rocprofv3 pass of the SQ MFMA counters and write the utilisation summary")
    ap.add_argument("--commit", action="store_true",
                    help="time the accepted-branch KV commit instead (one JSON line)")
    ap.add_argument("--accepted", type=int, default=20, help="accepted tokens per step for --commit")
    ap.add_argument("--accept", action="store_true",
                    help="time the greedy acceptance walk instead (one JSON line)")
    ap.add_argument("--workload", default=None,
                    help="comma-separated: " + ", ".join(list(OTHER_WORKLOADS) + list(SYSTEM_WORKLOADS)) +
                         " (one JSON line each instead of the verify-step line)")
    ap.add_argument("--temperature", type=float, default=0.0, help="acceptance temperature for --workload step")
    ap.add_argument("--qk-rope", action="store_true",
                    help="time the fused QK RMSNorm + RoPE instead (one JSON line)")
    args = ap.parse_args()
    if args.commit:
        return measure_commit(args)
    if args.accept:
        return measure_accept(args)
    if args.qk_rope:
        return measure_qk_rope(args)
    if args.workload:
        return measure_workload(args)
    if args.traffic_workload:
        return traffic_workload(args)
    if args.measure_traffic:
        return measure_traffic(args)
    if args.measure_mfma:
        return measure_mfma(args)
    if args.measure_mix:
        return measure_mix(args)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every path here runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration).", file=sys.stderr)
        return 2

    import torch
    import d2sd
    from d2sd import workloads as wl

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    prob = wl.config2(args.seed, layers=args.layers)
    log(f"materialising {prob.name}: N={prob.total_q} nodes, {args.layers} layers")
    mp = wl.materialize(prob, dev)
    attn = d2sd.CascadeVerifyAttention(dev)
    wl.plan_for(attn, mp)
    info = attn.info
    T, hq, d = prob.total_q, prob.num_qo_heads, prob.head_dim
    outs = [(torch.empty(T, hq, d, dtype=torch.bfloat16, device=dev),
             torch.empty(T, hq, dtype=torch.float32, device=dev)) for _ in mp.layers]

    def layer_call(i, fn):
        lt = mp.layers[i]
        o, l = outs[i]
        fn(lt.q, lt.k_suffix, lt.v_suffix, lt.k_prefix, lt.v_prefix, out=o, lse=l)

    for i in range(len(mp.layers)):  # eager warm-up
        layer_call(i, attn.run)
    torch.cuda.synchronize()
    step = d2sd.HipGraph()
    with step.capture():
        for i in range(len(mp.layers)):
            layer_call(i, attn.run)
    g_attn = d2sd.HipGraph()
    with g_attn.capture():
        for i in range(len(mp.layers)):
            layer_call(i, attn.run_attention)
    g_merge = d2sd.HipGraph()
    with g_merge.capture():
        for i in range(len(mp.layers)):
            layer_call(i, attn.run_merge)
    log(f"plan: attention {info.num_items} workgroups x {info.waves_per_block} waves "
        f"({info.rows_per_tile} rows each), {info.max_splits_used} prefix splits, {info.num_slots} partial "
        f"slots, {info.num_merges} merge workgroups")

    for _ in range(args.warmup):
        step.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(args.steps):
        step.replay(s)
    e1.record(s)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    us_layer = ms_per_step * 1000.0 / len(mp.layers)
    log(f"timed {args.steps} steps: {ms_per_step:.4f} ms/step, {us_layer:.3f} us/layer")

    # per-kernel averages (graphs of the 36 launches of one kernel)
    attn_us = time_graph(g_attn, args.kernel_reps, torch) * 1000.0 / len(mp.layers)
    merge_us = time_graph(g_merge, args.kernel_reps, torch) * 1000.0 / len(mp.layers)
    log(f"attention kernel {attn_us:.3f} us/launch, merge kernel {merge_us:.3f} us/launch")

    # host work around the step: plan() from scratch, a same-shape re-plan
    # into the existing device buffers, and issuing one replay of the step
    def median_us(fn, n):
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append((time.perf_counter() - t0) * 1e6)
        return float(sorted(ts)[n // 2])

    plan_us = median_us(lambda: wl.plan_for(d2sd.CascadeVerifyAttention(dev), mp), 11)
    replan_us = median_us(lambda: wl.plan_for(attn, mp), 11)
    torch.cuda.synchronize()
    replay_us = median_us(step.replay, 21)
    torch.cuda.synchronize()
    log(f"host: plan {plan_us:.0f} us, same-shape re-plan {replan_us:.0f} us, replay issue {replay_us:.1f} us")

    vb, vf = wl.verify_bytes_flops(prob)
    ab, af = wl.attention_launch_bytes_flops(prob)
    # dominant kernel: the attention launch (prefix key chunks + suffix trees),
    # priced at its algorithmic bytes / flops (K/V, Q, page table, tree mask;
    # visible (query, key) pairs)
    t_hbm, t_mfma = ab / (HBM_PEAK_GBPS * 1e9), af / (MFMA_BF16_PEAK_TFLOPS * 1e12)
    if t_mfma > t_hbm:
        achieved = af / (attn_us * 1e-6) / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / MFMA_BF16_PEAK_TFLOPS}
    else:
        achieved = ab / (attn_us * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBPS}
    roof["traffic"] = read_traffic()
    roof["kernel"] = "d2sd::verify_attn_kernel<128, %d, ...> (prefix chunks + suffix trees)" % info.waves_per_block
    roof["kernel_us"] = attn_us
    roof["algorithmic_bytes"] = ab
    roof["algorithmic_flops"] = af
    roof["hbm_gbps"] = ab / (attn_us * 1e-6) / 1e9
    roof["hbm_frac"] = roof["hbm_gbps"] / HBM_PEAK_GBPS
    roof["mfma_frac"] = af / (attn_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS

    layer_gbps = vb / (us_layer * 1e-6) / 1e9
    result = {
        "metric": METRIC,
        "value": us_layer,
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: Q/K/V ~ N(0,1) rounded to bf16, seeded; tree from seeded DFlash confidences",
        "config": {"workload": prob.name, "layers": len(mp.layers), "prefix_len": 4096, "page_size": 16,
                   "tree_nodes": T, "tree_rows": 5, "row_len": 32, "num_qo_heads": hq, "num_kv_heads": 8,
                   "head_dim": d, "replay": "hipGraph of 36 x (attention launch + merge launch)"},
        "queries_per_s": T / (us_layer * 1e-6),
        "hbm_gbps": layer_gbps,
        "hbm_frac": layer_gbps / HBM_PEAK_GBPS,
        "mfma_frac": vf / (us_layer * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "roofline_floor_us": max(vb / (HBM_PEAK_GBPS * 1e9), vf / (MFMA_BF16_PEAK_TFLOPS * 1e12)) * 1e6,
        "layer_bytes": vb,
        "layer_flops": vf,
        "kernels_us": {"attention": attn_us, "merge": merge_us},
        "roofline": roof,
        "host_us": {"plan": plan_us, "replan_same_shape": replan_us, "step_replay_issue": replay_us,
                    "note": "outside the timed region; with a dynamic-prefix plan no host work runs per step"},
    }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (oracle, fp32 torch sdpa): config 2 layer 0, then config 1")
        result["cpu_baseline"] = cpu_baseline(mp, args.cpu_reps, torch, "config 2 layer 0 of 36")
        mp1 = wl.materialize(wl.config1(args.seed), dev, layers=1)
        result["cpu_baseline_config1"] = cpu_baseline(mp1, max(args.cpu_reps, 20), torch, "config 1")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
