"""Benchmark of the causal GQA FlashAttention hot path on one MI355X.

One step = forward + backward of the attention op on one batch of the workload:
``ttfa_fwd`` then ``ttfa_bwd_dq`` then ``ttfa_bwd_dkdv`` (the three launches
``ttfa_fwd`` + ``ttfa_bwd`` make in bf16), or ``ttfa_fwd`` then ``ttfa_bwd`` for fp32,
whose backward is one launch, called through the C ABI on preallocated device buffers
on torch's current stream.  The default workload is C2, the 112M pretrain
attention shape (B=16, Hq=Hkv=12, T=1024, D=64, bf16), the configuration the headline
metric is quoted on.

FLOPs follow the FlashAttention convention with the causal half counted:
fwd = 2*B*Hq*T^2*D, bwd = 2.5*fwd, step = 3.5*fwd.

Inputs rotate over several resident sets (more than 512 MB in total) so the 256 MB
last-level cache does not hold one step's operands from the previous step.

Prints ONE JSON line on stdout.  ``--gpus`` above 1 is refused: this build runs on one
GPU, and the attention op needs no collective (each (batch, kv-head) is independent).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk
PEAK_F32_TFLOPS = 157.3     # MI355X dense fp32 matrix
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def _cpu_model() -> str:
    """Host CPU model: lscpu's "Model name" (with family/model/stepping when the name is
    generic, as on virtualised hosts), else /proc/cpuinfo."""
    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if ":" in line:
                key, val = line.split(":", 1)
                fields[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    name = fields.get("Model name", "")
    if not name:
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    name = name or platform.processor() or "unknown"
    ids = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if k in fields]
    sockets = fields.get("Socket(s)")
    extra = ", ".join(ids + ([f"{sockets} socket(s)"] if sockets else []))
    return f"{name} ({extra})" if extra else name


def _cpu_threads() -> tuple[int, int, str]:
    """(threads to use, logical CPUs visible, why).  All visible CPUs, unless
    OMP_NUM_THREADS names fewer: a GPU host that shares its cores between GPUs states each
    GPU's share there (16 per GPU on the MI355X boxes this runs on)."""
    visible = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and 0 < int(omp) < visible:
        return int(omp), visible, f"OMP_NUM_THREADS={omp} (this GPU's share of the host)"
    return visible, visible, "all visible logical CPUs"


def _cpu_baseline(cfg, budget_s: float) -> dict:
    """Oracle (repeat_interleave + SDPA, fp32, fwd + autograd bwd) on the host CPU.

    Runs on leading batch slices of the same seeded workload; the slice size is
    chosen so one repetition takes about a second, and repetitions continue until
    ``budget_s`` seconds of CPU work have been spent (at least 3).
    """
    import torch

    from oracle.eager_attention import eager_attention, eager_attention_grads
    from tinytrain_amd.workloads import make_inputs

    threads, visible, why = _cpu_threads()
    torch.set_num_threads(threads)
    q, k, v, do, _ = make_inputs(cfg, seed=0)

    def run(b: int) -> float:
        t0 = time.perf_counter()
        eager_attention_grads(q[:b], k[:b], v[:b], do[:b])
        return time.perf_counter() - t0

    run(1)  # warmup
    backend = "unknown"
    try:  # which SDPA kernel the CPU build dispatches to (profiler op names)
        from torch.profiler import ProfilerActivity, profile
        with profile(activities=[ProfilerActivity.CPU]) as prof:
            run(1)
        names = {e.key for e in prof.key_averages()}
        hits = sorted(n for n in names if "scaled_dot_product" in n or "_flash_attention" in n)
        backend = ", ".join(hits) if hits else "math (no fused SDPA op)"
    except Exception as exc:  # profiler unavailable: report, do not fail the baseline
        backend = f"unknown ({type(exc).__name__})"
    t1 = run(1)
    b = max(1, min(cfg.B, int(1.0 / max(t1, 1e-6))))
    times, spent = [], 0.0
    while spent < 0.75 * budget_s or len(times) < 3:
        t = run(b)
        times.append(t)
        spent += t
        if len(times) >= 400:
            break
    med = statistics.median(times)
    # forward alone (no autograd graph), same slice, the rest of the budget
    ftimes, fspent = [], 0.0
    with torch.no_grad():
        while fspent < 0.25 * budget_s or len(ftimes) < 3:
            t0 = time.perf_counter()
            eager_attention(q[:b], k[:b], v[:b])
            ftimes.append(time.perf_counter() - t0)
            fspent += ftimes[-1]
            if len(ftimes) >= 400:
                break
    fmed = statistics.median(ftimes)
    flop = 3.5 * cfg.fwd_flop() * b / cfg.B
    return {
        "value": round(flop / med / 1e12, 5),
        "forward_tflops": round(cfg.fwd_flop() * b / cfg.B / fmed / 1e12, 5),
        "seconds_full_workload": {"fwd": round(fmed * cfg.B / b, 4),
                                  "fwd_bwd": round(med * cfg.B / b, 4)},
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{cfg.name} batch slice b={b} of B={cfg.B} (same seeded inputs), fp32 "
                   f"repeat_interleave + causal SDPA forward + autograd backward on the CPU, "
                   f"median of {len(times)} runs ({spent:.1f} s of CPU work); forward alone "
                   f"(no grad) median of {len(ftimes)} runs ({fspent:.1f} s)"),
        "seconds_per_sample": round(med, 4),
        "cpu_model": _cpu_model(),
        "logical_cpus_visible": visible,
        "threads_rule": why,
        "torch_threads": torch.get_num_threads(),
        "sdpa_cpu_ops": backend,
    }


def _gemm_reference(dev, n: int = 8192, steps: int = 30) -> dict:
    """Measured bf16 GEMM throughput (torch.matmul -> hipBLASLt, fp32 accumulate) on an
    n x n x n problem: the practical matrix-core ceiling the attention numbers are also
    compared against."""
    import torch

    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    for _ in range(5):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    evs = [(HipTimingEvent(), HipTimingEvent()) for _ in range(steps)]
    for e0, e1 in evs:
        e0.record(stream)
        torch.matmul(a, b)
        e1.record(stream)
    torch.cuda.synchronize()
    ms = statistics.median(e0.elapsed_time(e1) for e0, e1 in evs)
    return {"shape": [n, n, n], "library": "torch.matmul (hipBLASLt), bf16 in, fp32 accumulate",
            "median_ms": round(ms, 4), "tflops": round(2 * n ** 3 / (ms * 1e-3) / 1e12, 1)}


TRAFFIC_DIR = ROOT / "profiles"


def _traffic_file(config: str) -> Path:
    return TRAFFIC_DIR / f"hbm_traffic_{config}.txt"


def _pmc_pass(counter: str, cmd: list, out_dir: Path) -> dict:
    """One ``rocprofv3 --pmc <counter>`` pass over ``cmd`` (a child process); returns
    {kernel symbol: mean counter value per dispatch (KiB)}."""
    return {k: v[counter] for k, v in _pmc_multi([counter], cmd, out_dir).items() if counter in v}


def _pmc_multi(counters: list, cmd: list, out_dir: Path) -> dict:
    """One ``rocprofv3 --pmc c1 c2 ...`` pass over ``cmd`` (a child process); returns
    {kernel name: {counter: mean value per dispatch}}.  The counters must fit one pass
    (at most 8 SQ, 4 TCC, 2 GRBM counters)."""
    import csv
    import subprocess

    out_dir.mkdir(parents=True, exist_ok=True)
    full = ["rocprofv3", "--pmc", *counters, "-d", str(out_dir), "-o", "run",
            "--output-format", "csv", "--", sys.executable, *cmd]
    print("[traffic] " + " ".join(full), file=sys.stderr, flush=True)
    with open(out_dir / "rocprofv3.log", "w") as log:
        subprocess.run(full, check=True, timeout=180, stdout=log, stderr=subprocess.STDOUT,
                       cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"})
    sums: dict = {}
    for path in out_dir.rglob("*counter_collection.csv"):
        for row in csv.DictReader(open(path)):
            if row["Counter_Name"] not in counters:
                continue
            key = (row["Kernel_Name"], row["Counter_Name"])
            tot, n = sums.get(key, (0.0, 0))
            sums[key] = (tot + float(row["Counter_Value"]), n + 1)
    res: dict = {}
    for (name, ctr), (tot, n) in sums.items():
        res.setdefault(name, {})[ctr] = tot / n
    return res


# Two passes of SQ counters (8 SQ + 1 GRBM each): matrix-core and vector-ALU activity,
# LDS bank conflicts.
SQ_PASSES = (
    ("SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU",
     "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_ACTIVE_INST_VALU", "GRBM_GUI_ACTIVE"),
    ("SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_WAIT_INST_LDS", "SQ_WAIT_INST_ANY",
     "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_ANY", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_INSTS_SALU",
     "GRBM_GUI_ACTIVE"),
)


def _measure_sq(config: str, out: Path) -> int:
    """MFMA-busy, VALU, co-execution and LDS bank-conflict counters per attention kernel
    on ``config`` (two rocprofv3 --pmc passes), summarised per kernel."""
    me = str(ROOT / "bench.py")
    work = ["--config", config, "--steps", "10", "--warmup", "2", "--cpu-budget", "0",
            "--settle-ms", "0", "--no-traffic", "--no-extras"]
    tmp = Path("/tmp") / f"ttfa_sq_{os.getpid()}"
    merged: dict = {}
    for i, ctrs in enumerate(SQ_PASSES):
        for name, vals in _pmc_multi(list(ctrs), [me, *work], tmp / f"pass{i}").items():
            if "ttfa::" not in name:
                continue
            sym = name.split("ttfa::", 1)[1].split("(", 1)[0]
            d = merged.setdefault(sym, {})
            for c, v in vals.items():
                d[c if c != "GRBM_GUI_ACTIVE" else f"GRBM_GUI_ACTIVE_{i}"] = v
    simds, xcds = 1024, 8  # MI355X: 256 CUs x 4 SIMDs; GRBM_GUI_ACTIVE sums the 8 XCDs
    rows, summary = [], {}
    for sym, c in sorted(merged.items()):
        gui = c.get("GRBM_GUI_ACTIVE_0", float("nan")) / xcds
        waves = max(c.get("SQ_WAVES", 1.0), 1.0)
        r = {
            "mfma_busy": c["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * simds),
            "valu_mfma_coexec": c["SQ_VALU_MFMA_COEXEC_CYCLES"] / (gui * simds),
            "lds_bank_conflict_per_active": c["SQ_LDS_BANK_CONFLICT"] / max(c["SQ_LDS_IDX_ACTIVE"], 1.0),
            "lds_active": c["SQ_LDS_IDX_ACTIVE"] / (gui * simds / 4),
            "wait_lds_frac": c["SQ_WAIT_INST_LDS"] / max(c["SQ_WAVE_CYCLES"], 1.0),
            "valu_insts_per_wave": c["SQ_INSTS_VALU"] / waves,
            "mfma_insts_per_wave": c["SQ_INSTS_MFMA"] / waves,
            "lds_insts_per_wave": c["SQ_INSTS_LDS"] / waves,
            "salu_insts_per_wave": c["SQ_INSTS_SALU"] / waves,
            "wait_inst_any_frac": c["SQ_WAIT_INST_ANY"] / max(c["SQ_WAVE_CYCLES"], 1.0),
            "waves": waves,
        }
        summary[sym] = {k: round(v, 4) for k, v in r.items()}
        rows.append(f"{sym:<32}{r['mfma_busy']:>9.3f}{r['valu_mfma_coexec']:>9.3f}"
                    f"{r['lds_bank_conflict_per_active']:>9.3f}{r['valu_insts_per_wave']:>9.0f}"
                    f"{r['mfma_insts_per_wave']:>7.0f}{r['lds_insts_per_wave']:>7.0f}"
                    f"{r['salu_insts_per_wave']:>7.0f}{r['wait_inst_any_frac']:>8.3f}"
                    f"{r['lds_active']:>8.3f}{r['wait_lds_frac']:>8.3f}")
    lines = [
        f"# SQ activity per attention kernel, workload {config} (rocprofv3 --pmc, two passes)",
        "# command: python bench.py --measure-sq --config " + config,
        "# passes:  rocprofv3 --pmc " + " ".join(SQ_PASSES[0]) + " -- python bench.py " + " ".join(work),
        "#          rocprofv3 --pmc " + " ".join(SQ_PASSES[1]) + " -- python bench.py " + " ".join(work),
        "# mfma = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE/8 x 1024 SIMDs): matrix-core busy share",
        "# coex = SQ_VALU_MFMA_COEXEC_CYCLES on the same base: cycles a VALU op issued under a busy MFMA",
        "# bank = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE: LDS cycles lost to bank conflicts per active cycle",
        "# per-wave instruction counts; wait = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES",
        "# lds = SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE/8 x 256 CUs): share of cycles the CU's LDS works on",
        "#   indexed accesses; wlds = SQ_WAIT_INST_LDS / SQ_WAVE_CYCLES",
        f"{'kernel':<32}{'mfma':>9}{'coex':>9}{'bank':>9}{'VALU/w':>9}{'MFMA':>7}{'LDS':>7}{'SALU':>7}{'wait':>8}"
        f"{'lds':>8}{'wlds':>8}",
        *rows,
        "JSON " + json.dumps({"config": config, "kernels": summary}),
    ]
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text("\n".join(lines) + "\n")
    print("\n".join(lines), flush=True)
    return 0


# Two passes of memory-path counters (each within one pass's limits: at most 4 TCC,
# 4 TCP, 2 TA, 2 TD, 2 GRBM).  TCC is the L2 of an XCD, TCP the CU's vector L1, TA/TD
# its address and data units.
L2_PASSES = (
    ("TCC_HIT", "TCC_MISS", "TCC_EA0_RDREQ", "TCC_EA0_RDREQ_DRAM", "GRBM_GUI_ACTIVE"),
    ("TA_TA_BUSY", "TA_ADDR_STALLED_BY_TC_CYCLES", "TCP_PENDING_STALL_CYCLES",
     "TCP_TCC_READ_REQ", "TCP_TCC_READ_REQ_LATENCY", "TD_TD_BUSY", "TD_TC_STALL",
     "GRBM_GUI_ACTIVE"),
)


def _measure_l2(config: str, out: Path) -> int:
    """L2 hit rate, L2 read latency and the CU memory pipeline's busy / stall shares per
    attention kernel on ``config`` (two rocprofv3 --pmc passes), summarised per kernel."""
    me = str(ROOT / "bench.py")
    work = ["--config", config, "--steps", "10", "--warmup", "2", "--cpu-budget", "0",
            "--settle-ms", "0", "--no-traffic", "--no-extras"]
    tmp = Path("/tmp") / f"ttfa_l2_{os.getpid()}"
    merged: dict = {}
    for i, ctrs in enumerate(L2_PASSES):
        for name, vals in _pmc_multi(list(ctrs), [me, *work], tmp / f"pass{i}").items():
            if "ttfa::" not in name:
                continue
            sym = name.split("ttfa::", 1)[1].split("(", 1)[0]
            d = merged.setdefault(sym, {})
            for c, v in vals.items():
                d[c if c != "GRBM_GUI_ACTIVE" else f"GRBM_GUI_ACTIVE_{i}"] = v
    cus, xcds = 256, 8  # GRBM_GUI_ACTIVE sums the 8 XCDs; one TA / TD / TCP per CU
    rows, summary = [], {}
    for sym, c in sorted(merged.items()):
        gui0 = c.get("GRBM_GUI_ACTIVE_0", float("nan")) / xcds
        gui1 = c.get("GRBM_GUI_ACTIVE_1", float("nan")) / xcds
        hit, miss = c.get("TCC_HIT", 0.0), c.get("TCC_MISS", 0.0)
        rdreq = max(c.get("TCC_EA0_RDREQ", 0.0), 1.0)
        r = {
            "l2_hit_rate": hit / max(hit + miss, 1.0),
            "l2_requests": hit + miss,
            "ea_read_requests": c.get("TCC_EA0_RDREQ", 0.0),
            "ea_read_dram_share": c.get("TCC_EA0_RDREQ_DRAM", 0.0) / rdreq,
            "l2_read_latency_cycles": c.get("TCP_TCC_READ_REQ_LATENCY", 0.0)
            / max(c.get("TCP_TCC_READ_REQ", 0.0), 1.0),
            "tcp_l2_read_requests": c.get("TCP_TCC_READ_REQ", 0.0),
            "ta_busy": c.get("TA_TA_BUSY", 0.0) / (gui1 * cus),
            "ta_addr_stalled_by_tc": c.get("TA_ADDR_STALLED_BY_TC_CYCLES", 0.0) / (gui1 * cus),
            "tcp_pending_stall": c.get("TCP_PENDING_STALL_CYCLES", 0.0) / (gui1 * cus),
            "td_busy": c.get("TD_TD_BUSY", 0.0) / (gui1 * cus),
            "td_tc_stall": c.get("TD_TC_STALL", 0.0) / (gui1 * cus),
            "gui_cycles_per_xcd": gui0,
        }
        summary[sym] = {k: round(v, 4) for k, v in r.items()}
        rows.append(f"{sym:<34}{r['l2_hit_rate']:>8.3f}{r['ea_read_dram_share']:>8.3f}"
                    f"{r['l2_read_latency_cycles']:>9.0f}{r['ta_busy']:>8.3f}"
                    f"{r['ta_addr_stalled_by_tc']:>9.3f}{r['tcp_pending_stall']:>9.3f}"
                    f"{r['td_busy']:>8.3f}{r['td_tc_stall']:>8.3f}")
    lines = [
        f"# L2 and CU memory-pipeline counters per attention kernel, workload {config} "
        "(rocprofv3 --pmc, two passes)",
        "# command: python bench.py --measure-l2 --config " + config,
        "# passes:  rocprofv3 --pmc " + " ".join(L2_PASSES[0]) + " -- python bench.py " + " ".join(work),
        "#          rocprofv3 --pmc " + " ".join(L2_PASSES[1]) + " -- python bench.py " + " ".join(work),
        "# hit  = TCC_HIT / (TCC_HIT + TCC_MISS): L2 hit rate over all L2 requests",
        "# dram = TCC_EA0_RDREQ_DRAM / TCC_EA0_RDREQ: share of L2 read misses sent to DRAM",
        "# lat  = TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ: mean L2 read latency seen by a CU (cycles)",
        "# ta, ta_tc, tcp_p, td, td_tc: TA_TA_BUSY, TA_ADDR_STALLED_BY_TC_CYCLES, "
        "TCP_PENDING_STALL_CYCLES, TD_TD_BUSY, TD_TC_STALL",
        "#   per CU, as shares of GRBM_GUI_ACTIVE / 8 (cycles per XCD)",
        f"{'kernel':<34}{'hit':>8}{'dram':>8}{'lat':>9}{'ta':>8}{'ta_tc':>9}{'tcp_p':>9}{'td':>8}{'td_tc':>8}",
        *rows,
        "JSON " + json.dumps({"config": config, "kernels": summary}),
    ]
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text("\n".join(lines) + "\n")
    print("\n".join(lines), flush=True)
    return 0


# bench.py's symbol stems -> the key of its per-kernel event average in the JSON line
_EVENT_KEYS = (("fa_fwd_", ("passes", "fwd", "ms")), ("fa_bwd_dq_", ("passes", "bwd_dq_ms")),
               ("fa_bwd_dkdv_", ("passes", "bwd_dkdv_ms")), ("fa_bwd_f32_", ("passes", "bwd", "ms")))


def _measure_kernels(config: str, out: Path) -> int:
    """rocprofv3 --kernel-trace --stats over one default bench run of ``config`` (a child
    process): rocprofv3's per-kernel statistics, and the kernel-trace average over the
    run's per-kernel breakdown steps next to bench.py's own event average for the same
    launches."""
    import csv
    import statistics
    import subprocess

    me = str(ROOT / "bench.py")
    work = ["--config", config, "--cpu-budget", "0"]
    tmp = Path("/tmp") / f"ttfa_kt_{os.getpid()}"
    tmp.mkdir(parents=True, exist_ok=True)
    full = ["rocprofv3", "--kernel-trace", "--stats", "-d", str(tmp), "-o", "run",
            "--output-format", "csv", "--", sys.executable, me, *work]
    print("[kernels] " + " ".join(full), file=sys.stderr, flush=True)
    log_path = tmp / "bench.log"
    with open(log_path, "w") as log:
        rc = subprocess.run(full, timeout=900, stdout=log, stderr=subprocess.STDOUT, cwd="/tmp",
                            env={**os.environ, "TMPDIR": "/tmp"}).returncode
    line = None
    for text in open(log_path):
        if text.startswith("{"):
            line = json.loads(text)
    stats = sorted(tmp.rglob("*kernel_stats.csv"))
    traces = sorted(tmp.rglob("*kernel_trace.csv"))
    if line is None or not stats or not traces:
        print(f"[kernels] rocprofv3 exited {rc} without a bench line or its csv files; "
              f"see {log_path}", file=sys.stderr)
        return 1
    steps, warmup = line["steps"], line["warmup"]
    warmup += (line.get("settle") or {}).get("steps", 0)  # settle steps precede the warmup
    durs: dict = {}
    for row in sorted(csv.DictReader(open(traces[0])), key=lambda r: int(r["Start_Timestamp"])):
        name = row["Kernel_Name"]
        if "ttfa::" not in name:
            continue
        sym = name.split("ttfa::", 1)[1].split("(", 1)[0]
        durs.setdefault(sym, []).append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    c = line["config"]
    desc = (f"B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} T={c['T']} D={c['D']} {line['dtype']}")
    lines = [
        f"# rocprofv3 kernel-trace statistics, workload {config} ({desc}), 1x MI355X",
        f"# command: python bench.py --measure-kernels --config {config}",
        "# which runs: cd /tmp && TMPDIR=/tmp rocprofv3 --kernel-trace --stats -d <out> -o run "
        f"--output-format csv -- python bench.py {' '.join(work)}",
        f"# Dispatches per kernel: {warmup} settle + warmup + {steps} timed steps (no event between "
        f"launches) + {steps} breakdown steps (timing-only HIP events between launches) + "
        "hot-cache and graph-replay launches.",
        "# 'Calls'/'AverageNs' below are rocprofv3's own statistics over all of them.",
        "",
    ]
    for row in csv.reader(open(stats[0])):
        if row[0] == "Name" or "ttfa::" in row[0]:
            lines.append(",".join(f'"{x}"' if i == 0 else x for i, x in enumerate(row)))
    lines += [
        "",
        f"# Breakdown steps (dispatches {warmup + steps + 1}-{warmup + 2 * steps} of each kernel, "
        "rotated input sets) from the kernel trace,",
        "# against bench.py's event averages for the same launches in the same run:",
        f"{'kernel':36s} {'rocprof avg us':>15s} {'bench events us':>16s}  difference",
    ]
    summary = {}
    for sym, d in durs.items():
        window = d[warmup + steps:warmup + 2 * steps]
        keys = next((k for stem, k in _EVENT_KEYS if sym.startswith(stem)), None)
        if not window or keys is None:
            continue
        ev = line
        for k in keys:
            ev = ev[k]
        avg = statistics.mean(window)
        summary[sym] = {"rocprof_avg_us": round(avg, 3), "bench_event_us": round(ev * 1e3, 3)}
        lines.append(f"{sym:36s} {avg:15.2f} {ev * 1e3:16.2f}  {100 * (ev * 1e3 / avg - 1):+.1f}%")
    r = line["roofline"]
    dom = next((sym for sym in durs if sym == r["kernel"]), None)
    if dom is not None:
        timed = durs[dom][warmup:warmup + steps]
        if timed:
            a = statistics.mean(timed)
            summary["roofline_kernel"] = {"kernel": dom, "rocprof_avg_us_timed_steps": round(a, 3),
                                          "bench_avg_launch_us": round(r["avg_launch_ms"] * 1e3, 3)}
            lines += [
                "# The roofline kernel inside the timed steps (no event between launches), against",
                "# bench.py's avg_launch_ms (its breakdown-step event average less the event gap,",
                f"# {r.get('event_gap_ms', 0) * 1e3:.2f} us in this run), the roofline's kernel time:",
                f"{dom:36s} {a:15.2f} {r['avg_launch_ms'] * 1e3:16.2f}  "
                f"{100 * (r['avg_launch_ms'] * 1e3 / a - 1):+.1f}%",
            ]
    g = line.get("graph_replay") or {}
    lines += [
        "# The events time launch to launch on the stream, so they include the dispatch gap between",
        "# back-to-back kernels (a few microseconds); rocprofv3 times the kernel alone.",
        f"# bench.py in this run (under the profiler): value {line['value']} TFLOP/s, ms_per_step "
        f"{line['ms_per_step']}, graph-replay ms_per_step {g.get('ms_per_step')}, roofline "
        f"{r['kernel']} achieved {r['achieved']} TFLOP/s ({r['frac']})",
        "JSON " + json.dumps({"config": config, "kernels": summary, "bench": {
            k: line[k] for k in ("value", "ms_per_step", "passes", "roofline", "graph_replay")}}),
    ]
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text("\n".join(lines) + "\n")
    print("\n".join(lines), flush=True)
    if rc != 0:  # rocprofv3 can exit non-zero after the program's complete run
        print(f"[kernels] rocprofv3 exited {rc} after a complete bench run", file=sys.stderr)
    return 0


def _measure_traffic(config: str, out: Path) -> int:
    """FETCH_SIZE and WRITE_SIZE per dispatch of each attention kernel on ``config``,
    scaled by what the same counters read for a plain 256 MB device copy."""
    me = str(ROOT / "bench.py")
    work = ["--config", config, "--steps", "10", "--warmup", "2", "--cpu-budget", "0",
            "--settle-ms", "0", "--no-traffic", "--no-extras"]
    copy_mb = 256.0
    copy = ["--copy-probe-mb", str(copy_mb), "--steps", "10"]
    tmp = Path("/tmp") / f"ttfa_traffic_{os.getpid()}"
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        res[counter] = _pmc_pass(counter, [me, *work], tmp / f"{counter}_work")
        res[counter + "_copy"] = _pmc_pass(counter, [me, *copy], tmp / f"{counter}_copy")
    copy_kib = int(copy_mb * 1e6) // 16 * 16 / 1024.0

    def copy_factor(counter):
        vals = [v for k, v in res[counter + "_copy"].items() if "copyBuffer" in k or "copy" in k.lower()]
        return copy_kib / max(vals) if vals else float("nan")

    fr, fw = copy_factor("FETCH_SIZE"), copy_factor("WRITE_SIZE")
    kernels = {}
    for name, kib in res["FETCH_SIZE"].items():
        if "ttfa::" not in name:
            continue
        sym = name.split("ttfa::", 1)[1].split("(", 1)[0]
        wk = res["WRITE_SIZE"].get(name, float("nan"))
        kernels[sym] = {"fetch_kib_raw": round(kib, 1), "write_kib_raw": round(wk, 1),
                        "read_bytes": round(kib * fr * 1024), "write_bytes": round(wk * fw * 1024),
                        "traffic_bytes": round((kib * fr + wk * fw) * 1024)}
    summary = {"config": config, "fetch_scale": round(fr, 4), "write_scale": round(fw, 4),
               "copy_probe_bytes": copy_kib * 1024, "kernels": kernels}
    lines = [
        f"# HBM traffic per dispatch, workload {config} (rocprofv3 --pmc, one counter per pass)",
        "# command: python bench.py --measure-traffic --config " + config,
        f"# passes: rocprofv3 --pmc FETCH_SIZE|WRITE_SIZE -- python bench.py {' '.join(work)}",
        f"#         rocprofv3 --pmc FETCH_SIZE|WRITE_SIZE -- python bench.py {' '.join(copy)}",
        f"# calibration: a {copy_mb:.0f} MB device copy reads FETCH_SIZE x{fr:.3f} and "
        f"WRITE_SIZE x{fw:.3f} of its true size;",
        "# read/write bytes below are the raw KiB scaled by those factors.",
        f"{'kernel':<34}{'FETCH KiB':>12}{'WRITE KiB':>12}{'read MB':>10}{'write MB':>10}",
    ]
    for sym, r in sorted(kernels.items()):
        lines.append(f"{sym:<34}{r['fetch_kib_raw']:>12.1f}{r['write_kib_raw']:>12.1f}"
                     f"{r['read_bytes'] / 1e6:>10.2f}{r['write_bytes'] / 1e6:>10.2f}")
    lines.append("JSON " + json.dumps(summary))
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text("\n".join(lines) + "\n")
    print("\n".join(lines), flush=True)
    return 0


def _load_traffic(config: str, kernel: str):
    """Bytes per launch of ``kernel`` from the committed PMC summary, or None."""
    path = _traffic_file(config)
    if not path.exists():
        return None, None
    for line in path.read_text().splitlines():
        if line.startswith("JSON "):
            rec = json.loads(line[5:]).get("kernels", {}).get(kernel)
            if rec:
                return rec["traffic_bytes"], str(path.relative_to(ROOT))
    return None, None


def _copy_probe(mb: float, steps: int, dev) -> int:
    """A plain copy of known size: each launch reads and writes exactly ``mb`` MB."""
    import torch

    n = int(mb * 1e6) // 16 * 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"copy_probe_bytes": src.nbytes, "steps": steps,
                      "GB_per_s_read_plus_write": round(2 * src.nbytes / dt / 1e9, 1)}), flush=True)
    return 0


class HipTimingEvent:
    """A HIP event for timing only, recorded on a given stream: created with
    hipEventDisableSystemFence, so its completion carries no system-scope release.  On
    MI355X a default event (torch.cuda.Event) recorded between two launches adds a few
    microseconds to their span; this one adds about half of that.  Same record /
    elapsed_time interface as torch.cuda.Event."""

    _hip = None
    FLAGS = 0x20000000  # hipEventDisableSystemFence (hip_runtime_api.h)

    @classmethod
    def _lib(cls):
        if cls._hip is None:
            import ctypes

            h = ctypes.CDLL("libamdhip64.so")
            h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                              ctypes.c_void_p]
            h.hipEventDestroy.argtypes = [ctypes.c_void_p]
            cls._hip = h
        return cls._hip

    def __init__(self):
        import ctypes

        self._e = ctypes.c_void_p()
        if self._lib().hipEventCreateWithFlags(ctypes.byref(self._e), self.FLAGS) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")

    def record(self, stream):
        if self._lib().hipEventRecord(self._e, stream.cuda_stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_time(self, other) -> float:
        import ctypes

        ms = ctypes.c_float()
        if self._lib().hipEventElapsedTime(ctypes.byref(ms), self._e, other._e) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def __del__(self):
        if self._e and self._hip is not None:
            self._hip.hipEventDestroy(self._e)


def _settle(fn, ms: float) -> dict:
    """Untimed calls of ``fn`` in chunks of 8 until ``ms`` of wall time has passed, so the
    timed calls that follow run at the clocks a loaded GPU settles to (as the main bench's
    settle phase); returns the ``settle`` field of the line."""
    import torch

    n, t0 = 0, time.perf_counter()
    while ms > 0 and (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            fn()
        n += 8
        torch.cuda.synchronize()
    return {"calls": n, "seconds": round(time.perf_counter() - t0, 3)}


def _ev_time(fn, steps: int, warmup: int) -> float:
    """Median ms of ``fn`` over ``steps`` calls (timing-only HIP events on the current
    stream around each call)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(HipTimingEvent(), HipTimingEvent()) for _ in range(steps)]
    for e0, e1 in evs:
        e0.record(stream)
        fn()
        e1.record(stream)
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in evs)


def _prologue_bench(dev, steps: int, warmup: int, settle_ms: float = 0.0) -> int:
    """Fused q/k norm + RoPE + layout op vs the eager expressions it replaces
    (model.py:83-93), forward and backward, at the reference model's attention inputs
    (B=32, T=512, Hq=8, Hkv=2, D=128, bf16).  The op is HBM-bound: its roofline is the
    bytes it must move over 8 TB/s."""
    import torch

    from tinytrain_amd.attention import apply_rope, precompute_rope
    from tinytrain_amd.kernels.qk_prologue import qk_norm_rope_bwd, qk_norm_rope_fwd

    B, T, Hq, Hkv, D, eps = 32, 512, 8, 2, 128, 1e-6
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, T, Hq, D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(B, T, Hkv, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, Hkv, D, device=dev, generator=g).to(torch.bfloat16)
    wq = torch.ones(D, device=dev) + 0.1 * torch.randn(D, device=dev, generator=g)
    wk = torch.ones(D, device=dev) + 0.1 * torch.randn(D, device=dev, generator=g)
    cos, sin = (t.to(dev) for t in precompute_rope(D, T, 1e6))
    gq = torch.randn(B, Hq, T, D, device=dev, generator=g).to(torch.bfloat16)
    gk = torch.randn(B, Hkv, T, D, device=dev, generator=g).to(torch.bfloat16)

    out = qk_norm_rope_fwd(q, k, v, wq, wk, cos, sin, eps)
    rq, rk = out[3], out[4]
    settle = _settle(lambda: (qk_norm_rope_fwd(q, k, v, wq, wk, cos, sin, eps),
                              qk_norm_rope_bwd(gq, gk, gk, q, k, wq, wk, cos, sin, rq, rk)),
                     settle_ms)
    op_fwd = _ev_time(lambda: qk_norm_rope_fwd(q, k, v, wq, wk, cos, sin, eps), steps, warmup)
    op_bwd = _ev_time(lambda: qk_norm_rope_bwd(gq, gk, gk, q, k, wq, wk, cos, sin, rq, rk),
                      steps, warmup)
    # the C ABI alone (tables already bf16, outputs preallocated): the kernels' time
    from tinytrain_amd import _lib

    lib = _lib.load()
    cb, sb = cos.to(torch.bfloat16).contiguous(), sin.to(torch.bfloat16).contiguous()
    qo, ko, vo = (torch.empty_like(t) for t in out[:3])
    dqr, dkr, dvr = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dwq, dwk = torch.empty_like(wq), torch.empty_like(wk)
    ws = torch.empty(lib.ttfa_qk_prologue_workspace_bytes(B, T, Hq, Hkv, D) // 4, device=dev)
    sp = torch.cuda.current_stream(dev).cuda_stream

    def abi_fwd():
        _lib.check(lib.ttfa_qk_prologue_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), wq.data_ptr(), wk.data_ptr(), cb.data_ptr(),
            sb.data_ptr(), qo.data_ptr(), ko.data_ptr(), vo.data_ptr(), rq.data_ptr(),
            rk.data_ptr(), B, T, Hq, Hkv, D, eps, sp))

    def abi_bwd():
        _lib.check(lib.ttfa_qk_prologue_bwd(
            gq.data_ptr(), gk.data_ptr(), gk.data_ptr(), q.data_ptr(), k.data_ptr(),
            wq.data_ptr(), wk.data_ptr(), cb.data_ptr(), sb.data_ptr(), rq.data_ptr(),
            rk.data_ptr(), dqr.data_ptr(), dkr.data_ptr(), dvr.data_ptr(), dwq.data_ptr(),
            dwk.data_ptr(), ws.data_ptr(), B, T, Hq, Hkv, D, sp))

    fused_fwd = _ev_time(abi_fwd, steps, warmup)
    fused_bwd = _ev_time(abi_bwd, steps, warmup)

    def norm(x, w):
        xf = x.float()
        return (w * xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)

    def eager(qr, kr, vr, wq_, wk_):
        qn, kn = norm(qr, wq_).transpose(1, 2), norm(kr, wk_).transpose(1, 2)
        c, s_ = cos[:T], sin[:T]
        return (apply_rope(qn, c, s_).contiguous(), apply_rope(kn, c, s_).contiguous(),
                vr.transpose(1, 2).contiguous())

    eager_fwd = _ev_time(lambda: eager(q, k, v, wq, wk), steps, warmup)
    leaves = [t.clone().requires_grad_() for t in (q, k, v, wq, wk)]
    outs = eager(*leaves)

    def eager_bwd():
        torch.autograd.grad(outs, leaves, (gq, gk, gk), retain_graph=True)

    eager_bwd_ms = _ev_time(eager_bwd, steps, warmup)
    rows_q, rows_kv = B * T * Hq, B * T * Hkv
    elems = (rows_q + 2 * rows_kv) * D
    fwd_bytes = 2 * elems * 2 + (rows_q + rows_kv) * 4          # read + write bf16, rstd
    bwd_bytes = 2 * elems * 2 + (rows_q + rows_kv) * D * 2 + (rows_q + rows_kv) * 4
    # bwd: read dq/dk/dv + write the three input grads, re-read q_raw/k_raw, read rstd
    peak = 8000.0
    line = {
        "metric": "fused q/k RMSNorm + RoPE + layout prologue, fwd and bwd",
        "config": {"workload": "reference model attention inputs", "B": B, "T": T, "Hq": Hq,
                   "Hkv": Hkv, "D": D, "dtype": "bf16"},
        "fused": {"fwd_ms": round(fused_fwd, 4), "bwd_ms": round(fused_bwd, 4),
                  "note": "C ABI calls (kernels only; bwd = main pass + weight-gradient sum)"},
        "fused_op": {"fwd_ms": round(op_fwd, 4), "bwd_ms": round(op_bwd, 4),
                     "note": "torch custom op: adds the bf16 table conversion and allocation"},
        "eager_torch": {"fwd_ms": round(eager_fwd, 4), "bwd_ms": round(eager_bwd_ms, 4),
                        "note": "model.py:83-93 expressions: norm, transpose, apply_rope, "
                                ".contiguous(); backward through autograd"},
        "speedup": {"fwd": round(eager_fwd / fused_fwd, 2), "bwd": round(eager_bwd_ms / fused_bwd, 2),
                    "op_fwd": round(eager_fwd / op_fwd, 2), "op_bwd": round(eager_bwd_ms / op_bwd, 2)},
        "roofline": {
            "bound": "hbm", "unit": "GB/s", "peak": peak,
            "fwd": {"bytes": fwd_bytes, "achieved": round(fwd_bytes / fused_fwd / 1e6, 1),
                    "frac": round(fwd_bytes / fused_fwd / 1e6 / peak, 4)},
            "bwd": {"bytes": bwd_bytes, "achieved": round(bwd_bytes / fused_bwd / 1e6, 1),
                    "frac": round(bwd_bytes / fused_bwd / 1e6 / peak, 4)},
        },
        "settle": settle,
    }
    print(json.dumps(line), flush=True)
    return 0


def _varlen_bench(dev, steps: int, warmup: int, settle_ms: float = 0.0) -> int:
    """Packed variable-length causal attention at C2's head shape (Hq = Hkv = 12, D = 64)
    and token count (16 x 1024): seeded lengths 64..2048, fwd and bwd through the C ABI,
    algorithmic FLOPs summed per sequence (2 * Hq * len^2 * D forward, x2.5 backward)."""
    import torch

    from tinytrain_amd import _lib

    Hq = Hkv = 12
    D, total_target = 64, 16 * 1024
    g = torch.Generator().manual_seed(0)
    lens = []
    while sum(lens) < total_target:
        lens.append(int(torch.randint(64, 2049, (1,), generator=g)))
    lens[-1] -= sum(lens) - total_target
    if lens[-1] <= 0:
        lens.pop()
    total = sum(lens)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32, device=dev)
    mk = lambda h: torch.randn(h, total, D, device=dev).to(torch.bfloat16)
    q, k, v, do = mk(Hq), mk(Hkv), mk(Hkv), mk(Hq)
    o, lse = torch.empty_like(q), torch.empty(Hq, total, device=dev)
    delta = torch.empty(Hq, total, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    lib = _lib.load()
    sp = torch.cuda.current_stream(dev).cuda_stream
    scale = 1.0 / math.sqrt(D)
    args = (cu.data_ptr(), len(lens), total, max(lens), Hq, Hkv, D, _lib.TTFA_BF16, scale, sp)

    def fwd():
        _lib.check(lib.ttfa_varlen_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                       lse.data_ptr(), *args))

    def bwd():
        _lib.check(lib.ttfa_varlen_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                       do.data_ptr(), lse.data_ptr(), delta.data_ptr(),
                                       dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), *args))

    fwd()
    settle = _settle(lambda: (fwd(), bwd()), settle_ms)
    f_ms, b_ms = _ev_time(fwd, steps, warmup), _ev_time(bwd, steps, warmup)
    fwd_flop = sum(2.0 * Hq * L * L * D for L in lens)
    line = {
        "metric": "packed varlen causal attention fwd / bwd TFLOP/s (cu_seqlens)",
        "config": {"workload": "C2 heads and token count, seeded lengths 64..2048",
                   "Hq": Hq, "Hkv": Hkv, "D": D, "total_tokens": total, "n_seq": len(lens),
                   "max_seqlen": max(lens), "dtype": "bf16"},
        "fwd": {"ms": round(f_ms, 4), "tflops": round(fwd_flop / f_ms / 1e9, 1)},
        "bwd": {"ms": round(b_ms, 4), "tflops": round(2.5 * fwd_flop / b_ms / 1e9, 1)},
        "fwd_bwd_tflops": round(3.5 * fwd_flop / (f_ms + b_ms) / 1e9, 1),
        "frac_of_peak": round(3.5 * fwd_flop / (f_ms + b_ms) / 1e9 / PEAK_BF16_TFLOPS, 4),
        "settle": settle,
    }
    print(json.dumps(line), flush=True)
    return 0


def _decode_bench(dev, steps: int, warmup: int, settle_ms: float = 0.0) -> int:
    """KV-cache decode (one new token per sequence) at the C4/C5 head shape (Hq 16,
    Hkv 8, D 128): a rollout-sized batch (B 32, caches of 4096) and one long sequence
    (B 1, 16384).  HBM-bound: the roofline is the cache bytes read (K and V of every
    cached key once) over 8 TB/s."""
    import torch

    from tinytrain_amd import _lib

    lib = _lib.load()
    sp = torch.cuda.current_stream(dev).cuda_stream
    out = []
    for B, L in ((32, 4096), (1, 16384), (128, 1024)):
        Hq, Hkv, D, Tq = 16, 8, 128, 1
        q = torch.randn(B, Hq, Tq, D, device=dev).to(torch.bfloat16)
        kc = torch.randn(B, Hkv, L, D, device=dev).to(torch.bfloat16)
        vc = torch.randn(B, Hkv, L, D, device=dev).to(torch.bfloat16)
        lens = torch.full((B,), L, dtype=torch.int32, device=dev)
        o = torch.empty_like(q)
        lse = torch.empty(B, Hq, Tq, device=dev)
        ws = torch.empty(lib.ttfa_decode_workspace_bytes(B, Hq, Hkv, Tq, L, D) // 4 + 4, device=dev)

        def call():
            _lib.check(lib.ttfa_decode_fwd(q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                           lens.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                           ws.data_ptr(), B, Hq, Hkv, Tq, L, D, _lib.TTFA_BF16,
                                           1.0 / math.sqrt(D), sp))

        settle = _settle(call, settle_ms if not out else 0.0)  # once, before the first case
        ms = _ev_time(call, steps, warmup)
        # the same calls back to back, timed as one block: the launches queue ahead of the
        # GPU, so no host time falls between them (per-call events expose it when a call
        # is short)
        stream = torch.cuda.current_stream(dev)
        e0, e1 = HipTimingEvent(), HipTimingEvent()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        ms_b2b = e0.elapsed_time(e1) / steps
        nbytes = 2 * B * Hkv * L * D * 2 + 2 * B * Hq * Tq * D * 2
        out.append({"B": B, "Hq": Hq, "Hkv": Hkv, "D": D, "Tq": Tq, "cache_len": L,
                    "ms": round(ms, 4), "cache_bytes": nbytes,
                    "GB_per_s": round(nbytes / ms / 1e6, 1),
                    "frac_of_hbm_peak": round(nbytes / ms / 1e6 / 8000.0, 4),
                    "ms_back_to_back": round(ms_b2b, 4),
                    "GB_per_s_back_to_back": round(nbytes / ms_b2b / 1e6, 1),
                    "frac_of_hbm_peak_back_to_back": round(nbytes / ms_b2b / 1e6 / 8000.0, 4),
                    **({"settle": settle} if settle["calls"] else {})})
    print(json.dumps({"metric": "KV-cache decode attention, HBM GB/s (split + merge launches)",
                      "roofline": {"bound": "hbm", "peak": 8000.0, "unit": "GB/s"},
                      "timing": "ms: median of timing-only events around each call (includes the "
                                "host time between calls when a call is short); ms_back_to_back: "
                                "the same calls queued back to back, one event pair around all",
                      "cases": out}), flush=True)
    return 0


def _model_bench(dev, steps: int, warmup: int, batch: int) -> int:
    """Whole-model training step (forward, backward, AdamW) of the reference's 112M shape
    under torch.compile, with attn_impl "sdpa" (enable_gqa, the reference's
    "compile + GQA" row, docs/results.md:178) vs "hip" vs "hip" + fused prologue; plus
    the logits of the same weights and tokens under each implementation."""
    import torch

    from tinytrain_amd.model import ModelConfig, ModelForCausalLM

    torch.manual_seed(0)
    c = ModelConfig()
    T = c.max_seq_len
    model = ModelForCausalLM(c).to(dev)
    try:
        opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)
        opt_name = "AdamW (fused)"
    except (RuntimeError, ValueError):
        opt = torch.optim.AdamW(model.parameters(), lr=1e-4)
        opt_name = "AdamW (foreach)"
    tok = torch.randint(0, c.vocab_size, (batch, T + 1), device=dev)
    inp, tgt = tok[:, :-1].contiguous(), tok[:, 1:].contiguous()
    impls = [("sdpa", False, True), ("hip", False, False), ("hip", True, False)]

    # logits of one set of weights under each implementation (eager, no grad)
    logits = {}
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        for name, fused, gqa in impls:
            model.set_attn_impl(name, fused_prologue=fused, enable_gqa=gqa)
            logits[(name, fused)] = model(inp[:4])[0].float()
    ref = logits[("sdpa", False)]
    parity = {f"{n}{'+fused_prologue' if f else ''}": {
        "max_abs_vs_sdpa": round((l - ref).abs().max().item(), 5),
        "mean_abs_vs_sdpa": round((l - ref).abs().mean().item(), 6)}
        for (n, f), l in logits.items() if (n, f) != ("sdpa", False)}

    res = {}
    for name, fused, gqa in impls:
        model.set_attn_impl(name, fused_prologue=fused, enable_gqa=gqa)
        torch._dynamo.reset()
        cm = torch.compile(model)

        def step():
            with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                _, loss = cm(inp, tgt)
            loss.backward()
            opt.step()
            opt.zero_grad(set_to_none=True)

        ms = _ev_time(step, steps, warmup)
        tps = batch * T / (ms * 1e-3)
        key = f"{name}{'+fused_prologue' if fused else ''}"
        res[key] = {"ms_per_step": round(ms, 3), "tokens_per_s": round(tps, 1),
                    "model_tflops": round(c.train_flop_per_token(T) * tps / 1e12, 1)}
        print(f"[model] {key}: {ms:.2f} ms/step, {tps:.0f} tok/s", file=sys.stderr, flush=True)
    base = res["sdpa"]["tokens_per_s"]
    for r in res.values():
        r["vs_sdpa"] = round(r["tokens_per_s"] / base, 3)
    line = {
        "metric": "whole-model training tokens/s, attn_impl hip vs sdpa (torch.compile)",
        "config": {"workload": "reference 112M pretrain shape", "B": batch, "T": T,
                   "hidden": c.hidden_size, "layers": c.num_hidden_layers,
                   "Hq": c.num_attention_heads, "Hkv": c.num_key_value_heads,
                   "D": c.head_dim, "vocab": c.vocab_size, "params": c.params(),
                   "optimizer": opt_name, "dtype": "bf16 autocast",
                   "data": "synthetic tokens (seeded)"},
        "flop_per_token": c.train_flop_per_token(T),
        "results": res,
        "logits_parity": parity,
        "reference_published": {"note": "RTX 4070 Ti Super, docs/results.md:178,184",
                                "compile+GQA sdpa tok/s": 84638, "compile+GQA triton tok/s": 82634},
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=600.0,
                    help="before the warmup, run untimed steps for at least this much wall "
                         "time, so the clocks and power state have reached their loaded "
                         "level whatever --warmup says (reported as 'settle' in the line)")
    ap.add_argument("--config", default="C2",
                    help="workload: C1..C5, or REF112M (the reference model's attention shape); "
                         "default C2")
    ap.add_argument("--sets", type=int, default=0,
                    help="input sets to rotate over (0: enough for > 512 MB)")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU work for the CPU baseline (0 disables it)")
    ap.add_argument("--copy-probe-mb", type=float, default=0.0,
                    help="instead of the workload, run --steps plain device copies of this "
                         "many MB (calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--measure-traffic", action="store_true",
                    help="run rocprofv3 FETCH_SIZE / WRITE_SIZE passes over --config and a "
                         "plain copy, and write the per-kernel HBM traffic summary")
    ap.add_argument("--traffic-out", default="",
                    help="where --measure-traffic writes (default profiles/hbm_traffic_<cfg>.txt)")
    ap.add_argument("--measure-sq", action="store_true",
                    help="run two rocprofv3 SQ-counter passes over --config (MFMA busy, VALU, "
                         "LDS bank conflicts) and write profiles/sq_counters_<cfg>.txt")
    ap.add_argument("--measure-l2", action="store_true",
                    help="run two rocprofv3 passes of L2 / TA / TD / TCP counters over --config "
                         "and write profiles/l2_ta_<cfg>.txt")
    ap.add_argument("--measure-kernels", action="store_true",
                    help="run bench.py --config under rocprofv3 --kernel-trace --stats and "
                         "write profiles/fa_kernels_<cfg>_kernel_stats.txt")
    ap.add_argument("--prologue", action="store_true",
                    help="benchmark the fused q/k norm + RoPE + layout op against the eager "
                         "expressions it replaces (prints its own JSON line)")
    ap.add_argument("--model", action="store_true",
                    help="whole-model training benchmark at the reference 112M shape: "
                         "attn_impl sdpa vs hip vs hip + fused prologue (own JSON line)")
    ap.add_argument("--model-batch", type=int, default=32)
    ap.add_argument("--decode", action="store_true",
                    help="KV-cache decode attention bandwidth at the C4/C5 head shape "
                         "(own JSON line)")
    ap.add_argument("--varlen", action="store_true",
                    help="packed variable-length attention at C2's heads and token count "
                         "(own JSON line)")
    ap.add_argument("--no-traffic", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-extras", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the attention op shards by (batch, kv-head) "
              "with no exchange, and no multi-GPU run is part of this build. Use --gpus 1.",
              file=sys.stderr)
        return 2

    if args.measure_traffic:  # parent never touches the GPU; the passes are children
        out = Path(args.traffic_out) if args.traffic_out else _traffic_file(args.config)
        return _measure_traffic(args.config, out)
    if args.measure_sq:
        return _measure_sq(args.config, TRAFFIC_DIR / f"sq_counters_{args.config}.txt")
    if args.measure_l2:
        return _measure_l2(args.config, TRAFFIC_DIR / f"l2_ta_{args.config}.txt")
    if args.measure_kernels:
        return _measure_kernels(args.config,
                                TRAFFIC_DIR / f"fa_kernels_{args.config}_kernel_stats.txt")

    import torch

    from tinytrain_amd.workloads import CONFIGS, make_inputs
    from tinytrain_amd import _lib

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe_mb > 0:
        return _copy_probe(args.copy_probe_mb, args.steps, dev)
    if args.prologue:
        return _prologue_bench(dev, args.steps, args.warmup, args.settle_ms)
    if args.varlen:
        return _varlen_bench(dev, args.steps, args.warmup, args.settle_ms)
    if args.decode:
        return _decode_bench(dev, args.steps, args.warmup, args.settle_ms)
    if args.model:
        return _model_bench(dev, min(args.steps, 20), min(max(args.warmup, 3), 5),
                            args.model_batch)
    cfg = CONFIGS[args.config]
    lib = _lib.load()
    B, Hq, Hkv, T, D = cfg.B, cfg.Hq, cfg.Hkv, cfg.T, cfg.D
    dt_code = _lib.TTFA_BF16 if cfg.dtype == torch.bfloat16 else _lib.TTFA_F32
    scale = 1.0 / math.sqrt(D)

    q0, k0, v0, do0, _ = make_inputs(cfg, seed=0)
    set_bytes = 2 * (q0.nbytes + do0.nbytes) + 3 * (k0.nbytes + v0.nbytes) + 2 * B * Hq * T * 4
    nsets = args.sets or max(2, math.ceil(512e6 / set_bytes) + 1)
    sets = []
    for i in range(nsets):
        if i == 0:
            q, k, v, do = (t.to(dev) for t in (q0, k0, v0, do0))
        else:  # perturbed copies: same statistics, different bits
            q, k, v, do = (t.to(dev).roll(i, dims=2).contiguous() for t in (q0, k0, v0, do0))
        o = torch.empty_like(q)
        lse = torch.empty((B, Hq, T), device=dev, dtype=torch.float32)
        delta = torch.empty((B * Hq, T), device=dev, dtype=torch.float32)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        sets.append((q, k, v, do, o, lse, delta, dq, dk, dv))
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream

    # fp32: ttfa_bwd is a single launch (both passes), timed as one kernel "bwd".
    one_launch_bwd = cfg.dtype == torch.float32
    kernel_names = ("fwd", "bwd") if one_launch_bwd else ("fwd", "bwd_dq", "bwd_dkdv")

    launch_sp = [sp]  # the stream the launches go to (a capture stream while capturing)

    def launch_one(name, s):
        q, k, v, do, o, lse, delta, dq, dk, dv = s
        if name == "fwd":
            _lib.check(lib.ttfa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                    lse.data_ptr(), B, Hq, Hkv, T, D, dt_code, scale, launch_sp[0]))
        elif name == "bwd":
            _lib.check(lib.ttfa_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                    do.data_ptr(), lse.data_ptr(), delta.data_ptr(), dq.data_ptr(),
                                    dk.data_ptr(), dv.data_ptr(), B, Hq, Hkv, T, D, dt_code, scale,
                                    launch_sp[0]))
        elif name == "bwd_dq":
            _lib.check(lib.ttfa_bwd_dq(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                       do.data_ptr(), lse.data_ptr(), delta.data_ptr(), dq.data_ptr(),
                                       B, Hq, Hkv, T, D, dt_code, scale, launch_sp[0]))
        else:
            _lib.check(lib.ttfa_bwd_dkdv(q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(),
                                         lse.data_ptr(), delta.data_ptr(), dk.data_ptr(),
                                         dv.data_ptr(), B, Hq, Hkv, T, D, dt_code, scale,
                                         launch_sp[0]))

    def launch(s, ev=None):
        for i, name in enumerate(kernel_names):
            if ev is not None:
                ev[i].record(stream)
            launch_one(name, s)
        if ev is not None:
            ev[len(kernel_names)].record(stream)

    # Settle phase (untimed): an idle GPU starts a run below its loaded clocks, and a few
    # warmup steps (under 1 ms of work at C2) do not bring it there.  Steps run in chunks
    # of 8 until --settle-ms of wall time has passed; the warmup and the timed region
    # below are unchanged by it.
    settle_steps, t_settle = 0, time.perf_counter()
    while args.settle_ms > 0 and (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for i in range(8):
            launch(sets[(settle_steps + i) % nsets])
        settle_steps += 8
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_settle

    for i in range(args.warmup):
        launch(sets[i % nsets])
    torch.cuda.synchronize()

    # Timed region: K steps back to back, bracketed by events after a synchronize; no
    # event between the launches (one recorded between two kernels lengthens the step).
    K = args.steps
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(K):
        launch(sets[i % nsets])
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(end) / K

    # Per-kernel breakdown: K more steps on the same rotation, with timing-only HIP events
    # on the launch stream between the three launches of every step.
    evs = [[HipTimingEvent() for _ in range(len(kernel_names) + 1)] for _ in range(K)]
    torch.cuda.synchronize()
    for i in range(K):
        launch(sets[i % nsets], evs[i])
    torch.cuda.synchronize()

    def per_kernel(evlist):
        kms = {n: [] for n in kernel_names}
        for ev in evlist:
            for i, n in enumerate(kernel_names):
                kms[n].append(ev[i].elapsed_time(ev[i + 1]))
        return kms

    kms = per_kernel(evs)
    avg = {n: sum(x) / len(x) for n, x in kms.items()}
    med = {n: statistics.median(x) for n, x in kms.items()}

    # Each event recorded between two launches adds a dispatch gap to the launch-to-launch
    # times above: their sum per step exceeds the timed region's step, which has no event
    # between launches and no gap (the kernels run back to back).  The gap per kernel is
    # that excess shared equally; a kernel's duration inside the step is its event time
    # less the gap, the figure a profiler's kernel trace reports for the timed steps.
    gap_ms = max(0.0, (sum(avg.values()) - ms_step) / len(avg))
    dom = max(avg, key=avg.get)
    dom_ms = avg[dom] - gap_ms

    # Hot-cache pass (outside the timed region above): the same input set every step, so
    # K/V and Q stay in the Infinity Cache; reported separately.
    Kh = 0 if args.no_extras else min(K, 50)
    evh = [[HipTimingEvent() for _ in range(4)] for _ in range(Kh)]
    for i in range(5 if Kh else 0):
        launch(sets[0])
    hot_step_ms = None
    if Kh:
        hs, he = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        hs.record(stream)
        for i in range(Kh):
            launch(sets[0])
        he.record(stream)
        torch.cuda.synchronize()
        hot_step_ms = hs.elapsed_time(he) / Kh
    for i in range(Kh):
        launch(sets[0], evh[i])
    torch.cuda.synchronize()
    hot = {n: statistics.median(x) for n, x in per_kernel(evh).items()} if Kh else None
    gemm = _gemm_reference(dev) if cfg.dtype == torch.bfloat16 and not args.no_extras else None

    # Graph replay (outside the timed region above): the same launches, one step per
    # input set over up to 8 sets, captured once in a HIP graph and replayed, so the host
    # issues one graph launch instead of one call per kernel.  Where the kernels are
    # shorter than the host's per-call cost (C1), this is the GPU-side step time.
    graph_ms = None
    if not args.no_extras:
        gsets = min(nsets, 8)
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):  # warm-up off the default stream, as capture wants
            launch_sp[0] = side.cuda_stream
            for i in range(gsets):
                launch(sets[i])
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            launch_sp[0] = torch.cuda.current_stream(dev).cuda_stream
            for i in range(gsets):
                launch(sets[i])
        launch_sp[0] = sp
        reps = max(1, K // gsets)
        # The capture leaves the GPU idle for milliseconds, after which its clocks take
        # longer than the few replays below to come back (measured: the same kernels ~20%
        # slower for 40 steps after a 50 ms pause, eager or replayed alike), so replays
        # run for --settle-ms first, as the timed region's own settle phase does.
        graph_settle = _settle(graph.replay, args.settle_ms)
        for _ in range(2):
            graph.replay()
        gs, ge = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        gs.record(stream)
        for _ in range(reps):
            graph.replay()
        ge.record(stream)
        torch.cuda.synchronize()
        graph_ms = gs.elapsed_time(ge) / (reps * gsets)

    fwd_f = cfg.fwd_flop()
    peak = PEAK_BF16_TFLOPS if cfg.dtype == torch.bfloat16 else PEAK_F32_TFLOPS
    step_tflops = 3.5 * fwd_f / (ms_step * 1e-3) / 1e12
    fwd_tflops = fwd_f / (avg["fwd"] * 1e-3) / 1e12
    bwd_of = lambda d: d["bwd"] if one_launch_bwd else d["bwd_dq"] + d["bwd_dkdv"]
    bwd_ms = bwd_of(avg)
    bwd_tflops = 2.5 * fwd_f / (bwd_ms * 1e-3) / 1e12

    # Dominant kernel: per causal (query row, key) pair a kernel's MFMA work is 2*D
    # FLOPs per matmul it needs for its outputs: fwd 2 (S, O), dQ pass 3 (S, dP, dQ),
    # dK/dV pass 4 (S, dP, dV, dK), one-launch fp32 backward 7; pairs = B*Hq*T^2/2.
    n_mm = {"fwd": 2, "bwd_dq": 3, "bwd_dkdv": 4, "bwd": 7}
    kern_flop = n_mm[dom] * fwd_f / 2
    achieved = kern_flop / (dom_ms * 1e-3) / 1e12
    kernel_symbol = {"fwd": "fa_fwd_bf16_kernel", "bwd_dq": "fa_bwd_dq_bf16_kernel",
                     "bwd_dkdv": "fa_bwd_dkdv_bf16_kernel", "bwd": "fa_bwd_f32_kernel"}[dom]
    if cfg.dtype == torch.float32:
        kernel_symbol = kernel_symbol.replace("bf16", "f32")
    kernel_symbol += f"<{D}>"
    traffic, traffic_src = (None, None) if args.no_traffic else _load_traffic(cfg.name, kernel_symbol)

    line = {
        "metric": "causal GQA FA fwd+bwd TFLOP/s & % bf16 MFMA peak on 1 MI355X",
        "value": round(step_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "f32",
        "data": "synthetic (seeded; q,k unit-RMS, v~N(0,1), dO~N(0,1)*1e-2)",
        "config": {"workload": f"{cfg.name}: causal {'GQA' if cfg.group > 1 else 'MHA'} attention "
                               f"fwd+bwd", "B": B, "Hq": Hq, "Hkv": Hkv, "T": T, "D": D,
                   "input_sets_rotated": nsets},
        "frac_of_peak": round(step_tflops / peak, 4),
        "passes": {
            "fwd": {"ms": round(avg["fwd"], 5), "tflops": round(fwd_tflops, 2),
                    "frac": round(fwd_tflops / peak, 4)},
            "bwd": {"ms": round(bwd_ms, 5), "tflops": round(bwd_tflops, 2),
                    "frac": round(bwd_tflops / peak, 4)},
            **({} if one_launch_bwd else {"bwd_dq_ms": round(avg["bwd_dq"], 5),
                                          "bwd_dkdv_ms": round(avg["bwd_dkdv"], 5)}),
            "median_ms": {n: round(x, 5) for n, x in med.items()},
            "timing": "per-kernel times from a second run of K steps right after the timed "
                      "region, timing-only HIP events (hipEventDisableSystemFence) between "
                      "the launches on their stream; value and ms_per_step come from the "
                      "timed region, which records no event between launches",
        },
        "hot_cache": None if hot is None else {
            "note": "same input set every step (working set resident in the 256 MB Infinity "
                    "Cache); the headline value above rotates sets to defeat it",
            "ms_per_step": round(hot_step_ms, 5),
            "fwd_bwd_tflops": round(3.5 * fwd_f / (hot_step_ms * 1e-3) / 1e12, 2),
            "median_ms": {n: round(x, 5) for n, x in hot.items()},
            "fwd_tflops": round(fwd_f / (hot["fwd"] * 1e-3) / 1e12, 2),
            "bwd_tflops": round(2.5 * fwd_f / (bwd_of(hot) * 1e-3) / 1e12, 2),
        },
        "graph_replay": None if graph_ms is None else {
            "note": "the same launches captured in one HIP graph (one step per input set, "
                    "up to 8 sets) and replayed after replays for --settle-ms: the step "
                    "without per-call host overhead",
            "ms_per_step": round(graph_ms, 5),
            "fwd_bwd_tflops": round(3.5 * fwd_f / (graph_ms * 1e-3) / 1e12, 2),
            "settle": graph_settle,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": kernel_symbol,
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "avg_launch_ms": round(dom_ms, 5),
            "avg_launch_ms_between_events": round(avg[dom], 5),
            "event_gap_ms": round(gap_ms, 5),
            "timing": "avg_launch_ms: the kernel's launch-to-launch event average in the "
                      "per-kernel breakdown steps less event_gap_ms, the dispatch gap each "
                      "event adds ((sum of the per-kernel event averages - ms_per_step) / "
                      "kernels per step); it is the kernel's duration inside the timed steps",
            "flop_per_launch": kern_flop,
        },
        "wall_s_timed": round(wall, 4),
        "settle": {"steps": settle_steps, "seconds": round(settle_s, 3),
                   "note": "untimed steps run before the warmup for at least --settle-ms of "
                           "wall time (clocks at their loaded level); not part of the timed "
                           "region"},
    }
    if gemm is not None:
        gemm["step_frac_of_gemm"] = round(step_tflops / gemm["tflops"], 4)
        gemm["fwd_frac_of_gemm"] = round(fwd_tflops / gemm["tflops"], 4)
        gemm["bwd_frac_of_gemm"] = round(bwd_tflops / gemm["tflops"], 4)
        line["gemm_reference"] = gemm
    if args.cpu_budget > 0:
        line["cpu_baseline"] = _cpu_baseline(cfg, args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
