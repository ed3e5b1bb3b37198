#!/usr/bin/env python
"""MoE block forward+backward throughput on one MI355X (Qwen3-30B-A3B shape).

One step = router (fp32 logits, top-8 softmax) -> permute -> grouped SwiGLU
expert GEMMs -> weighted combine -> Switch aux loss, then the full backward of
<out, d_out> + 0.001 * aux, on seeded synthetic inputs already resident in
HBM.  Prints one JSON line (metric, value, ..., roofline, cpu_baseline).

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--config c2]

The dominant kernel's duration comes from HIP events recorded around its
launches, on the stream the kernels run on, inside the timed region, in every
`--event-every`-th timed step (default 4); no other launch in the timed region
carries events (an event pair costs several microseconds of stream time).  The per-entry-point table comes from an
untimed instrumented pass (events around every launch) after the warm-up,
which also picks the dominant kernel.  The CPU
baseline times the reference's op sequence (F.grouped_mm on the CPU, the
config's dtype) on a bounded sample of the same layer.  After the C2
headline the run also times the MFMA-bound layers C4 and C5 briefly
(`other_configs` in the same JSON line; `--no-other-configs` skips them).
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
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
MFMA_FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 (the fp32 path, C1)
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def mfma_peak(w) -> float:
    return MFMA_FP32_PEAK_TFLOPS if w.dtype == "fp32" else MFMA_BF16_PEAK_TFLOPS


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_work(w, T: int, S: int):
    """Algorithmic work per launch, per timer tag: (flops or None, bytes).

    Bytes are the HBM traffic of an ideal kernel: every operand read once and
    every output written once (bf16 activations and weights, or fp32 for
    the fp32 path; fp32 router logits and scores).  A kernel's bound is
    whichever of flops / MFMA peak and bytes / HBM peak is larger."""
    H, I, E, k = w.hidden, w.intermediate, w.experts, w.top_k
    b = 4 if w.dtype == "fp32" else 2  # bytes per activation / weight element
    Wgu, Wdn = E * 2 * I * H * b, E * H * I * b  # expert weights
    xp, act, pre, y = S * H * b, S * I * b, S * 2 * I * b, S * H * b  # permuted rows, SwiGLU act, gate|up, down out
    fused_router = 0.0 if (w.local_experts or w.dtype == "fp32") else 6.0 * T * E + 8.0 * T * k
    return {
        "up_fwd": (4.0 * S * H * I, xp + Wgu + act + pre),
        "down_fwd": (2.0 * S * H * I, act + Wdn + y),
        "down_dgrad": (2.0 * S * H * I, y + Wdn + pre + pre),
        "down_wgrad": (2.0 * S * H * I, y + act + Wdn),
        "up_dgrad": (4.0 * S * H * I, pre + Wgu + xp),
        "up_wgrad": (4.0 * S * H * I, pre + xp + Wgu),
        "router_fwd": (2.0 * T * H * E, T * H * b + E * H * b + 8.0 * T * E + 12.0 * T * k),
        "router_gemm_bwd": (4.0 * T * H * E, T * E * b + T * H * b + E * H * b + T * H * b + 4.0 * E * H),
        # read each x row once and the routes, write permuted rows and maps
        "permute_fwd": (None, T * H * b + S * H * b + 16.0 * S),
        "combine_fwd": (None, S * H * b + 8.0 * S + T * H * b),
        # the bf16 block's combine backward also runs the router's top-k
        # backward: logits and routes in, bf16 d_logits out
        "combine_bwd": (None, T * H * b + 2.0 * S * H * b + 12.0 * S + fused_router),
        # the routes' rows, the router's dX added in (d_add), and d_hidden
        "permute_bwd": (None, S * H * b + 2.0 * T * H * b + 4.0 * S),
        # logits in, bf16 d_logits out (the aux gradient formed in the same pass)
        "router_topk_bwd": (None, 4.0 * T * E + 2.0 * T * E + 16.0 * T * k),
        "aux_fwd": (None, 4.0 * T * E),
        "aux_bwd": (None, 8.0 * T * E),
    }


def bound_of(flops, nbytes, peak_tflops=MFMA_BF16_PEAK_TFLOPS):
    if flops is not None and flops / (peak_tflops * 1e12) > nbytes / (HBM_PEAK_GBS * 1e9):
        return "mfma"
    return "hbm"


def read_traffic(tag: str, workload: str):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary, or None."""
    path = ROOT / "profiles" / f"{tag}_{workload}_pmc.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


# Kernels launched by each timed entry point (tag), matched on demangled names.
_TAG_KERNELS = {
    "router_fused_fwd_kernel": "router_fwd",
    "router_reduce_topk_kernel": "router_fwd",
    "router_bwd_gemm_kernel": "router_gemm_bwd",
    "reduce_partials_bf16_kernel": "router_gemm_bwd",
    "router_topk_bwd_kernel": "router_topk_bwd",
    "aux_partial_kernel": "aux_fwd",
    "aux_reduce_kernel": "router_fwd",  # in the step, moe_router_aux_fwd's loss reduction
    "aux_finalize_kernel": "router_fwd",
    "aux_bwd_kernel": "aux_bwd",
    "permute_count_kernel": "permute_fwd",
    "permute_scatter_kernel": "permute_fwd",
    "scatter_rows_kernel": "permute_fwd",
    "combine_fwd_kernel": "combine_fwd",
    "combine_bwd_kernel": "combine_bwd",
    "combine_router_bwd_kernel": "combine_bwd",  # the block's combine backward with the router top-k backward
    "permute_bwd_kernel": "permute_bwd",
    "swiglu_bwd_kernel": "down_dgrad",
}
_GEMM_RE = r"grouped_gemm_kernel<(\d), (true|false), (\d), moe::TileCfg<([0-9, ]+)>"
# Expert-GEMM instantiations (mode, B K-contiguous, epilogue) -> the entry points
# that launch them, in the order one step launches them.
_GEMM_ORDER = {
    (0, True, 2): ["up_fwd"],
    (0, True, 0): ["down_fwd"],
    (0, False, 0): ["down_dgrad", "up_dgrad"],  # backward runs the down projection first
    (1, False, 4): ["up_wgrad", "down_wgrad"],  # ... and the weight gradients last, up first
}


def tag_dispatches(names):
    """Bench timer tag of each kernel dispatch, given kernel names in dispatch order.

    The expert GEMMs are the grouped_gemm instantiations with tiles of 256 or
    more rows (the router GEMMs use 128-row tiles); entry points that share a
    (mode, operand layout, epilogue) signature are told apart by their
    occurrence order (each step launches them in a fixed order)."""
    import re

    parsed = [re.search(_GEMM_RE, n) for n in names]
    seen = {}
    tags = []
    for n, m in zip(names, parsed):
        if m:
            key = (int(m[1]), m[2] == "true", int(m[3]))
            if int(m[4].split(",")[0]) >= 256 and key in _GEMM_ORDER:
                order = _GEMM_ORDER[key]
                i = seen.get(key, 0)
                seen[key] = i + 1
                tags.append(order[i % len(order)])
            else:
                tags.append("router_fwd" if key[:2] == (0, True) else "router_gemm_bwd")
            continue
        tags.append(next((t for k, t in _TAG_KERNELS.items() if f"moe::{k}" in n or f" {k}(" in n or n.startswith(k)), None))
    return tags


def _read_csvs(d):
    import csv

    rows = []
    for f in sorted(Path(d).rglob("*counter_collection.csv")):
        with open(f) as fh:
            rows.extend(csv.DictReader(fh))
    if not rows:
        raise SystemExit(f"no counter_collection.csv under {d}")
    return rows


def profile_summary(args) -> int:
    """Writes profiles/ summaries from rocprofv3 outputs of this script.

    Kernel durations come from a --kernel-trace --stats run; HBM bytes per
    launch from one --pmc FETCH_SIZE and one --pmc WRITE_SIZE run, each scaled
    by what the same counter reads for a 1 GiB device copy (--copy-calibration).
    """
    import csv
    from collections import defaultdict

    from parallel_amd.workloads import WORKLOADS

    w = WORKLOADS[args.config]
    prof = ROOT / "profiles"
    prof.mkdir(exist_ok=True)
    cmd = args.profile_commands or ""

    # ---- kernel durations (per dispatch, from the --kernel-trace CSV of the --stats run)
    with open(args.trace_csv) as fh:
        trace = sorted(csv.DictReader(fh), key=lambda r: int(r["Dispatch_Id"]))
    tags = tag_dispatches([r["Kernel_Name"] for r in trace])
    disp = defaultdict(list)
    for r, tag in zip(trace, tags):
        disp[(tag or "-", r["Kernel_Name"])].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    grand = sum(sum(v) for v in disp.values())
    lines = [f"# rocprofv3 kernel statistics, workload {w.name} ({args.steps_profiled} timed steps plus the warm-up "
             f"and instrumented steps)",
             f"# command: {cmd.splitlines()[0] if cmd else '(not recorded)'}",
             f"# {'tag':16s} {'calls':>6s} {'avg_us':>10s} {'total_us':>11s} {'pct':>6s}  kernel"]
    per_tag = defaultdict(lambda: [0.0, 0])
    for (tag, name), ds in sorted(disp.items(), key=lambda kv: -sum(kv[1])):
        total = sum(ds)
        short = name.replace("moe::", "").split("(")[0][:100]
        lines.append(f"  {tag:16s} {len(ds):6d} {total / len(ds):10.1f} {total:11.1f} {100 * total / grand:6.2f}  {short}")
        if tag != "-":
            per_tag[tag][0] += total
            per_tag[tag][1] = max(per_tag[tag][1], len(ds))
    lines.append("# per entry point (sum of its kernels / calls):")
    for tag, (total, calls) in sorted(per_tag.items(), key=lambda kv: -kv[1][0]):
        lines.append(f"avg_us_per_call {tag}: {total / calls:.1f}")
    (prof / f"kernel_stats_{w.name}.txt").write_text("\n".join(lines) + "\n")
    if not (args.pmc_fetch and args.pmc_write and args.cal_fetch and args.cal_write):
        log(f"wrote kernel_stats_{w.name}.txt under {prof} (no counter runs given)")
        return 0

    # ---- HBM traffic
    def per_kernel(d, counter):
        acc = defaultdict(list)
        for r in _read_csvs(d):
            if r["Counter_Name"] == counter:
                acc[(r["Kernel_Name"], int(r["Dispatch_Id"]))].append(float(r["Counter_Value"]))
        return acc

    def cal_factor(d, counter, expect_kib):
        vals = [v for (n, g), vs in per_kernel(d, counter).items() if "copyBuffer" in n for v in vs]
        if not vals:
            raise SystemExit(f"calibration run {d} holds no copy kernel")
        return expect_kib / statistics.fmean(vals), statistics.fmean(vals)

    f_fac, f_cal = cal_factor(args.cal_fetch, "FETCH_SIZE", 1 << 20)
    w_fac, w_cal = cal_factor(args.cal_write, "WRITE_SIZE", 1 << 20)
    fetch = per_kernel(args.pmc_fetch, "FETCH_SIZE")
    write = per_kernel(args.pmc_write, "WRITE_SIZE")
    work = kernel_work(w, w.tokens, w.slots)
    by_tag = defaultdict(lambda: {"fetch": 0.0, "write": 0.0, "kernels": set()})
    for runs, field in ((fetch, "fetch"), (write, "write")):
        keys = sorted(runs, key=lambda k: k[1])  # dispatch order
        for key, tag in zip(keys, tag_dispatches([k[0] for k in keys])):
            if tag:
                by_tag[tag][field] += sum(runs[key])
                by_tag[tag]["kernels"].add(key[0].replace("moe::", "").split("(")[0])
    for tag, d in by_tag.items():
        calls = args.pmc_calls
        rd = d["fetch"] / calls * f_fac * 1024
        wr = d["write"] / calls * w_fac * 1024
        flops, amount = work[tag]
        body = [
            f"# HBM traffic per launch of entry point '{tag}', workload {w.name}",
            "# kernels: " + "; ".join(sorted(d["kernels"])),
            "# commands (one counter per pass; calibration = 1 GiB device copy):",
            *[f"#   {c}" for c in cmd.splitlines()],
            f"# calibration: copy of 1 GiB reads FETCH_SIZE {f_cal:.1f} KiB (factor {f_fac:.3f}), "
            f"writes WRITE_SIZE {w_cal:.1f} KiB (factor {w_fac:.3f})",
            f"launches_profiled: {calls}",
            f"fetch_size_kib_per_launch: {d['fetch'] / calls:.1f}",
            f"write_size_kib_per_launch: {d['write'] / calls:.1f}",
            f"read_bytes_per_launch: {rd:.0f}",
            f"write_bytes_per_launch: {wr:.0f}",
            f"hbm_bytes_per_launch: {rd + wr:.0f}",
            f"algorithmic_bytes_per_launch: {amount:.0f}",
            f"algorithmic_flops_per_launch: {flops:.0f}" if flops is not None else "algorithmic_flops_per_launch: -",
            f"bound: {bound_of(flops, amount, mfma_peak(w))}",
        ]
        (prof / f"{tag}_{w.name}_pmc.txt").write_text("\n".join(body) + "\n")
    log(f"wrote {len(by_tag)} traffic summaries and kernel_stats_{w.name}.txt under {prof}")
    if args.pmc_util and args.pmc_ta and args.pmc_tcp:
        units_summary(args, w, prof, cmd)
    return 0


_UNIT_COUNTERS = {
    "pmc_util": "MfmaUtil LdsUtil LdsBankConflict",
    "pmc_ta": "TA_BUSY_avr TA_ADDR_STALLED_BY_TC_CYCLES_sum GRBM_GUI_ACTIVE SQ_VMEM_TA_ADDR_FIFO_FULL "
              "SQ_VMEM_TA_CMD_FIFO_FULL SQ_LDS_DATA_FIFO_FULL SQ_BUSY_CYCLES",
    "pmc_tcp": "TCP_TCC_READ_REQ_LATENCY_sum TCP_TCC_READ_REQ_sum TCP_PENDING_STALL_CYCLES_sum "
               "TCP_TCR_TCP_STALL_CYCLES_sum GRBM_GUI_ACTIVE",
}


def units_summary(args, w, prof, cmd) -> None:
    """The expert GEMMs' unit utilisation from three counter passes over this
    script (--pmc-util, --pmc-ta, --pmc-tcp; one counter set per pass).
    GRBM_GUI_ACTIVE sums the 8 XCDs, the SQ and TCP sums cover every CU, and
    TA_BUSY_avr averages over the texture units."""
    from collections import defaultdict

    gemms = ["up_fwd", "down_fwd", "down_dgrad", "up_dgrad", "up_wgrad", "down_wgrad"]
    acc = defaultdict(lambda: defaultdict(list))
    for d in (args.pmc_util, args.pmc_ta, args.pmc_tcp):
        per = defaultdict(dict)
        for r in _read_csvs(d):
            e = per[int(r["Dispatch_Id"])]
            e["name"] = r["Kernel_Name"]
            e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        ids = sorted(per)
        for i, tag in zip(ids, tag_dispatches([per[i]["name"] for i in ids])):
            if tag in gemms and "grouped_gemm_kernel" in per[i]["name"]:  # not the SwiGLU backward
                for c, v in per[i].items():
                    if c != "name":
                        acc[tag][c].append(v)
    cus = 256
    mean = statistics.fmean
    rows = ["| GEMM | launches | MFMA busy | LDS active | TA busy | TA FIFO full | L1 waiting on L2 | L2 read latency |",
            "|---|---|---|---|---|---|---|---|"]
    for tag in gemms:
        d = acc[tag]
        if not d:
            continue
        cyc = mean(d["GRBM_GUI_ACTIVE"]) / 8.0  # per-XCD cycles
        lat = sum(d["TCP_TCC_READ_REQ_LATENCY_sum"]) / sum(d["TCP_TCC_READ_REQ_sum"])
        rows.append(f"| {tag} | {len(d['MfmaUtil'])} | {mean(d['MfmaUtil']):.0f}% | {mean(d['LdsUtil']):.0f}% | "
                    f"{100 * mean(d['TA_BUSY_avr']) / cyc:.0f}% | "
                    f"{100 * mean(d['SQ_VMEM_TA_ADDR_FIFO_FULL']) / (cus * cyc):.0f}% | "
                    f"{100 * mean(d['TCP_PENDING_STALL_CYCLES_sum']) / (cus * cyc):.0f}% | {lat:.0f} cycles |")
    conflicts = [mean(acc[t]["LdsBankConflict"]) for t in gemms if acc[t]]
    body = [
        f"# Expert-GEMM unit utilisation, workload {w.name} (per launch, averaged over the launches of each",
        "# entry point in the profiled run: warm-up, instrumented and timed steps)",
        "# commands (one counter set per pass):",
        *([f"#   {c}" for c in cmd.splitlines() if any(f"--pmc {v} " in c for v in _UNIT_COUNTERS.values())] or
          [f"#   cd /tmp && rocprofv3 --pmc {c} -f csv -d <out>/{n} -o run -- python3 <repo>/bench.py --steps 2 "
           f"--warmup 1 --no-cpu-baseline" for n, c in _UNIT_COUNTERS.items()]),
        *[f"#   {c}" for c in cmd.splitlines() if "--profile-summary" in c],
        "# Normalisation: GRBM_GUI_ACTIVE sums the 8 XCDs (per-XCD cycles = value / 8; with the kernel",
        "# durations this gives about 2.1 GHz); SQ_VMEM_TA_ADDR_FIFO_FULL and the TCP sums cover 256 CUs;",
        "# TA_BUSY_avr is the average over the texture units. MfmaUtil and LdsUtil are rocprofv3's derived",
        f"# metrics (busy cycles over active cycles x SIMDs / CUs). LdsBankConflict: "
        f"{min(conflicts):.1f}-{max(conflicts):.1f}%.",
        "# The weight-gradient GEMMs share one kernel; dispatches alternate up_wgrad, down_wgrad in each step.",
        *rows,
    ]
    (prof / f"gemm_units_{w.name}_pmc.txt").write_text("\n".join(body) + "\n")
    log(f"wrote gemm_units_{w.name}_pmc.txt")


def cpu_model_name() -> str | None:
    """The host CPU's model name, as lscpu's "Model name" shows it (read from
    /proc/cpuinfo, where lscpu takes it, so that no child process is started
    from a process that holds the GPU)."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(w, tokens: int):
    """Reference op sequence on the host CPU (bounded sample of the same layer)."""
    import torch

    from oracle import moe_oracle as O
    from parallel_amd.workloads import make_block_inputs, scaled

    ws = scaled(w, tokens)
    dtype = torch.float32 if w.dtype == "fp32" else torch.bfloat16
    inp = make_block_inputs(ws, seed=0, dtype=dtype)
    leaves = O.make_leaves(inp["x"], inp["router_weight"], inp["gate_up_proj"], inp["down_proj"])
    times = []
    for i in range(4):
        t0 = time.perf_counter()
        O.reference_step(leaves, inp["d_out"], top_k=w.top_k, norm_topk_prob=w.norm_topk_prob, aux_coef=w.aux_coef,
                         compute_dtype=dtype, logit_bias=inp.get("logit_bias"))
        times.append(time.perf_counter() - t0)
    med = statistics.median(times[1:])
    return {
        "value": round(tokens / med, 1),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": cpu_model_name(),
        "torch_threads": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{tokens} tokens of the {w.name} layer (H={w.hidden}, E={w.experts}, top-{w.top_k}, "
                  f"I={w.intermediate}), {w.dtype}, fwd+bwd via F.grouped_mm on the CPU; median of 3 after 1 warm-up "
                  f"({med:.2f} s/step)",
    }


def calibration(w) -> dict:
    """The box's own ceilings, measured after the timed region so that the
    spec peaks the roofline quotes can be read against them: a 1 GiB
    device-to-device copy (read + write bytes), hipBLASLt's dense bf16 GEMM
    (torch.mm, 8192^3, the second operand K-contiguous as nn.Linear keeps
    it) and its batched bf16 GEMM on the workload's up projection with the
    routed rows split equally over the experts (torch.bmm, contiguous
    operands: a transposed right operand is kept out of batched products).
    Reference kernels, not this build's."""
    import torch

    dev = "cuda"

    def timed(fn, reps=5):
        for _ in range(2):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3

    out = {}
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
    dst = torch.empty_like(src)
    out["torch_copy_gbs"] = round(2.0 * 4 * src.numel() / timed(lambda: dst.copy_(src)) / 1e9, 1)
    del src, dst
    n = 8192
    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16)  # [N, K], used as K-contiguous (nn.Linear's layout)
    out["hipblaslt_dense_bf16_tflops"] = round(2.0 * n ** 3 / timed(lambda: torch.mm(a, b.t())) / 1e12, 1)
    del a, b
    E, H, I = (w.local_experts or w.experts), w.hidden, w.intermediate
    rows = max(1, w.slots // E)
    x = torch.randn(E, rows, H, device=dev, dtype=torch.bfloat16)
    wt = torch.randn(E, H, 2 * I, device=dev, dtype=torch.bfloat16)  # contiguous [E, H, 2I]
    out["hipblaslt_batched_up_bf16_tflops"] = round(2.0 * E * rows * H * 2 * I /
                                                    timed(lambda: torch.bmm(x, wt)) / 1e12, 1)
    out["batched_shape"] = f"{E} x [{rows} x {H}] . [{H} x {2 * I}]"
    del x, wt
    torch.cuda.empty_cache()
    return out


def measure(w, steps: int, warmup: int, instrumented_steps: int, event_every: int = 4, bf16_logits: bool = False):
    """Builds workload w's inputs on the GPU, runs `warmup` steps, an
    instrumented pass (events around every launch, outside the timed region)
    and `steps` timed steps in which only the dominant entry point carries
    events, in every `event_every`-th step.  Returns the step time, the per-entry-point durations and the
    dominant entry point's launches in the timed region."""
    import torch

    from parallel_amd import _lib, ops
    from parallel_amd.workloads import make_block_inputs

    class _Args:
        pass

    args = _Args()
    args.steps, args.warmup, args.instrumented_steps = steps, warmup, instrumented_steps
    dev = "cuda"
    torch.manual_seed(0)
    dtype = torch.float32 if w.dtype == "fp32" else torch.bfloat16  # C1 runs the fp32 path
    inp = make_block_inputs(w, seed=0, device=dev, dtype=dtype, weights_on_device_rng=True)
    gu = inp["gate_up_proj"].requires_grad_()
    dn = inp["down_proj"].requires_grad_()
    if w.local_experts:
        # C3: the expert step of EP rank 0 on its receive buffer (source-rank
        # major rows, one local expert each, token_dispatch.py:101-158), as a
        # rank of an ep=2 group runs it between the two exchanges.
        from parallel_amd.workloads import ep_receive_buffer

        _, _, (src, tok, lexp, lsc) = ep_receive_buffer(w, seed=0)
        rows = len(src)
        g = torch.Generator(device=dev).manual_seed(1)
        xs = torch.randn(w.sources, w.tokens, w.hidden, device=dev, generator=g).to(torch.bfloat16)
        x = xs[torch.from_numpy(src).to(dev), torch.from_numpy(tok).to(dev)].contiguous().requires_grad_()
        r_idx = torch.from_numpy(lexp).view(rows, 1).to(dev)
        r_sc = torch.from_numpy(lsc).view(rows, 1).to(dev).requires_grad_()
        d_out = torch.randn(rows, w.hidden, device=dev, generator=g).to(torch.bfloat16)
        params = (x, r_sc, gu, dn)
        log(f"workload {w.name}: {w.sources} x {w.tokens} source tokens, {rows} routed rows to "
            f"{w.local_experts} of {w.experts} experts, H={w.hidden} I={w.intermediate}")

        def step():
            for p in params:
                p.grad = None
            ops.experts(x, r_idx, r_sc, gu, dn).backward(d_out)
    else:
        rows = w.slots
        x = inp["x"].requires_grad_()
        rw = inp["router_weight"].requires_grad_()
        d_out = inp["d_out"]
        bias = inp.get("logit_bias")
        coef = torch.tensor(w.aux_coef, device=dev)
        # C4 accumulates the weight gradients into pre-existing, seeded
        # gradient buffers (inside the weight-gradient kernel); the other
        # configs start every step from cleared gradients.
        accumulate = w.name == "c4"
        if accumulate:
            g = torch.Generator(device=dev).manual_seed(3)
            for p in (rw, gu, dn):
                p.grad = torch.randn(p.shape, generator=g, device=dev).mul_(1e-3).to(p.dtype)
        params = (x,) if accumulate else (x, rw, gu, dn)
        log(f"workload {w.name}: T={w.tokens} H={w.hidden} E={w.experts} k={w.top_k} I={w.intermediate}"
            + (" (dW accumulated into existing gradients)" if accumulate else ""))

        def step():
            for p in params:
                p.grad = None
            # Router, aux loss and experts as one op: the router's own softmax
            # and top-k also give the Switch aux loss (TF load_balancing_loss_func
            # recomputes both from the logits), and the backward adds the
            # router's input gradient to the experts' inside the permute
            # backward instead of a separate elementwise add.
            out, _, _, _, aux = ops.moe_block(x, rw, gu, dn, w.top_k, w.norm_topk_prob, None, bias, accumulate,
                                              bf16_logits)
            torch.autograd.backward([out, aux], [d_out, coef])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"warm-up done ({args.warmup} steps)")

    # Per-entry-point durations from an instrumented pass outside the timed
    # region: an event pair around every launch costs several microseconds of
    # stream time per launch, which would show up in the step time.
    _lib.TIMER.reset()
    _lib.TIMER.only = None
    _lib.TIMER.enabled = True
    for _ in range(args.instrumented_steps):
        step()
    torch.cuda.synchronize()
    _lib.TIMER.enabled = False
    durations = _lib.TIMER.durations_ms()
    dominant = max(durations, key=lambda t: sum(durations[t]))

    # The timed region: only the dominant kernel's launches carry events, in
    # every event_every-th step (each event pair leaves a gap of a few
    # microseconds in the stream).
    _lib.TIMER.reset()
    _lib.TIMER.only = {dominant}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        _lib.TIMER.enabled = i % event_every == 0
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.TIMER.enabled = False
    _lib.TIMER.only = None
    dominant_ms = _lib.TIMER.durations_ms()[dominant]
    ms_per_step = 1e3 * elapsed / args.steps
    tokens_per_s = w.sources * w.tokens * args.steps / elapsed  # source tokens (one source but for C3)
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step, {tokens_per_s:,.0f} tokens/s")

    return dict(ms_per_step=ms_per_step, tokens_per_s=tokens_per_s, elapsed=elapsed, durations=durations,
                dominant=dominant, dominant_ms=dominant_ms, rows=rows)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2",
                    help="workload key (c1 c2 c3 c4 c5); c2 is the headline, c1 the reference's fp32 CPU case")
    ap.add_argument("--router-logits", choices=("fp32", "bf16"), default="fp32",
                    help="router logits dtype: fp32 (the configurations' statement) or bf16 (the reference's "
                         "router under bf16 autocast)")
    ap.add_argument("--event-every", type=int, default=4,
                    help="timed steps per step whose dominant-kernel launches carry HIP events")
    ap.add_argument("--instrumented-steps", type=int, default=3,
                    help="untimed steps with events around every launch (the per-kernel table)")
    ap.add_argument("--cpu-baseline-tokens", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy 3 times (scales rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the C4/C5 side measurements after the C2 headline")
    ap.add_argument("--other-steps", type=int, default=10, help="timed steps of each C4/C5 side measurement")
    ap.add_argument("--profile-summary", action="store_true",
                    help="write profiles/ summaries from rocprofv3 outputs (--trace-csv, --pmc-*, --cal-*)")
    ap.add_argument("--trace-csv", help="kernel_trace.csv of a rocprofv3 --kernel-trace --stats run")
    ap.add_argument("--pmc-fetch")
    ap.add_argument("--pmc-write")
    ap.add_argument("--cal-fetch")
    ap.add_argument("--cal-write")
    ap.add_argument("--pmc-calls", type=int, default=6,
                    help="entry-point calls in the --pmc runs: warm-up + instrumented + timed steps (1 + 3 + 2)")
    ap.add_argument("--steps-profiled", type=int, default=10)
    ap.add_argument("--profile-commands", help="the rocprofv3 command lines, one per line, recorded in the summaries")
    ap.add_argument("--pmc-util", help="counter_collection dir of a --pmc MfmaUtil LdsUtil LdsBankConflict run")
    ap.add_argument("--pmc-ta", help="counter_collection dir of the texture-unit counter run")
    ap.add_argument("--pmc-tcp", help="counter_collection dir of the L1 (TCP) counter run")
    args = ap.parse_args()
    if args.profile_summary:
        sys.path.insert(0, str(ROOT))
        return profile_summary(args)
    if args.copy_calibration:
        import torch

        src = torch.ones(1 << 29, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copied 1 GiB three times")
        return 0
    if args.gpus != 1:
        print(
            f"bench.py runs one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
            "it measures one rank's share on one MI355X",
            file=sys.stderr,
        )
        return 2

    import torch

    sys.path.insert(0, str(ROOT))
    from parallel_amd import _lib, ops
    from parallel_amd.workloads import WORKLOADS, make_block_inputs

    w = WORKLOADS[args.config]
    m = measure(w, args.steps, args.warmup, args.instrumented_steps, max(1, args.event_every),
                args.router_logits == "bf16")
    ms_per_step, tokens_per_s, elapsed = m["ms_per_step"], m["tokens_per_s"], m["elapsed"]
    durations, dominant, dominant_ms, rows = m["durations"], m["dominant"], m["dominant_ms"], m["rows"]

    if w.local_experts:  # the experts see `rows` tokens of one route each, over the local experts
        import dataclasses

        work = kernel_work(dataclasses.replace(w, experts=w.local_experts, top_k=1), rows, rows)
    else:
        work = kernel_work(w, w.tokens, w.slots)
    peak = mfma_peak(w)
    kernels = {}
    for tag, ds in sorted(durations.items()):
        avg = statistics.fmean(ds)
        entry = {"avg_ms": round(avg, 4), "launches_per_step": len(ds) // args.instrumented_steps}
        if tag in work:
            flops, nbytes = work[tag]
            entry["bound"] = bound_of(flops, nbytes, peak)
            if flops is not None:
                tf = flops / (avg * 1e-3) / 1e12
                entry.update(tflops=round(tf, 1), mfma_frac=round(tf / peak, 4))
            gbs = nbytes / (avg * 1e-3) / 1e9
            entry.update(gbs=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK_GBS, 4))
        kernels[tag] = entry
        log(f"  {tag:16s} {avg * 1e3:9.1f} us  {entry}")
    flops, nbytes = work[dominant]
    avg_s = statistics.fmean(dominant_ms) * 1e-3  # measured inside the timed region
    if bound_of(flops, nbytes, peak) == "mfma":
        achieved = flops / avg_s / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(achieved / peak, 4)}
    else:
        achieved = nbytes / avg_s / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4)}
    roofline["traffic"] = read_traffic(dominant, w.name)
    roofline["kernel"] = dominant
    roofline["avg_us_in_timed_region"] = round(avg_s * 1e6, 1)
    roofline["launches_timed"] = len(m["dominant_ms"])
    roofline["algorithmic_bytes_per_launch"] = nbytes
    roofline["flops_per_launch"] = flops
    if flops is not None:
        roofline["mfma_tflops"] = round(flops / avg_s / 1e12, 1)
    gemm_tags = [t for t in ("up_fwd", "down_fwd", "down_dgrad", "down_wgrad", "up_dgrad", "up_wgrad")
                 if t in durations]
    gemm_s = sum(statistics.fmean(durations[t]) for t in gemm_tags) * 1e-3
    gemm_flops = w.gemm_flops(rows)  # fwd + bwd over the routed rows
    gemm_tflops = gemm_flops / gemm_s / 1e12 if gemm_s else None

    # The MFMA-bound layers (C4: imbalanced routing, dW accumulated; C5: the
    # larger layer) timed briefly after the headline, in the same process.
    other = {}
    if args.config == "c2" and not args.no_other_configs:
        import gc

        del m
        gc.collect()
        torch.cuda.empty_cache()
        for name in ("c4", "c5"):
            wo = WORKLOADS[name]
            mo = measure(wo, args.other_steps, 2, 2)
            tags = [t for t in ("up_fwd", "down_fwd", "down_dgrad", "down_wgrad", "up_dgrad", "up_wgrad")
                    if t in mo["durations"]]
            g_s = sum(statistics.fmean(mo["durations"][t]) for t in tags) * 1e-3
            g_tf = wo.gemm_flops(mo["rows"]) / g_s / 1e12
            other[name] = {"ms_per_step": round(mo["ms_per_step"], 4), "tokens_per_s": round(mo["tokens_per_s"], 1),
                           "steps": args.other_steps, "warmup": 2, "tokens": wo.tokens, "hidden": wo.hidden,
                           "moe_intermediate": wo.intermediate,
                           "grouped_gemm": {"time_ms": round(g_s * 1e3, 4), "tflops": round(g_tf, 1),
                                            "mfma_frac": round(g_tf / MFMA_BF16_PEAK_TFLOPS, 4)}}
            log(f"{name}: {mo['ms_per_step']:.3f} ms/step, grouped GEMMs {g_tf:.0f} TFLOP/s")
            del mo
            gc.collect()
            torch.cuda.empty_cache()

    calib = None
    if args.config == "c2" and not args.no_other_configs:
        calib = calibration(w)
        log(f"calibration: {calib}")

    cpu = None
    if not args.no_cpu_baseline and not w.local_experts:
        log(f"cpu baseline: {args.cpu_baseline_tokens} tokens on {torch.get_num_threads()} threads")
        cpu = cpu_baseline(w, args.cpu_baseline_tokens)
        log(f"cpu baseline: {cpu['value']:,.0f} tokens/s")

    result = {
        "metric": "MoE block fwd+bwd tokens/s (Qwen3-30B-A3B shape, 1 GPU); grouped-GEMM MFMA %",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic (seeded normal inputs and weights)",
        "config": {"workload": {"c1": "c1: tiny Qwen3-MoE block (fp32)", "c2": "c2: Qwen3-30B-A3B MoE block",
                                "c4": "c4: Qwen3-30B-A3B MoE block"}.get(w.name, w.name),
                   "tokens": w.tokens, "hidden": w.hidden, "experts": w.experts, "top_k": w.top_k,
                   "moe_intermediate": w.intermediate, "router_logits": args.router_logits, "aux_coef": w.aux_coef,
                   "dW": "accumulated into existing gradients" if w.name == "c4" else "written"},
        "grouped_gemm": {"flops_fwd_bwd": gemm_flops, "time_ms": round(gemm_s * 1e3, 4),
                         "tflops": round(gemm_tflops, 1) if gemm_tflops else None,
                         "mfma_frac": round(gemm_tflops / peak, 4) if gemm_tflops else None},
        "roofline": roofline,
        "kernels": kernels,
        "kernels_source": f"untimed instrumented pass of {args.instrumented_steps} steps (events around every launch)",
        "cpu_baseline": cpu,
    }
    if calib:
        result["calibration"] = calib
    if other:
        result["other_configs"] = other
        result["other_configs_note"] = ("C4 and C5 step times in the same run (value is C2's); grouped_gemm from "
                                         "an instrumented pass of 2 steps")
    if w.local_experts:
        result["config"].update(sources=w.sources, local_experts=w.local_experts, routed_rows=rows,
                                zipf_alpha=w.zipf_alpha)
        result["routed_slots_per_s"] = round(rows * args.steps / elapsed, 1)
        result["value_is"] = "source tokens/s (sources x tokens / step time); routed_slots_per_s is rows / step time"
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
