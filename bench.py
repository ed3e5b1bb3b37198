#!/usr/bin/env python
"""MoE block forward+backward throughput on one MI355X (Qwen3-30B-A3B shape).

One step = router (fp32 logits, top-8 softmax) -> permute -> grouped SwiGLU
expert GEMMs -> weighted combine -> Switch aux loss, then the full backward of
<out, d_out> + 0.001 * aux, on seeded synthetic inputs already resident in
HBM.  Prints one JSON line (metric, value, ..., roofline, cpu_baseline).

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--config c2]

The dominant kernel's duration comes from HIP events recorded around every
launch on the stream the kernels run on, inside the timed region.  The CPU
baseline times the reference's op sequence (F.grouped_mm on the CPU, the
config's dtype) on a bounded sample of the same layer.
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
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_work(w, T: int, S: int):
    """Algorithmic work per launch: ('mfma', FLOP) or ('hbm', bytes), per timer tag."""
    H, I, E, k = w.hidden, w.intermediate, w.experts, w.top_k
    b = 2  # bf16
    return {
        "up_fwd": ("mfma", 4.0 * S * H * I),
        "down_fwd": ("mfma", 2.0 * S * H * I),
        "down_dgrad": ("mfma", 2.0 * S * H * I),
        "down_wgrad": ("mfma", 2.0 * S * H * I),
        "up_dgrad": ("mfma", 4.0 * S * H * I),
        "up_wgrad": ("mfma", 4.0 * S * H * I),
        "router_fwd": ("mfma", 2.0 * T * H * E),
        "router_gemm_bwd": ("mfma", 4.0 * T * H * E),
        # bytes: read x rows once per route and ids, write permuted rows and maps
        "permute_fwd": ("hbm", T * H * b + S * H * b + 16.0 * S),
        "combine_fwd": ("hbm", S * H * b + 8.0 * S + T * H * b),
        "combine_bwd": ("hbm", T * H * b + 2.0 * S * H * b + 12.0 * S),
        "permute_bwd": ("hbm", S * H * b + T * H * b + 4.0 * S),
        "router_topk_bwd": ("hbm", 8.0 * T * E + 2.0 * T * E + 16.0 * T * k),
        "aux_fwd": ("hbm", 4.0 * T * E),
        "aux_bwd": ("hbm", 8.0 * T * E),
    }


def read_traffic(tag: str, workload: str):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary, or None."""
    path = ROOT / "profiles" / f"{tag}_{workload}_pmc.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(w, tokens: int):
    """Reference op sequence on the host CPU (bounded sample of the same layer)."""
    import torch

    from oracle import moe_oracle as O
    from parallel_amd.workloads import make_block_inputs, scaled

    ws = scaled(w, tokens)
    inp = make_block_inputs(ws, seed=0, dtype=torch.bfloat16)
    leaves = O.make_leaves(inp["x"], inp["router_weight"], inp["gate_up_proj"], inp["down_proj"])
    times = []
    for i in range(4):
        t0 = time.perf_counter()
        O.reference_step(leaves, inp["d_out"], top_k=w.top_k, norm_topk_prob=w.norm_topk_prob, aux_coef=w.aux_coef,
                         compute_dtype=torch.bfloat16, logit_bias=inp.get("logit_bias"))
        times.append(time.perf_counter() - t0)
    med = statistics.median(times[1:])
    return {
        "value": round(tokens / med, 1),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{tokens} tokens of the {w.name} layer (H={w.hidden}, E={w.experts}, top-{w.top_k}, "
                  f"I={w.intermediate}), bf16, fwd+bwd via F.grouped_mm on the CPU; median of 3 after 1 warm-up "
                  f"({med:.2f} s/step)",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2", help="workload key (c2 c3 c4 c5); c2 is the headline")
    ap.add_argument("--cpu-baseline-tokens", type=int, default=1024)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy 3 times (scales rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
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
    from parallel_amd import _lib, load_balancing_loss_func, ops
    from parallel_amd.workloads import WORKLOADS, make_block_inputs

    w = WORKLOADS[args.config]
    if w.local_experts:
        raise SystemExit(f"{args.config} is a parity configuration, not a bench line; use c2, c4 or c5")
    dev = "cuda"
    torch.manual_seed(0)
    inp = make_block_inputs(w, seed=0, device=dev, dtype=torch.bfloat16, weights_on_device_rng=True)
    x = inp["x"].requires_grad_()
    rw = inp["router_weight"].requires_grad_()
    gu = inp["gate_up_proj"].requires_grad_()
    dn = inp["down_proj"].requires_grad_()
    d_out = inp["d_out"]
    bias = inp.get("logit_bias")
    coef = torch.tensor(w.aux_coef, device=dev)
    params = (x, rw, gu, dn)
    log(f"workload {w.name}: T={w.tokens} H={w.hidden} E={w.experts} k={w.top_k} I={w.intermediate}")

    def step():
        for p in params:
            p.grad = None
        logits, scores, idx = ops.router_fwd(x, rw, w.top_k, w.norm_topk_prob, bias)
        out = ops.experts(x, idx, scores, gu, dn)
        aux = load_balancing_loss_func((logits,), w.experts, w.top_k)
        torch.autograd.backward([out, aux], [d_out, coef])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"warm-up done ({args.warmup} steps)")

    _lib.TIMER.reset()
    _lib.TIMER.enabled = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.TIMER.enabled = False
    durations = _lib.TIMER.durations_ms()
    ms_per_step = 1e3 * elapsed / args.steps
    tokens_per_s = w.tokens * args.steps / elapsed
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step, {tokens_per_s:,.0f} tokens/s")

    work = kernel_work(w, w.tokens, w.slots)
    kernels = {}
    for tag, ds in sorted(durations.items()):
        avg = statistics.fmean(ds)
        kind, amount = work.get(tag, ("hbm", None))
        entry = {"avg_ms": round(avg, 4), "launches_per_step": len(ds) // args.steps}
        if amount is not None:
            rate = amount / (avg * 1e-3)
            if kind == "mfma":
                entry.update(tflops=round(rate / 1e12, 1), mfma_frac=round(rate / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4))
            else:
                entry.update(gbs=round(rate / 1e9, 1), hbm_frac=round(rate / 1e9 / HBM_PEAK_GBS, 4))
        kernels[tag] = entry
        log(f"  {tag:16s} {avg * 1e3:9.1f} us  {entry}")
    dominant = max(durations, key=lambda t: sum(durations[t]))
    kind, amount = work[dominant]
    avg_s = statistics.fmean(durations[dominant]) * 1e-3
    if kind == "mfma":
        achieved = amount / avg_s / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4)}
    else:
        achieved = amount / avg_s / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4)}
    roofline["kernel"] = dominant
    roofline["work_per_launch"] = amount
    roofline["traffic"] = read_traffic(dominant, w.name)
    gemm_tags = [t for t in ("up_fwd", "down_fwd", "down_dgrad", "down_wgrad", "up_dgrad", "up_wgrad") if t in durations]
    gemm_s = sum(statistics.fmean(durations[t]) for t in gemm_tags) * 1e-3
    gemm_tflops = w.gemm_flops() / gemm_s / 1e12 if gemm_s else None

    cpu = None
    if not args.no_cpu_baseline:
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
        "dtype": "bf16",
        "data": "synthetic (seeded normal inputs and weights)",
        "config": {"workload": f"{w.name}: Qwen3-30B-A3B MoE block" if w.name in ("c2", "c4") else w.name,
                   "tokens": w.tokens, "hidden": w.hidden, "experts": w.experts, "top_k": w.top_k,
                   "moe_intermediate": w.intermediate, "router_logits": "fp32", "aux_coef": w.aux_coef},
        "grouped_gemm": {"flops_fwd_bwd": w.gemm_flops(), "time_ms": round(gemm_s * 1e3, 4),
                         "tflops": round(gemm_tflops, 1) if gemm_tflops else None,
                         "mfma_frac": round(gemm_tflops / MFMA_BF16_PEAK_TFLOPS, 4) if gemm_tflops else None},
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
