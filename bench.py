#!/usr/bin/env python3
"""Benchmark of the Gemma-4 MoE decode hot path on one MI355X.

Prints ONE JSON line (rank 0, N=1):
  value        whole-job throughput (tok/s) with inputs resident in HBM
  roofline     the dominant kernel's achieved HBM GB/s (algorithmic bytes per
               launch / average launch time from HIP events in the timed region)
               against the 8 TB/s MI355X peak
  cpu_baseline the CPU oracle (the torch-CPU restatement of the reference's
               model.py) timed on this host's cores on a bounded sample

Workloads (--workload):
  moe_block  the isolated MoE decode block: hidden 2816, router 2816x128,
             128 experts top-8 of width 704, bf16, seed 1, batch --batch
             (1, 4 or 8); the hidden state of each step is drawn from a bank of
             1024 N(0,1) vectors so the routed experts change every step.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kaggle-tpu-inference_amd"))
sys.path.insert(0, ROOT)

METRIC = "batch-1 decode tok/s @32K ctx + MoE-decode HBM GB/s as % of MI355X peak"
HBM_PEAK_GBS = 8000.0


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _cpu_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# ------------------------------------------------------------------ moe block
class MoeBlock:
    H, E, K, F = 2816, 128, 8, 704
    SEED = 1
    BANK = 1024

    def __init__(self, batch: int):
        import torch

        from gemma4_mi import ops
        from gemma4_mi.weights import tensor_key

        self.torch, self.ops = torch, ops
        self.n = batch
        dev = "cuda:0"
        H, E, F = self.H, self.E, self.F

        def gen(shape, name, std):
            t = torch.empty(shape, dtype=torch.bfloat16, device=dev)
            ops.fill_normal_(t, tensor_key(self.SEED, name), std)
            return t

        self.proj = gen((E, H), "router.proj", 0.02)
        self.scale = torch.ones(H, dtype=torch.bfloat16, device=dev)
        self.pes = torch.ones(E, dtype=torch.bfloat16, device=dev)
        self.gate_up = gen((E, 2, F, H), "experts.gate_up_proj", 0.02)
        self.down = gen((E, H, F), "experts.down_proj", 0.02)
        self.bank = gen((self.BANK, batch, H), f"x.bank.n{batch}", 1.0)
        self.top_w = torch.empty((batch, self.K), dtype=torch.float32, device=dev)
        self.top_i = torch.empty((batch, self.K), dtype=torch.int32, device=dev)
        self.act = torch.empty((batch, self.K, F), dtype=torch.bfloat16, device=dev)
        self.out = torch.empty((batch, H), dtype=torch.bfloat16, device=dev)
        self.experts_seen = 0
        torch.cuda.synchronize()

    def step(self, i: int, ev=None):
        ops = self.ops
        x = self.bank[i % self.BANK]
        ops.moe_router_topk(x, self.scale, self.proj, self.pes, self.K, 1e-6, out=(self.top_w, self.top_i))
        if ev is not None:
            ev[0].record()
        ops.moe_gateup(x, self.gate_up, self.top_w, self.top_i, act=self.act)
        if ev is not None:
            ev[1].record()
        ops.moe_down(self.act, self.down, self.top_i, out=self.out)

    def unique_experts(self, steps: int) -> float:
        """Mean |union of routed experts| per step over the bank (for bytes)."""
        torch = self.torch
        tot = 0
        m = min(steps, self.BANK)
        for i in range(m):
            self.ops.moe_router_topk(self.bank[i], self.scale, self.proj, self.pes, self.K, 1e-6,
                                     out=(self.top_w, self.top_i))
            tot += int(torch.unique(self.top_i).numel())
        return tot / m

    def bytes_per_step(self, uniq: float) -> float:
        return self.E * self.H * 2 + uniq * 3 * self.F * self.H * 2

    def gateup_bytes(self) -> float:
        # weights of the selected (token, slot) rows + x + act written
        return self.n * self.K * 2 * self.F * self.H * 2 + self.n * self.H * 2 + self.n * self.K * self.F * 2

    def cpu_baseline(self, budget_s: float) -> dict:
        torch = self.torch
        from oracle import twin

        class C:
            hidden_size, num_experts, top_k_experts, moe_intermediate_size = self.H, self.E, self.K, self.F
            rms_norm_eps = 1e-6

        lp = {
            "router.proj": self.proj.cpu(), "router.scale": self.scale.cpu(),
            "router.per_expert_scale": self.pes.cpu(), "experts.gate_up_proj": self.gate_up.cpu(),
            "experts.down_proj": self.down.cpu(),
        }
        bank = self.bank.cpu()
        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        twin.moe(C, lp, bank[0], dense=False, precise=False)  # warm-up
        done, t0 = 0, time.perf_counter()
        while True:
            twin.moe(C, lp, bank[done % self.BANK], dense=False, precise=False)
            done += 1
            el = time.perf_counter() - t0
            if el >= budget_s and done >= 3:
                break
        return {
            "value": done * self.n / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{done} MoE-block steps of batch {self.n} (torch-CPU oracle, bf16 GEMMs) "
                      f"in {el:.1f}s on {_cpu_name()}",
        }


def run_moe_block(args) -> dict:
    import torch

    wl = MoeBlock(args.batch)
    _log(f"moe_block batch={args.batch}: weights ready")
    for i in range(args.warmup):
        wl.step(i)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        wl.step(args.warmup + i, evs[i])
    stop.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    gu_ms = sum(a.elapsed_time(b) for a, b in evs) / args.steps
    uniq = wl.unique_experts(args.steps)
    bps = wl.bytes_per_step(uniq)
    ms = total_ms / args.steps
    achieved = wl.gateup_bytes() / (gu_ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": args.batch / (ms * 1e-3),
        "unit": "tok/s",
        "ms_per_step": ms,
        "dtype": "bf16",
        "config": {
            "workload": "moe_decode_block", "hidden": wl.H, "experts": wl.E, "top_k": wl.K,
            "moe_intermediate": wl.F, "batch": args.batch, "seed": wl.SEED,
            "bytes_per_step": bps, "mean_unique_experts": uniq,
            "block_hbm_gbs": bps / (ms * 1e-3) / 1e9,
            "block_frac_of_peak": bps / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        },
        "roofline": {
            "kernel": "moe_gateup_kernel", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
            "bytes_per_launch": wl.gateup_bytes(), "avg_launch_us": gu_ms * 1e3,
        },
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = wl.cpu_baseline(args.cpu_seconds)
    return res


WORKLOADS = {"moe_block": run_moe_block}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="moe_block")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: this build has no multi-GPU path (--gpus {args.gpus} refused)",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    res = WORKLOADS[args.workload](args)
    line = {
        "metric": res.pop("metric"),
        "value": res.pop("value"),
        "unit": res.pop("unit"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res.pop("dtype"),
        "data": "synthetic (seeded random-init weights and inputs)",
        "config": res.pop("config"),
    }
    line.update(res)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
