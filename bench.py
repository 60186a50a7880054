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
  decode     (default) the 26B-A4B-shaped model (30 layers: 25 sliding window
             1024 / 5 full k==v; hidden 2816; 128 experts top-8 of width 704
             beside a 2112 dense MLP; vocab 262,144), random-init bf16 weights
             N(0, 0.02), seed 3, 47 GiB in HBM; a 32,768-position cache; a
             54-token uniform-random prompt, then greedy batch-1 decode:
             warm-up steps + timed steps = 768 tokens.  value = decode tok/s.
             config.decode_118_822: the same stream timed over positions
             118-822 (704 steps) whatever --steps is.
             config.filled_cache_decode: the same engine after every cache
             page is filled with N(0,1), 64 timed steps at positions
             32,703-32,766 (full layers attending ~32.7K positions).
             roofline.moe_block: the isolated MoE block (below) at batches
             1, 4 and 8, 1,000 steps each.
  moe_block  the isolated MoE decode block: hidden 2816, router 2816x128,
             128 experts top-8 of width 704, bf16, seed 1, batch --batch
             (1, 4 or 8).  One HIP graph holds up to 64 consecutive steps, each
             on its own N(0,1) hidden state, so the routed experts change every
             step (the 1.5 GB expert table is 6x the 256 MB Infinity Cache).
  copy       a 1 GiB device-to-device copy of known size: the calibration run
             for the HBM byte counters (FETCH_SIZE / WRITE_SIZE).
  prefill    the batched prefill of the 26B-A4B-shaped model (seed 4) over
             --prompt-len uniform-random tokens (2048 for the prefill +
             batched-decode configuration); value = prompt tok/s, roofline =
             the dense-MoE prefill block against HBM (the selected experts'
             weight bytes) or MFMA (useful TFLOP/s), whichever its FLOP per
             weight byte puts it under; both figures are in the object.
  gateup     the decode expert gate/up kernel alone (rocprofv3 counter runs).
  batch_decode  batched greedy decode (seed 4): --batch sequences (default
             8) at --prompt-len positions each (8192 for the prefill +
             batched-decode configuration), --steps batched steps; value =
             aggregate tok/s.
  attention  isolated decode attention at position 32,767 (seed 2, softcap
             50): the sliding layer (16 q / 8 KV heads, head_dim 256, window
             1024) and the full k==v layer (16 q / 2 KV heads, head_dim 512);
             value = the full layer's GB/s of attended K/V bytes.
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
WINDOW = (118, 822)  # decode positions timed as a fixed window in every decode run


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


# ------------------------------------------------------------------ helpers
def _chunk(steps: int, cap: int = 64) -> int:
    """Largest divisor of `steps` that is <= cap (steps per captured graph)."""
    for g in range(min(cap, steps), 0, -1):
        if steps % g == 0:
            return g
    return 1


def _capture(fn):
    """Captures fn() (a sequence of launches on the current stream) in a HIP graph."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm: first-call allocations happen outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def _time_graph(g, replays: int) -> float:
    """ms for `replays` replays, bracketed by HIP events on the replay stream."""
    import torch

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b)


# ------------------------------------------------------------------ moe block
class MoeBlock:
    H, E, K, F = 2816, 128, 8, 704
    SEED = 1

    def __init__(self, batch: int, bank: int):
        import torch

        from gemma4_mi import ops
        from gemma4_mi.weights import tensor_key

        self.torch, self.ops = torch, ops
        self.n = batch
        self.nbank = bank
        dev = "cuda:0"
        H, E, F, K = self.H, self.E, self.F, self.K

        def gen(shape, name, std):
            t = torch.empty(shape, dtype=torch.bfloat16, device=dev)
            ops.fill_normal_(t, tensor_key(self.SEED, name), std)
            return t

        self.proj = gen((E, H), "router.proj", 0.02)
        self.scale = torch.ones(H, dtype=torch.bfloat16, device=dev)
        self.pes = torch.ones(E, dtype=torch.bfloat16, device=dev)
        self.gate_up = gen((E, 2, F, H), "experts.gate_up_proj", 0.02)
        self.down = gen((E, H, F), "experts.down_proj", 0.02)
        self.bank = gen((bank, batch, H), f"x.bank.n{batch}", 1.0)
        self.out = torch.empty((bank, batch, H), dtype=torch.bfloat16, device=dev)
        self.tw = torch.empty((bank, batch, K), dtype=torch.float32, device=dev)
        self.ti = torch.empty((bank, batch, K), dtype=torch.int32, device=dev)
        self.scores = torch.empty((bank, batch, E), dtype=torch.float32, device=dev)
        self.act = torch.empty((bank, batch, K, F), dtype=torch.bfloat16, device=dev)
        torch.cuda.synchronize()

    def block(self, i: int):
        self.ops.moe_block(self.bank[i], self.scale, self.proj, self.pes, self.gate_up, self.down, self.K, 1e-6,
                           out=self.out[i], route=(self.tw[i], self.ti[i]))

    def gateup(self, i: int):
        self.ops.moe_gateup_routed(self.bank[i], self.scores[i], self.pes, self.gate_up, self.K, act=self.act[i],
                                   route=(self.tw[i], self.ti[i]))

    def bytes_per_step(self, steps: int) -> tuple[float, float]:
        """(mean algorithmic bytes per step, mean |union of experts|) over the bank."""
        torch = self.torch
        uniq = [int(torch.unique(self.ti[i]).numel()) for i in range(min(steps, self.nbank))]
        u = sum(uniq) / len(uniq)
        return self.E * self.H * 2 + u * 3 * self.F * self.H * 2 + 2 * self.n * self.H * 2, u

    def gateup_bytes(self) -> float:
        # selected rows of gate_up + x + scores read + act written
        n, K, F, H, E = self.n, self.K, self.F, self.H, self.E
        return n * K * 2 * F * H * 2 + n * H * 2 + n * E * 4 + n * K * F * 2

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
            twin.moe(C, lp, bank[done % self.nbank], dense=False, precise=False)
            done += 1
            el = time.perf_counter() - t0
            if el >= budget_s and done >= 3:
                break
        return {
            "value": done * self.n / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{done} MoE-block steps of batch {self.n} (torch-CPU oracle, bf16 GEMMs) "
                      f"in {el:.1f}s on {_cpu_name()}",
        }


def _moe_block_traffic() -> dict:
    """HBM bytes per step of the isolated MoE block by batch, from the
    committed rocprofv3 counter summary (lines `batch B: fetch F write W`,
    copy-calibrated bytes per step summed over the block's kernels)."""
    out = {}
    try:
        for line in open(os.path.join(ROOT, "profiles", "moe_block_26b_a4b_traffic.txt")):
            if line.startswith("batch ") and "fetch" in line:
                b = int(line.split(":", 1)[0].split()[1])
                f = line.split(":", 1)[1].split()
                out[b] = {"fetch": float(f[f.index("fetch") + 1]), "write": float(f[f.index("write") + 1])}
    except (OSError, ValueError, IndexError):
        return {}
    return out


def _moe_block_roofline(steps: int = 1000, batches=(1, 4, 8)) -> dict:
    """The isolated MoE decode block (router, experts, combine) at each batch:
    `steps` steps on rotating inputs in HIP graphs of 50, bytes per step (the
    router table, the distinct selected experts' rows, inputs and outputs),
    the fraction of the 8 TB/s peak, and the counter-measured HBM bytes."""
    import torch

    traffic = _moe_block_traffic()
    out = {"peak": HBM_PEAK_GBS, "unit": "GB/s", "steps": steps}
    for b in batches:
        G = _chunk(steps, 50)
        wl = MoeBlock(b, G)
        g = _capture(lambda: [wl.block(i) for i in range(G)])
        _time_graph(g, 2)
        us = _time_graph(g, steps // G) / steps * 1e3
        bps, uniq = wl.bytes_per_step(G)
        gbs = bps / (us * 1e-6) / 1e9
        t = traffic.get(b)
        out[f"batch_{b}"] = {"us_per_step": us, "bytes_per_step": bps, "mean_unique_experts": uniq,
                             "achieved": gbs, "frac": gbs / HBM_PEAK_GBS,
                             "traffic": (t["fetch"] + t["write"]) if t else None,
                             "traffic_fetch": t["fetch"] if t else None}
        _log(f"moe block batch {b}: {us:.2f} us/step, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.3f} of peak)")
        del g, wl
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    out["traffic_source"] = "profiles/moe_block_26b_a4b_traffic.txt (rocprofv3 FETCH_SIZE/WRITE_SIZE per step)"
    return out


def run_moe_block(args) -> dict:
    G = _chunk(args.steps)
    wl = MoeBlock(args.batch, G)
    _log(f"moe_block batch={args.batch}: weights ready; {G} steps per graph")
    g_block = _capture(lambda: [wl.block(i) for i in range(G)])
    _time_graph(g_block, max(1, args.warmup // G))
    total_ms = _time_graph(g_block, args.steps // G)
    ms = total_ms / args.steps
    bps, uniq = wl.bytes_per_step(G)
    if args.block_only:  # counter runs: the block's own launches only
        return {"metric": f"isolated MoE decode block tok/s (26B-A4B experts, batch {args.batch})",
                "value": args.batch / (ms * 1e-3), "unit": "tok/s", "ms_per_step": ms, "dtype": "bf16",
                "config": {"workload": "moe_decode_block", "batch": args.batch, "bytes_per_step": bps,
                           "mean_unique_experts": uniq}}
    # dominant kernel: the routed gate/up, G launches per graph on the same inputs
    for i in range(G):
        wl.ops.moe_router_scores(wl.bank[i], wl.scale, wl.proj, 1e-6, out=wl.scores[i])
    g_gu = _capture(lambda: [wl.gateup(i) for i in range(G)])
    _time_graph(g_gu, 2)
    gu_us = _time_graph(g_gu, max(1, args.steps // G)) / (max(1, args.steps // G) * G) * 1e3
    achieved = wl.gateup_bytes() / (gu_us * 1e-6) / 1e9
    res = {
        "metric": f"isolated MoE decode block tok/s (26B-A4B experts, batch {args.batch})",
        "value": args.batch / (ms * 1e-3),
        "unit": "tok/s",
        "ms_per_step": ms,
        "dtype": "bf16",
        "config": {
            "workload": "moe_decode_block", "hidden": wl.H, "experts": wl.E, "top_k": wl.K,
            "moe_intermediate": wl.F, "batch": args.batch, "seed": wl.SEED, "inputs_rotated": G,
            "bytes_per_step": bps, "mean_unique_experts": uniq,
            "block_hbm_gbs": bps / (ms * 1e-3) / 1e9,
            "block_frac_of_peak": bps / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "kernels_per_step": 3, "launch": "HIP graph",
        },
        "roofline": {
            "kernel": "moe_gateup_kernel (routed)", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
            "bytes_per_launch": wl.gateup_bytes(), "avg_launch_us": gu_us,
        },
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = wl.cpu_baseline(args.cpu_seconds)
    return res


def run_attention(args) -> dict:
    """Isolated decode attention, one query token at position 32,767 (seed 2),
    RoPE and softcap 50, over paged bf16 caches (64-position pages) filled
    with N(0, 1):
      (a) sliding layer: 16 q / 8 KV heads, head_dim 256, window 1024;
      (b) full layer: 16 q / 2 KV heads, head_dim 512, k==v, 32,768 cached
          positions (K and V rows stored separately, as the decode step does).
    Each case is the decode step's call (append of the new K/V row, then the
    split qk and pv kernels), --steps launches captured in HIP graphs and
    timed with HIP events.  Consecutive launches rotate over `caches`
    independent caches in one page pool (one page table each) holding at
    least 512 MiB of attended rows together, twice the 256 MB Infinity
    Cache, so every launch streams its K/V rows from HBM as a decode step
    does (a step visits 29 other layers between two visits of one cache).
    Algorithmic bytes per launch: the attended K and V rows,
    2 * positions * KV * D * 2 B.  value = (b)'s GB/s."""
    import torch
    from gemma4_mi import model as gm
    from gemma4_mi import ops
    from gemma4_mi.weights import tensor_key

    dev, seed, lmax, page, pos = "cuda:0", 2, 32768, 64, 32767
    rotate_bytes = 512 << 20
    cases = {
        "sliding": dict(NH=16, KV=8, D=256, window=1024, k_eq_v=False, theta=1e4, partial=1.0),
        "full": dict(NH=16, KV=2, D=512, window=0, k_eq_v=True, theta=1e6, partial=0.25),
    }
    steps = args.steps
    out = {}
    for name, c in cases.items():
        NH, KV, D = c["NH"], c["KV"], c["D"]

        def gen(shape, tag, std=1.0):
            t = torch.empty(shape, dtype=torch.bfloat16, device=dev)
            ops.fill_normal_(t, tensor_key(seed, f"attn.{name}.{tag}"), std)
            return t

        q_raw, k_raw = gen((1, NH, D), "q"), gen((1, KV, D), "k")
        v_raw = None if c["k_eq_v"] else gen((1, KV, D), "v")
        q_norm, k_norm = gen((D,), "q_norm", 0.5), gen((D,), "k_norm", 0.5)
        cos, sin = gm.rope_table(D, c["theta"], c["partial"], lmax, dev)
        span = min(pos + 1, c["window"]) if c["window"] else pos + 1
        nbytes = 2 * span * KV * D * 2
        n_caches = -(-rotate_bytes // nbytes)
        max_pages = lmax // page
        lo_page = (pos + 1 - span) // page  # first attended page
        per = max_pages - lo_page           # pages each cache holds (the attended ones)
        kp, vp = gen((n_caches * per, KV, page, D), "cache_k"), gen((n_caches * per, KV, page, D), "cache_v")
        pts = torch.full((n_caches, max_pages), -1, dtype=torch.int32, device=dev)
        pts[:, lo_page:] = torch.arange(n_caches * per, dtype=torch.int32, device=dev).view(n_caches, per)
        p_t = torch.tensor([pos], dtype=torch.int32, device=dev)
        ns = gm.decode_splits(KV, span)  # the decode step's split count for this layer
        ctx = torch.empty((1, NH, D), dtype=torch.bfloat16, device=dev)
        ws = torch.zeros(int(ops._lib.lib().g4mi_decode_attention_workspace_bytes(1, NH, D, lmax, ns)),
                         dtype=torch.uint8, device=dev)
        G = max(n_caches, (_chunk(steps) // n_caches) * n_caches)  # launches per graph, a multiple of n_caches

        def call(i):
            ops.decode_attention(q_raw, k_raw, v_raw, q_norm, k_norm, cos, sin, kp, vp, pts[i % n_caches:][:1], p_t,
                                 c["window"], 50.0, 1e-6, lmax, n_split_max=ns, append=True, ctx=ctx, ws=ws)

        g = _capture(lambda: [call(i) for i in range(G)])
        _time_graph(g, max(1, -(-args.warmup // G)))
        reps = max(1, steps // G)
        us = _time_graph(g, reps) / (reps * G) * 1e3
        out[name] = {"heads": NH, "kv_heads": KV, "head_dim": D, "window": c["window"], "k_eq_v": c["k_eq_v"],
                     "positions_attended": span, "splits": ns, "caches_rotated": n_caches,
                     "rotated_bytes": n_caches * nbytes, "launches_timed": reps * G, "us_per_launch": us,
                     "bytes_per_launch": nbytes, "gbs": nbytes / (us * 1e-6) / 1e9}
        _log(f"attention {name}: {us:.2f} us, {out[name]['gbs']:.0f} GB/s over {n_caches} caches")
        del kp, vp, g
        torch.cuda.empty_cache()
    full = out["full"]
    return {
        "metric": "isolated decode attention GB/s (full layer, 32K positions)",
        "value": full["gbs"],
        "unit": "GB/s",
        "ms_per_step": full["us_per_launch"] * 1e-3,
        "dtype": "bf16",
        "config": {"workload": "isolated decode attention at position 32767, softcap 50, seed 2, "
                               "caches rotated per launch (>= 512 MiB)", **out, "launch": "HIP graph"},
        "roofline": {
            "kernel": "attn_qk + attn_pv + attn_reduce (full layer, 32K positions)", "bound": "hbm",
            "achieved": full["gbs"],
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": full["gbs"] / HBM_PEAK_GBS,
            "traffic": _measured_traffic("attn_qk_kernel+attn_pv_kernel+attn_reduce_kernel<512>",
                                         "attention_32k_traffic.txt"),
            "bytes_per_launch": full["bytes_per_launch"], "avg_launch_us": full["us_per_launch"],
        },
    }


def run_copy(args) -> dict:
    import torch

    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(args.warmup):
        b.copy_(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    gbs = 2 * n / (ms * 1e-3) / 1e9
    return {
        "metric": "device copy GB/s (read + write)", "value": gbs, "unit": "GB/s", "ms_per_step": ms,
        "dtype": "u8", "config": {"workload": "copy_1GiB", "bytes_read": n, "bytes_written": n},
        "roofline": {"kernel": "copy", "bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None},
    }


# ------------------------------------------------------------------ full-model decode
def _e2e_decode(args) -> dict:
    """Batch-1 greedy decode of the 26B-A4B-shaped model with a 32K cache,
    through the Engine API (engine.py's compile_all / prefill_fn / decode_fn)."""
    import numpy as np
    import torch

    from gemma4_mi.config import gemma4_26b_a4b_config
    from gemma4_mi.engine import PREFILL_BUCKET, Engine
    from gemma4_mi.weights import decode_bytes, param_bytes

    cfg = gemma4_26b_a4b_config()
    seed, prompt_len = 3, args.prompt_len
    t0 = time.perf_counter()
    eng = Engine.random(cfg, seed=seed, max_len=args.max_len)
    _log(f"weights: {param_bytes(cfg) / 2**30:.1f} GiB generated, engine ready in {time.perf_counter() - t0:.1f}s")
    comp = eng.compile_all(PREFILL_BUCKET)
    _log("step graphs captured: " + ", ".join(f"{k}={v:.3f}" for k, v in comp.items()))
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab_size, size=prompt_len).tolist()
    bucket = max(PREFILL_BUCKET, ((prompt_len + PREFILL_BUCKET - 1) // PREFILL_BUCKET) * PREFILL_BUCKET)

    # TTFT: the prompt through the prefill graphs (dense-MoE combine), first token to the host
    toks_in = torch.tensor(prompt, dtype=torch.int32)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok, cache, pos = eng.prefill_fn(bucket)(eng.params, toks_in, eng.cache, prompt_len, seed, 0.0, 1.0)
    first = int(tok.item())
    ttft = time.perf_counter() - t0
    dec = eng.decode_fn()
    for _ in range(args.warmup):
        tok, cache, pos = dec(eng.params, tok, cache, pos, seed, 0.0, 1.0)
    torch.cuda.synchronize()
    p0 = int(pos)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        tok, cache, pos = dec(eng.params, tok, cache, pos, seed, 0.0, 1.0)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    p1 = int(pos)
    toks = eng._runner.hist[prompt_len: p1 + 1].cpu().tolist()
    # a fixed window of the same stream: positions 118-822 (704 steps), the
    # stretch the 704-step default run times after its 64 warm-up steps
    window = None
    w0, w1 = WINDOW
    if p1 <= w0 and w1 < args.max_len:
        while int(pos) < w0:
            tok, cache, pos = dec(eng.params, tok, cache, pos, seed, 0.0, 1.0)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(w1 - w0):
            tok, cache, pos = dec(eng.params, tok, cache, pos, seed, 0.0, 1.0)
        e1.record()
        torch.cuda.synchronize()
        wms = e0.elapsed_time(e1) / (w1 - w0)
        wbytes = float(np.mean([decode_bytes(cfg, p) for p in range(w0, w1)]))
        wgbs = wbytes / (wms * 1e-3) / 1e9
        window = {"positions_timed": [w0, w1], "steps": w1 - w0, "ms_per_token": wms, "tok_s": 1000.0 / wms,
                  "bytes_per_token": wbytes, "e2e_hbm_gbs": wgbs, "e2e_frac_of_roofline": wgbs / HBM_PEAK_GBS}
        _log(f"decode at positions {w0}-{w1 - 1}: {wms:.4f} ms/token ({1000.0 / wms:.1f} tok/s)")
    p2 = int(pos)
    # the median inter-token latency: up to 64 more steps with an event between
    # the graph replays (after the tokens above were read)
    n_itl = max(0, min(64, args.max_len - 1 - p2))
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n_itl + 1)]
    evs[0].record()
    for i in range(n_itl):
        tok, cache, pos = dec(eng.params, tok, cache, pos, seed, 0.0, 1.0)
        evs[i + 1].record()
    torch.cuda.synchronize()
    itl_median = float(np.median([evs[i].elapsed_time(evs[i + 1]) for i in range(n_itl)])) if n_itl else ms
    bytes_tok = float(np.mean([decode_bytes(cfg, p) for p in range(p0, p1)]))
    return {"cfg": cfg, "params": eng.params, "cache": eng.cache, "engine": eng, "ms": ms, "ttft": ttft,
            "first": first, "p0": p0, "p1": p1, "bytes_tok": bytes_tok, "tokens": toks, "prompt": prompt,
            "itl_median_ms": itl_median, "itl_median_positions": [p2, p2 + n_itl], "window": window}


def _filled_decode(res, steps: int = 64, warm: int = 4) -> dict:
    """The same engine decoding at the end of a filled cache: every K/V page
    of every layer is overwritten with N(0, 1) bf16 (a synthetic 32K-token
    history), the position is set to max_len - steps - warm - 1, and `steps`
    greedy steps are timed after `warm` untimed ones, so the full layers
    attend ~32,700 positions and the sliding layers their whole window."""
    import numpy as np
    import torch

    from gemma4_mi import ops
    from gemma4_mi.weights import decode_bytes, tensor_key

    eng, cfg = res["engine"], res["cfg"]
    max_len = eng.max_len
    for i, (k, v) in enumerate(zip(eng.cache["k"], eng.cache["v"])):
        ops.fill_normal_(k, tensor_key(5, f"bench.filled.k.{i}"), 1.0)
        ops.fill_normal_(v, tensor_key(5, f"bench.filled.v.{i}"), 1.0)
    eng._dirty[0] = max_len  # reset_cache clears the whole row
    p_start = max_len - steps - warm - 1
    dec = eng.decode_fn()
    tok = torch.tensor([[res["tokens"][-1]]], dtype=torch.int32)
    pos = p_start
    for _ in range(warm):
        tok, cache, pos = dec(eng.params, tok, eng.cache, pos, 3, 0.0, 1.0)
    torch.cuda.synchronize()
    p0 = int(pos)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        tok, cache, pos = dec(eng.params, tok, eng.cache, pos, 3, 0.0, 1.0)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    p1 = int(pos)
    bytes_tok = float(np.mean([decode_bytes(cfg, p) for p in range(p0, p1)]))
    gbs = bytes_tok / (ms * 1e-3) / 1e9
    _log(f"filled-cache decode at positions {p0}-{p1 - 1}: {ms:.3f} ms/token, {gbs:.0f} GB/s")
    return {"positions_timed": [p0, p1], "steps": steps, "warmup": warm, "ms_per_token": ms, "tok_s": 1000.0 / ms,
            "bytes_per_token": bytes_tok, "e2e_hbm_gbs": gbs, "e2e_frac_of_roofline": gbs / HBM_PEAK_GBS,
            "cache_fill": "N(0,1) bf16 in every K/V page of every layer (seed 5)"}


def _gateup_timing(cfg, params, n: int, steps: int) -> tuple[float, float]:
    """Average duration (us) of the decode path's expert gate/up kernel
    (moe_gateup_kernel with the routing that ffn_in selected) over `n`
    launches per graph cycling through the layers (different experts each
    launch, so the 1.5 GB expert tables defeat the MALL), and its algorithmic
    bytes per launch: the 8 experts' gate and up rows, the hidden state, the
    routing and the activations written."""
    import torch

    from gemma4_mi import ops
    from gemma4_mi.weights import tensor_key

    H, E, K, F = cfg.hidden_size, cfg.num_experts, cfg.top_k_experts, cfg.moe_intermediate_size
    L = cfg.num_hidden_layers
    xe = torch.empty((n, 1, H), dtype=torch.bfloat16, device="cuda:0")
    ops.fill_normal_(xe, tensor_key(7, "bench.xe"), 1.0)
    act = torch.empty((n, 1, K, F), dtype=torch.bfloat16, device="cuda:0")
    route = []
    lp = lambda i, k: params[f"layers.{i % L}.{k}"]  # noqa: E731
    for i in range(n):
        route.append(ops.moe_router_topk(xe[i], lp(i, "router.scale"), lp(i, "router.proj"),
                                         lp(i, "router.per_expert_scale"), K, cfg.rms_norm_eps))
    g = _capture(lambda: [ops.moe_gateup(xe[i], lp(i, "experts.gate_up_proj"), route[i][0], route[i][1], act=act[i])
                          for i in range(n)])
    _time_graph(g, 2)
    reps = max(1, steps // n)
    us = _time_graph(g, reps) / (reps * n) * 1e3
    nbytes = K * 2 * F * H * 2 + H * 2 + K * 8 + K * F * 2
    return us, nbytes


def _cpu_decode_baseline(res, budget_s: float, max_steps: int) -> dict:
    """The oracle (torch-CPU restatement of model.py, bf16 GEMMs) continuing the
    GPU's prefix: K/V of the prompt copied from the GPU cache, then greedy decode
    steps on the host cores until the budget is spent."""
    import numpy as np
    import torch

    from gemma4_mi import model as gm
    from oracle import twin

    cfg, params, cache = res["cfg"], res["params"], res["cache"]
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    t0 = time.perf_counter()
    cpu_params = {k: v.cpu() for k, v in params.items()}
    max_len = cache["max_len"]
    p = len(res["prompt"])
    ocache = {"k": [], "v": []}
    for i in range(cfg.num_hidden_layers):
        k, v = gm.cache_positions(cache, i)
        kk = torch.zeros((1,) + tuple(k.shape), dtype=torch.bfloat16)
        vv = torch.zeros_like(kk)
        kk[0, :p] = k[:p].cpu()
        vv[0, :p] = v[:p].cpu()
        ocache["k"].append(kk)
        ocache["v"].append(vv)
    _log(f"cpu baseline: state copied to host in {time.perf_counter() - t0:.1f}s")
    tok, pos = res["first"], p
    done, t_start, el = 0, None, 0.0
    oracle_tokens = []
    while done < max_steps:
        lg, ocache = twin.forward(cfg, cpu_params, np.array([[tok]]), np.array([pos]), ocache, pos,
                                  twin.decode_masks(cfg, max_len, pos), max_len, False, None, precise=False,
                                  inplace=True)
        tok, pos = twin.greedy(lg[0, 0]), pos + 1
        oracle_tokens.append(int(tok))
        if t_start is None:  # first step is the warm-up
            t_start = time.perf_counter()
            continue
        done += 1
        el = time.perf_counter() - t_start
        if el >= budget_s:
            break
    # the GPU's greedy tokens after the same first token (res["tokens"][0] is that token)
    gpu_tokens = res["tokens"][1:1 + len(oracle_tokens)]
    same = 0
    while same < min(len(gpu_tokens), len(oracle_tokens)) and gpu_tokens[same] == oracle_tokens[same]:
        same += 1
    return {
        "value": done / el if el > 0 else None, "unit": "tok/s", "cores": threads, "kind": "port",
        "tokens_compared": len(oracle_tokens), "tokens_identical_prefix": same,
        "oracle_tokens": oracle_tokens, "gpu_tokens": gpu_tokens,
        "sample": f"{done} batch-1 decode steps (after 1 warm-up) of the 26B-A4B-shaped model from position {p + 1}, "
                  f"attending the whole {max_len}-position cache as the reference's decode does; torch-CPU oracle "
                  f"with bf16 GEMMs on {threads} threads of {_cpu_name()}",
    }


def _measured_traffic(kernel: str, summary: str = "moe_gateup_26b_a4b_traffic.txt") -> float | None:
    """HBM bytes per launch of `kernel` from a committed rocprofv3 counter
    summary under profiles/ (FETCH_SIZE / WRITE_SIZE, copy-calibrated), or
    None."""
    path = os.path.join(ROOT, "profiles", summary)
    try:
        kv = dict(line.split(":", 1) for line in open(path) if ":" in line and not line.startswith("#"))
    except OSError:
        return None
    if kv.get("kernel", "").strip() != kernel:
        return None
    return float(kv["traffic_bytes_per_launch"])


def run_decode(args) -> dict:
    import numpy as np

    res = _e2e_decode(args)
    cfg = res["cfg"]
    ms = res["ms"]
    tps = 1000.0 / ms
    gu_us, gu_bytes = _gateup_timing(cfg, res["params"], 60, 600)
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    e2e_gbs = res["bytes_tok"] * tps / 1e9
    out = {
        "metric": METRIC,
        "value": tps,
        "unit": "tok/s",
        "ms_per_step": ms,
        "dtype": "bf16",
        "config": {
            "workload": "gemma4-26B-A4B-shaped random-init decode, batch 1, 32K resident cache",
            "layers": cfg.num_hidden_layers, "hidden": cfg.hidden_size, "experts": cfg.num_experts,
            "top_k": cfg.top_k_experts, "vocab": cfg.vocab_size, "max_len": args.max_len, "seed": 3,
            "prompt_len": args.prompt_len, "positions_timed": [res["p0"], res["p1"]],
            "ttft_s": res["ttft"], "itl_ms": ms, "itl_median_ms": res["itl_median_ms"],
            "itl_median_positions": res["itl_median_positions"],
            "bytes_per_token": res["bytes_tok"], "e2e_hbm_gbs": e2e_gbs,
            "e2e_frac_of_roofline": e2e_gbs / HBM_PEAK_GBS,
            "kernels_per_token": 7 * cfg.num_hidden_layers + 2, "launch": "HIP graph per token (Engine.decode_fn)",
            "prefill": "Engine.prefill_fn: batched (hand-written MFMA GEMMs, dense-MoE prefill on the selected "
                       "experts, MFMA prefill attention)",
            "first_tokens": res["tokens"][:8],
        },
        "roofline": {
            "kernel": "moe_gateup_kernel (8 selected experts x 1408 gate/up rows x 2816)", "bound": "hbm",
            "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            "traffic": _measured_traffic("moe_gateup_kernel"), "bytes_per_launch": gu_bytes, "avg_launch_us": gu_us,
            "traffic_source": "profiles/moe_gateup_26b_a4b_traffic.txt (rocprofv3 FETCH_SIZE/WRITE_SIZE)",
        },
    }
    if res["window"] is not None:
        out["config"]["decode_118_822"] = res["window"]
    elif [res["p0"], res["p1"]] == list(WINDOW):  # the main timing is that window
        out["config"]["decode_118_822"] = {"positions_timed": list(WINDOW), "steps": args.steps, "ms_per_token": ms,
                                           "tok_s": tps, "bytes_per_token": res["bytes_tok"], "e2e_hbm_gbs": e2e_gbs,
                                           "e2e_frac_of_roofline": e2e_gbs / HBM_PEAK_GBS}
    out["roofline"]["moe_block"] = _moe_block_roofline()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = _cpu_decode_baseline(res, args.cpu_seconds, 8)
    # after the CPU baseline, which reads the prompt's cache rows
    out["config"]["filled_cache_decode"] = _filled_decode(res)
    return out


def run_gateup(args) -> dict:
    """The decode path's expert gate/up kernel alone on the 26B-A4B expert
    tables (the roofline kernel of the decode workload; short, for rocprofv3
    counter runs)."""
    from gemma4_mi.config import gemma4_26b_a4b_config
    from gemma4_mi.weights import init_random_params

    cfg = gemma4_26b_a4b_config()
    params = init_random_params(cfg, 3, device="cuda:0")
    us, nbytes = _gateup_timing(cfg, params, 60, args.steps)
    gbs = nbytes / (us * 1e-6) / 1e9
    return {
        "metric": "expert gate/up kernel GB/s (algorithmic bytes)", "value": gbs, "unit": "GB/s",
        "ms_per_step": us * 1e-3, "dtype": "bf16",
        "config": {"workload": "moe_gateup_26b_a4b", "launches_per_graph": 60, "bytes_per_launch": nbytes},
        "roofline": {"kernel": "moe_gateup_kernel", "bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "traffic": None},
    }


def _prefill_flops(cfg, n: int) -> dict:
    """Useful FLOPs of an n-token prefill (model.py:333-386 over n rows): the
    projections, the dense MLP, the router, the selected experts' gate/up and
    down, and causal attention (QK^T and PV over each row's attended range)."""
    H, NH, I, F = cfg.hidden_size, cfg.num_attention_heads, cfg.intermediate_size, cfg.moe_intermediate_size
    out = {"proj": 0.0, "dense_mlp": 0.0, "router": 0.0, "experts": 0.0, "attention": 0.0}
    for lt in cfg.layer_types:
        d, kv = cfg.head_dim_for(lt), cfg.kv_heads_for(lt)
        rows = NH * d + kv * d * (1 if cfg.k_eq_v_for(lt) else 2)
        out["proj"] += 2.0 * n * H * rows + 2.0 * n * NH * d * H
        out["dense_mlp"] += 2.0 * n * H * 3 * I
        if cfg.enable_moe_block:
            out["router"] += 2.0 * n * H * cfg.num_experts
            out["experts"] += 2.0 * n * cfg.top_k_experts * 3 * F * H
        w = cfg.sliding_window if lt == "sliding_attention" else n
        attended = sum(min(t + 1, w) for t in range(n))
        out["attention"] += 2.0 * 2.0 * attended * NH * d
    out["total"] = sum(out.values())
    return out


def run_prefill(args) -> dict:
    """Prefill of the 26B-A4B-shaped model: --prompt-len uniform-random tokens
    (seed 4) through Engine.prefill_fn (batched: hand-written MFMA GEMMs, the
    dense-MoE prefill on the selected experts, MFMA prefill attention), first token sampled
    greedily.  value = prompt tok/s."""
    import numpy as np
    import torch

    from gemma4_mi import ops
    from gemma4_mi.config import gemma4_26b_a4b_config
    from gemma4_mi.engine import PREFILL_BUCKET, Engine

    cfg = gemma4_26b_a4b_config()
    seed, n = 4, args.prompt_len
    eng = Engine.random(cfg, seed=seed, max_len=args.max_len)
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab_size, size=n)
    toks = torch.tensor(prompt, dtype=torch.int32)
    bucket = max(PREFILL_BUCKET, ((n + PREFILL_BUCKET - 1) // PREFILL_BUCKET) * PREFILL_BUCKET)
    fn = eng.prefill_fn(bucket)
    for _ in range(max(1, args.warmup)):
        tok, _, _ = fn(eng.params, toks, eng.cache, n, seed, 0.0, 1.0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        tok, _, _ = fn(eng.params, toks, eng.cache, n, seed, 0.0, 1.0)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    first = int(tok.item())
    # the dense-MoE prefill block of one layer, HIP events around its launches
    pr = eng._prefill_runner
    lp = pr.layers[0]
    xe, tw, ti = pr.xe[:n], pr.top_w[:n], pr.top_i[:n]
    ops.moe_router_topk(xe, lp["router.scale"], lp["router.proj"], lp["router.per_expert_scale"],
                        cfg.top_k_experts, cfg.rms_norm_eps, out=(tw, ti))
    reps = 10
    ops.moe_prefill(xe, tw, ti, lp["experts.gate_up_proj"], lp["experts.down_proj"], out=pr.moe_out[:n])
    torch.cuda.synchronize()
    e0.record()
    for i in range(reps):
        lq = pr.layers[i % cfg.num_hidden_layers]
        ops.moe_prefill(xe, tw, ti, lq["experts.gate_up_proj"], lq["experts.down_proj"], out=pr.moe_out[:n])
    e1.record()
    torch.cuda.synchronize()
    moe_us = e0.elapsed_time(e1) / reps * 1e3
    fl = _prefill_flops(cfg, n)
    moe_flops = fl["experts"] / cfg.num_hidden_layers
    moe_tf = moe_flops / (moe_us * 1e-6) / 1e12
    # each selected expert's gate/up and down rows stream once per layer
    n_experts = int(torch.unique(ti).numel())
    w_bytes = n_experts * 3 * cfg.moe_intermediate_size * cfg.hidden_size * 2
    w_gbs = w_bytes / (moe_us * 1e-6) / 1e9
    intensity = moe_flops / w_bytes  # FLOP per weight byte; the bf16 ridge is 2500 / 8 = 312.5
    hbm_bound = intensity < 2500.0 / 8.0
    tfs = fl["total"] / (ms * 1e-3) / 1e12
    return {
        "metric": "prefill tok/s (batched prefill)",
        "value": n / (ms * 1e-3),
        "unit": "tok/s",
        "ms_per_step": ms,
        "dtype": "bf16",
        "config": {
            "workload": f"gemma4-26B-A4B-shaped random-init prefill of {n} tokens", "seed": seed,
            "prompt_len": n, "bucket": bucket, "max_len": args.max_len, "first_token": first,
            "useful_tflop": fl["total"] / 1e12, "useful_tflop_by_part": {k: v / 1e12 for k, v in fl.items()},
            "useful_tflops_per_s": tfs, "useful_frac_of_bf16_peak": tfs / 2500.0,
            "dense_moe_reference_tflop": 2.0 * n * cfg.num_experts * 3 * cfg.moe_intermediate_size
            * cfg.hidden_size * cfg.num_hidden_layers / 1e12,
        },
        "roofline": {
            "kernel": "moe_prefill (routing sort + grouped gate/up GEMM + grouped down GEMM + combine), one layer",
            "bound": "hbm" if hbm_bound else "mfma",
            "achieved": w_gbs if hbm_bound else moe_tf, "peak": HBM_PEAK_GBS if hbm_bound else 2500.0,
            "unit": "GB/s" if hbm_bound else "TFLOP/s",
            "frac": w_gbs / HBM_PEAK_GBS if hbm_bound else moe_tf / 2500.0,
            "traffic": None, "flops_per_launch": moe_flops, "expert_weight_bytes_per_launch": w_bytes,
            "selected_experts": n_experts, "flop_per_weight_byte": intensity, "avg_launch_us": moe_us,
            "mfma_tflops": moe_tf, "mfma_frac_of_bf16_peak": moe_tf / 2500.0,
        },
    }


def run_batch_decode(args) -> dict:
    """Batched greedy decode of the 26B-A4B-shaped model (seed 4): --batch
    sequences (8 by default) each prefilled with --prompt-len (default 8192)
    uniform-random tokens, then --steps batched steps (gemma4_mi.batch).
    value = aggregate tok/s (batch / step time)."""
    import numpy as np
    import torch

    from gemma4_mi.batch import BatchEngine
    from gemma4_mi.config import gemma4_26b_a4b_config
    from gemma4_mi.weights import active_params_per_token, init_random_params

    cfg = gemma4_26b_a4b_config()
    seed, B, ctx = 4, (args.batch if args.batch > 1 else 8), args.prompt_len
    max_len = ctx + args.warmup + args.steps + 64
    params = init_random_params(cfg, seed, device="cuda:0")
    eng = BatchEngine(cfg, params, batch=B, max_len=max_len, device="cuda:0")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for b in range(B):
        eng.add(b, np.random.default_rng(seed + b).integers(0, cfg.vocab_size, size=ctx).tolist())
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    _log(f"{B} sequences prefilled ({ctx} tokens each) in {prefill_s:.2f}s")
    for _ in range(args.warmup):
        eng.step()
    torch.cuda.synchronize()
    p0 = eng.pos_host[0]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        eng.step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    p1 = eng.pos_host[0]
    # algorithmic bytes per step: shared weights once, the union of the routed experts per layer (expected
    # value under uniform routing), and each sequence's window-clamped K/V
    H, E, K, F, L = (cfg.hidden_size, cfg.num_experts, cfg.top_k_experts, cfg.moe_intermediate_size,
                     cfg.num_hidden_layers)
    expert_bytes = 3 * F * H * 2
    shared = 2 * active_params_per_token(cfg) - L * K * expert_bytes
    union = E * (1.0 - (1.0 - K / E) ** B)
    pos_mid = (p0 + p1) // 2
    kv = 0
    for lt in cfg.layer_types:
        n = pos_mid + 1 if lt != "sliding_attention" else min(pos_mid + 1, cfg.sliding_window)
        kv += 2 * 2 * cfg.kv_heads_for(lt) * cfg.head_dim_for(lt) * n
    step_bytes = shared + L * union * expert_bytes + B * kv
    gbs = step_bytes / (ms * 1e-3) / 1e9
    return {
        "metric": "batched decode aggregate tok/s",
        "value": B / (ms * 1e-3),
        "unit": "tok/s",
        "ms_per_step": ms,
        "dtype": "bf16",
        "config": {
            "workload": f"gemma4-26B-A4B-shaped random-init batched greedy decode, {B} sequences at ~{ctx} positions",
            "seed": seed, "batch": B, "context": ctx, "positions_timed": [p0, p1], "prefill_s": prefill_s,
            "step_bytes": step_bytes, "expected_union_experts_per_layer": union,
        },
        "roofline": {"kernel": "whole batched decode step", "bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "traffic": None},
    }


def run_decode_eager(args) -> dict:
    """The batch-1 decode step of the 26B-A4B-shaped model launched kernel by
    kernel on the stream (no HIP graph), at the positions the decode workload
    times (a 54-token prompt, then --steps greedy steps, the full layers sized
    for 8,192 positions as in the engine's short-span graph).  For per-kernel
    hardware counters: the launches are the decode graph's, in its order.
    value = tok/s of the eager launches (host launch cost included)."""
    import numpy as np
    import torch

    from gemma4_mi import model as gm
    from gemma4_mi.config import gemma4_26b_a4b_config
    from gemma4_mi.weights import init_random_params

    cfg = gemma4_26b_a4b_config()
    seed, p_len, steps = 3, args.prompt_len, args.steps
    params = init_random_params(cfg, seed, device="cuda:0")
    cache = gm.init_cache(cfg, None, 1, args.max_len, device="cuda:0")
    r = gm.DecodeRunner(cfg, params, cache, device="cuda:0")
    pr = gm.PrefillRunner(cfg, params, cache, 256, device="cuda:0", rope=r.rope)
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab_size, size=p_len)
    pr.run(torch.tensor(prompt, dtype=torch.int32, device="cuda:0"), p_len)
    r.pos.fill_(p_len - 1)
    r.head(*pr.last_row(p_len))
    r.set_full_span(min(8192, args.max_len))
    _log(f"prefill of {p_len} tokens done; {args.warmup} + {steps} eager steps")
    for _ in range(args.warmup):
        r.launch("bf16_running", advance=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        r.launch("bf16_running", advance=True)
        if steps <= 16:  # a counter-collecting profiler makes each step slow: show progress
            torch.cuda.synchronize()
            _log(f"eager step {i + 1}/{steps}")
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / max(steps, 1)
    return {"metric": "batch-1 decode tok/s, eager launches (profiling)", "value": 1000.0 / ms, "unit": "tok/s",
            "ms_per_step": ms, "dtype": "bf16",
            "config": {"workload": "gemma4-26B-A4B-shaped random-init decode, batch 1, eager launches",
                       "prompt_len": p_len, "positions": [p_len + args.warmup, p_len + args.warmup + steps]},
            "roofline": None}


WORKLOADS = {"decode": run_decode, "decode_eager": run_decode_eager, "moe_block": run_moe_block, "copy": run_copy, "gateup": run_gateup,
             "prefill": run_prefill, "batch_decode": run_batch_decode, "attention": run_attention}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (decode: 704, moe_block: 1000)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (decode: 64, moe_block: 100)")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="decode")
    ap.add_argument("--max-len", type=int, default=32768)
    ap.add_argument("--prompt-len", type=int, default=None,
                    help="prompt tokens (decode: 54, prefill: 2048, batch_decode: 8192 per sequence)")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--block-only", action="store_true",
                    help="moe_block: time the block only (no gate/up roofline leg, no CPU leg), for counter runs")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = {"decode": 704, "prefill": 5, "batch_decode": 256}.get(args.workload, 1000)
    if args.warmup is None:
        args.warmup = {"decode": 64, "prefill": 1, "batch_decode": 8}.get(args.workload, 100)
    if args.prompt_len is None:
        args.prompt_len = {"prefill": 2048, "batch_decode": 8192}.get(args.workload, 54)
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
