"""Prefill/decode engine on one MI355X (gemma4_tpu/engine.py).

Same surface as the reference's Engine: the constructor, the attributes
callers read (cfg, max_len, batch, top_k, n_devices, params, cache,
load_seconds, param_bytes, cache_bytes, active_params, decode_step_seconds),
prefill_fn(t) / decode_fn() with the reference's calling convention,
reset_cache, _put, compile_all and the streaming generate() with lookahead
and the same event dicts (engine.py:26-221).

Each token step is a HIP graph of the library's kernels, captured once and
replayed:
  * "feed":  the layers with the dense-MoE combine (model.py:241-250), then
             the next prompt token is fed from a device buffer;
  * "head":  the same layers, lm_head and the sampler (or argmax), the
             token after a prefill (engine.py:60-67);
  * "decode": the layers with the decode path's bf16 running combine
             (model.py:262-294), lm_head and the sampler (or argmax);
             below SHORT_SPAN positions a second capture ("decode_short")
             whose full-attention layers are sized for SHORT_SPAN positions,
             and below TINY_SPAN a third ("decode_tiny") sized for TINY_SPAN
             (there the full layers' attention runs in one launch per layer,
             like the sliding layers').
The token, position and the whole token history stay on the device; the
host only replays graphs and copies each produced token into pinned memory,
so `lookahead` steps stay queued while it reads the oldest one.

Prefill (the default, prefill="batched") runs every prompt row through the
layers at once (model.PrefillRunner: MFMA GEMMs for the projections and the
dense-MoE experts, MFMA flash attention over the prompt rows), then the
head on the last row.  prefill="stepwise" instead feeds
the prompt one position at a time through the decode kernels with the
dense-MoE combine ("feed" graph, then "head").  Either way each prompt row
attends exactly the cached positions <= its own, the reference's causal
prefill; the prefill bucket is reported for compatibility but nothing is
padded.
"""

from __future__ import annotations

import time
from typing import Iterator

import torch

from . import model as M
from . import ops
from .config import TextConfig, load_text_config
from .limits import allowed_output_tokens
from .weights import active_params_per_token, init_random_params, load_params, param_bytes

PREFILL_BUCKET = 256
# Decode steps at positions below this replay a graph whose full-attention
# layers are sized for 8,192 positions (64 per split at 128 splits, one K tile
# per wave); later steps replay the max_len-sized graph.
SHORT_SPAN = 8192
# Below this position a third graph sizes the full-attention layers for 1,024
# positions, within reach of the one-launch attention (one XCD per KV head).
TINY_SPAN = 1024


def _round_up(x: int, m: int) -> int:
    return max(m, ((x + m - 1) // m) * m)


def _scalar(v) -> float:
    return float(v.item()) if isinstance(v, torch.Tensor) else float(v)


class Engine:
    def __init__(self, model_dir: str | None, max_len: int = 4096, batch: int = 1, top_k: int = 64, progress=None,
                 *, cfg: TextConfig | None = None, params: dict | None = None, device: str = "cuda:0",
                 prefill: str = "batched"):
        if batch < 1:
            raise ValueError("batch must be >= 1")
        if not 1 <= top_k <= 64:
            raise ValueError("top_k must be in [1, 64]")
        if prefill not in ("batched", "stepwise"):
            raise ValueError("prefill must be 'batched' or 'stepwise'")
        self.prefill_mode = prefill
        self.model_dir = model_dir
        self.cfg: TextConfig = cfg if cfg is not None else load_text_config(model_dir)
        self.max_len = int(max_len)
        self.batch = batch
        self.top_k = top_k
        self.device = torch.device(device)
        self.mesh = None
        self.n_devices = 1
        t0 = time.time()
        self.params = params if params is not None else load_params(self.cfg, model_dir, progress=progress,
                                                                    device=self.device)
        torch.cuda.synchronize(self.device)
        self.load_seconds = time.time() - t0
        self.cache = M.init_cache(self.cfg, None, batch, self.max_len, device=self.device)
        self.param_bytes = param_bytes(self.cfg)
        self.cache_bytes = M.cache_bytes(self.cfg, batch, self.max_len)
        self.active_params = active_params_per_token(self.cfg)
        self.decode_step_seconds = 0.0
        self._runner = M.DecodeRunner(self.cfg, self.params, self.cache, device=self.device,
                                      hist_len=self.max_len + 1)
        self._prompt = torch.zeros(self.max_len + 1, dtype=torch.int32, device=self.device)
        self._sp = ops.sample_params(0.0, 1.0, 0, self.device)
        self._sp_host = (0.0, 1.0, 0)
        self._graphs: dict[tuple, torch.cuda.CUDAGraph] = {}
        self._stream = torch.cuda.Stream(self.device)
        self._pos_host = 0
        # below this position the decode step replays a graph whose full
        # attention layers are sized for it (DecodeRunner.set_full_span)
        self._short_span = SHORT_SPAN if self.max_len > SHORT_SPAN else 0
        self._tiny_span = TINY_SPAN if self.max_len > TINY_SPAN else 0
        self._host_tok = torch.zeros(self.max_len + 1, dtype=torch.int32, pin_memory=True)
        self._prefill_runner: M.PrefillRunner | None = None
        # positions written per cache row since the last reset_cache()
        self._dirty = [0] * batch

    @classmethod
    def random(cls, cfg: TextConfig, seed: int = 3, max_len: int = 4096, top_k: int = 64, device: str = "cuda:0",
               prefill: str = "batched"):
        """An engine over seeded N(0, 0.02) random-init weights (no checkpoint)."""
        params = init_random_params(cfg, seed, device=device)
        return cls(None, max_len, 1, top_k, cfg=cfg, params=params, device=device, prefill=prefill)

    # ---------------------------------------------------------------- graphs
    def _graph(self, kind: str, greedy: bool) -> torch.cuda.CUDAGraph:
        key = (kind, greedy)
        g = self._graphs.get(key)
        if g is not None:
            return g
        r = self._runner
        sampler = None if greedy else (self._sp, self.top_k, 0 if kind == "head" else 1)

        def step():
            r.set_full_span({"decode_short": self._short_span, "decode_tiny": self._tiny_span}.get(kind) or None)
            try:
                if kind == "feed":
                    r.launch("f32", advance=True, feed=self._prompt)
                elif kind == "head":
                    r.launch("f32", advance=True, sampler=sampler)
                else:
                    r.launch("bf16_running", advance=True, sampler=sampler)
            finally:
                r.set_full_span(None)

        # warm the launch path once outside capture (library load, workspaces),
        # on a scratch position so no cache content the caller relies on changes
        saved_tok, saved_pos = r.tok.clone(), r.pos.clone()
        hist_save = r.hist.clone()
        r.pos.fill_(self.max_len - 1)
        torch.cuda.synchronize(self.device)
        s = self._stream
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream(self.device).wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
        r.tok.copy_(saved_tok)
        r.pos.copy_(saved_pos)
        r.hist.copy_(hist_save)
        # the warm step wrote K/V at the scratch position: clear those rows
        # again (only them: the rest of their page may hold the request's
        # positions, which the captured step is about to attend)
        self._zero_position(0, self.max_len - 1)
        torch.cuda.synchronize(self.device)
        self._graphs[key] = g
        return g

    def _set_sampling(self, key, temperature, top_p) -> bool:
        """Updates the device sampling parameters; returns True for greedy."""
        t, p, seed = _scalar(temperature), _scalar(top_p), int(key) if key is not None else 0
        if (t, p, seed) != self._sp_host:
            ops.sample_params(t, p, seed, self.device, out=self._sp)
            self._sp_host = (t, p, seed)
        return t <= 0.0

    # ---------------------------------------------------------------- steps
    def _prefill_for(self, n: int) -> M.PrefillRunner:
        """The batched prefill runner, grown to a multiple of the bucket >= n."""
        pr = self._prefill_runner
        if pr is None or pr.capacity < n:
            cap = min(self.max_len, _round_up(n, PREFILL_BUCKET))
            self._prefill_runner = pr = None
            pr = M.PrefillRunner(self.cfg, self.params, self.cache, cap, device=self.device,
                                 rope=self._runner.rope)
            self._prefill_runner = pr
        return pr

    def _build_prefill(self, t: int):
        r = self._runner

        def fn(params, tokens, cache, prompt_len, key, temperature, top_p):
            if params is not self.params or cache is not self.cache:
                raise ValueError("prefill_fn runs on the engine's own params and cache")
            n = int(_scalar(prompt_len))
            if not 1 <= n <= min(t, self.max_len):
                raise ValueError(f"prompt_len {n} outside [1, {min(t, self.max_len)}]")
            rows = torch.as_tensor(tokens)
            rows = rows.reshape(1, -1) if rows.ndim < 2 else rows.reshape(rows.shape[0], -1)
            if rows.shape[0] > self.batch or rows.shape[1] < n:
                raise ValueError(f"tokens {tuple(rows.shape)} for batch {self.batch} and prompt_len {n}")
            # rows 1.. (engine.py:60-67 runs every row of tokens [B, t]) fill
            # their own cache rows; the token comes from row 0, as there
            for b in range(1, rows.shape[0]):
                pb = self._prefill_for(n)
                self._prompt[:n].copy_(rows[b, :n].to(torch.int32))
                pb.run(self._prompt, n, seq=b)
                self._dirty[b] = max(self._dirty[b], n)
            toks = rows[0, :n].to(torch.int32)
            self._prompt[:n].copy_(toks)
            greedy = self._set_sampling(key, temperature, top_p)
            r.hist[:n].copy_(self._prompt[:n])
            if self.prefill_mode == "batched":
                # every prompt row through the layers at once, then the head on row n-1
                pr = self._prefill_for(n)
                pr.run(self._prompt, n)
                r.pos.fill_(n - 1)
                r.head(*pr.last_row(n), sampler=None if greedy else (self._sp, self.top_k, 0))
            else:
                r.tok.copy_(self._prompt[:1])
                r.pos.zero_()
                feed = self._graph("feed", True)
                for _ in range(n - 1):
                    feed.replay()
                self._graph("head", greedy).replay()
            self._pos_host = n
            self._dirty[0] = max(self._dirty[0], n)
            return r.hist[n:n + 1].view(1, 1), cache, torch.tensor(n, dtype=torch.int32)

        return fn

    def _build_decode(self):
        r = self._runner

        def fn(params, token, cache, pos, key, temperature, top_p):
            if params is not self.params or cache is not self.cache:
                raise ValueError("decode_fn runs on the engine's own params and cache")
            p = int(_scalar(pos))
            if not 0 <= p < self.max_len:
                raise ValueError(f"position {p} outside the cache (max_len {self.max_len})")
            tok_t = token if isinstance(token, torch.Tensor) else torch.as_tensor(token)
            own = tok_t.device == self.device and tok_t.data_ptr() == r.hist[p:p + 1].data_ptr()
            if not own:  # a token that is not the last step's output: write it into the history
                r.hist[p:p + 1].copy_(tok_t.reshape(-1)[:1].to(torch.int32))
            if not own or p != self._pos_host:
                r.tok.copy_(r.hist[p:p + 1])
                r.pos.fill_(p)
            greedy = self._set_sampling(key, temperature, top_p)
            kind = "decode_tiny" if p < self._tiny_span else ("decode_short" if p < self._short_span else "decode")
            self._graph(kind, greedy).replay()
            self._pos_host = p + 1
            self._dirty[0] = max(self._dirty[0], p + 1)
            return r.hist[p + 1:p + 2].view(1, 1), cache, torch.tensor(p + 1, dtype=torch.int32)

        return fn

    def prefill_fn(self, t: int):
        """fn(params, tokens[B,t] int32, cache, prompt_len, key, temperature, top_p)
        -> (tok [1,1] int32, cache, prompt_len) (engine.py:57-67).  `key` is an
        integer seed; the cache is updated in place and returned."""
        return self._build_prefill(int(t))

    def decode_fn(self):
        """fn(params, token[1,1] int32, cache, pos, key, temperature, top_p)
        -> (tok [1,1] int32, cache, pos + 1) (engine.py:71-83).  Decodes cache
        row 0 (the reference's engine samples logits[0, 0] and keeps one
        scalar position, engine.py:74-81)."""
        return self._build_decode()

    # ---------------------------------------------------------------- helpers
    def _zero_pages(self, b: int, lo: int, hi: int) -> None:
        """Zeroes the pages of cache row b that hold positions [lo, hi)."""
        page, mp = self.cache["page_size"], self.cache["page_table"].shape[1]
        p0, p1 = b * mp + lo // page, b * mp + (hi + page - 1) // page
        for t in self.cache["k"] + self.cache["v"]:
            t[p0:p1].zero_()

    def _zero_position(self, b: int, p: int) -> None:
        """Zeroes the K/V rows of position p of cache row b (pools [pages, KV, page, D])."""
        page, mp = self.cache["page_size"], self.cache["page_table"].shape[1]
        for t in self.cache["k"] + self.cache["v"]:
            t[b * mp + p // page, :, p % page].zero_()

    def reset_cache(self):
        """A zero cache again (engine.py:96-97 builds a new one; here the
        captured graphs keep these buffers, so they are cleared in place).
        Only the pages written since the last reset are zeroed: no kernel
        reads a position before the current request writes it, and a full
        clear of a 32K cache would move 7.4 GB per request."""
        for b, d in enumerate(self._dirty):
            if d:
                self._zero_pages(b, 0, d)
            self._dirty[b] = 0
        self._runner.hist.zero_()
        self._pos_host = 0

    def _put(self, value, dtype=torch.int32):
        return torch.as_tensor(value, dtype=dtype, device=self.device)

    def compile_all(self, bucket: int = PREFILL_BUCKET) -> dict[str, float]:
        """Captures the step graphs and times one decode step (engine.py:102-140)."""
        out = {}
        toks = torch.zeros((self.batch, bucket), dtype=torch.int32)
        t0 = time.perf_counter()
        if self.prefill_mode == "batched":
            # the prefill paths of a short and a full bucket once, so the first
            # request finds every kernel loaded
            for n in sorted({min(32, bucket), bucket}):
                self.prefill_fn(bucket)(self.params, toks, self.cache, n, 0, 0.0, 1.0)
        tok, self.cache, pos = self.prefill_fn(bucket)(self.params, toks, self.cache, 4, 0, 0.0, 1.0)
        if self.prefill_mode == "stepwise":
            self._graph("head", False)
        torch.cuda.synchronize(self.device)
        out["prefill_compile_s"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        tok, self.cache, pos = self.decode_fn()(self.params, tok, self.cache, pos, 0, 0.0, 1.0)
        self._graph("decode", False)
        if self._short_span:
            self._graph("decode_short", False)
        if self._tiny_span:
            self._graph("decode_tiny", False)
        torch.cuda.synchronize(self.device)
        out["decode_compile_s"] = time.perf_counter() - t0
        n = 8
        dec = self.decode_fn()
        t0 = time.perf_counter()
        for _ in range(n):
            tok, self.cache, pos = dec(self.params, tok, self.cache, pos, 0, 0.0, 1.0)
        torch.cuda.synchronize(self.device)
        self.decode_step_seconds = (time.perf_counter() - t0) / n
        out["decode_step_s"] = self.decode_step_seconds
        self.reset_cache()
        return out

    # ---------------------------------------------------------------- generation
    def generate(self, prompt_ids: list[int], max_new_tokens: int = 512, temperature: float = 1.0,
                 top_p: float = 0.95, seed: int = 0, stop_ids: tuple[int, ...] | None = None,
                 lookahead: int = 3) -> Iterator[dict]:
        """Yields one event per generated token (engine.py:143-221).  Decode
        steps are queued `lookahead` ahead of the host read; each step's token
        is copied to pinned host memory behind an event."""
        stop = set(stop_ids if stop_ids is not None else self.cfg.eos_token_ids)
        p_len = len(prompt_ids)
        available = self.max_len - p_len
        if available < 1:
            raise ValueError(f"prompt({p_len}) fills the resident context ({self.max_len})")
        max_new_tokens = allowed_output_tokens(max_new_tokens, p_len, self.max_len)
        bucket = min(_round_up(p_len, PREFILL_BUCKET), self.max_len)
        self.reset_cache()
        toks = torch.tensor(list(prompt_ids), dtype=torch.int32)
        t_start = time.perf_counter()
        tok, self.cache, pos = self.prefill_fn(bucket)(self.params, toks, self.cache, p_len, seed, temperature,
                                                       top_p)
        first = int(tok.item())
        ttft = time.perf_counter() - t_start
        yield {"kind": "prefill", "token": first, "ttft": ttft, "prompt_tokens": p_len, "prefill_bucket": bucket,
               "t": time.perf_counter()}
        if first in stop:
            return
        decode = self.decode_fn()
        stream = torch.cuda.current_stream(self.device)
        pending: list[tuple[int, torch.cuda.Event]] = []
        emitted = 1
        for _ in range(max_new_tokens - 1):
            tok, self.cache, pos = decode(self.params, tok, self.cache, pos, seed, temperature, top_p)
            p = int(pos)
            self._host_tok[p:p + 1].copy_(tok.reshape(-1), non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(stream)
            pending.append((p, ev))
            while len(pending) > lookahead:
                q, e = pending.pop(0)
                e.synchronize()
                value = int(self._host_tok[q])
                emitted += 1
                yield {"kind": "decode", "token": value, "index": emitted - 1, "t": time.perf_counter(),
                       "total_tokens": emitted}
                if value in stop:
                    stream.synchronize()
                    return
        for q, e in pending:
            e.synchronize()
            value = int(self._host_tok[q])
            emitted += 1
            yield {"kind": "decode", "token": value, "index": emitted - 1, "t": time.perf_counter(),
                   "total_tokens": emitted}
            if value in stop:
                stream.synchronize()
                return
