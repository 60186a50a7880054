"""Batched decode of several sequences, each at its own position.

The reference's Engine fills batch row 0 only and keeps one scalar position
(engine.py:74-81, 167-168); `forward` accepts B > 1 only with one shared
position and mask (model.py:402-408).  This module adds what serving several
prompts at once needs:

  PagePool           a free-list page allocator over the cache pools: each
                     sequence's page-table row is mapped on demand, so
                     sequences of different lengths share one pool
                     (model.py:174-185 keeps a dense [B, max_len] cache);
  BatchDecodeRunner  one greedy token for every sequence per step: the
                     layer math of model.py:297-322 over B rows (the prefill
                     row kernels, MFMA GEMMs at M = B for the projections and
                     the lm_head, decode attention with per-sequence
                     positions, the router and the selected-expert GEMVs of
                     the decode path with the bf16 running combine), then a
                     per-row softcap + argmax;
  BatchEngine        prefill per sequence (the batched prefill into that
                     sequence's pages, then its first token), batched decode
                     steps, and generate() over a list of prompts.
"""

from __future__ import annotations

import torch

from . import model as M
from .config import FULL, SLIDING, TextConfig


class PagePool:
    """Hands out cache pages to sequences (page table rows start at -1: a
    position without a page is neither written nor attended)."""

    def __init__(self, cache: dict):
        self.cache = cache
        self.page = cache["page_size"]
        self.num_pages = cache["k"][0].shape[0]
        self.batch, self.max_pages = cache["page_table"].shape
        self.free = list(range(self.num_pages - 1, -1, -1))
        self.owned: list[list[int]] = [[] for _ in range(self.batch)]
        cache["page_table"].fill_(-1)

    def ensure(self, b: int, n_positions: int) -> None:
        """Maps pages so that positions [0, n_positions) of sequence b exist."""
        need = (n_positions + self.page - 1) // self.page
        if need > self.max_pages:
            raise ValueError(f"sequence {b}: {n_positions} positions exceed the page table ({self.max_pages} pages)")
        have = len(self.owned[b])
        if need <= have:
            return
        if need - have > len(self.free):
            raise MemoryError(f"page pool exhausted ({self.num_pages} pages)")
        new = [self.free.pop() for _ in range(need - have)]
        self.owned[b].extend(new)
        row = self.cache["page_table"][b]
        row[have:need].copy_(torch.tensor(new, dtype=torch.int32), non_blocking=False)

    def release(self, b: int) -> None:
        """Returns sequence b's pages to the pool and unmaps its row."""
        self.free.extend(reversed(self.owned[b]))
        self.owned[b] = []
        self.cache["page_table"][b].fill_(-1)

    def free_pages(self) -> int:
        return len(self.free)


class BatchDecodeRunner:
    """One greedy decode step for B sequences on the current stream: tok [B]
    at positions pos [B] (device) -> the next tokens in tok, pos += 1,
    hist[b, pos[b]] = tok[b]."""

    def __init__(self, cfg: TextConfig, params: dict, cache: dict, device="cuda", hist_len: int | None = None,
                 rope=None):
        from . import ops

        self.ops, self.cfg, self.params, self.cache = ops, cfg, params, cache
        self.device = dev = torch.device(device)
        self.B = B = cache["page_table"].shape[0]
        self.max_len = cache["max_len"]
        self.layers = [{k[len(f"layers.{i}."):]: v for k, v in params.items() if k.startswith(f"layers.{i}.")}
                       for i in range(cfg.num_hidden_layers)]
        H, bf = cfg.hidden_size, torch.bfloat16
        z = lambda *shape, dt=bf: torch.zeros(shape, dtype=dt, device=dev)  # noqa: E731
        self.x, self.x1, self.xn, self.xm, self.o = z(B, H), z(B, H), z(B, H), z(B, H), z(B, H)
        self.mlp_out = z(B, H)
        moe = cfg.enable_moe_block
        self.xe = z(B, H) if moe else None
        self.moe_out = z(B, H) if moe else None
        q_max = max(cfg.num_attention_heads * cfg.head_dim_for(lt) for lt in cfg.layer_types)
        kv_max = max(cfg.kv_heads_for(lt) * cfg.head_dim_for(lt) for lt in cfg.layer_types)
        self.q, self.ctx = z(B * q_max), z(B * q_max)
        self.k, self.v = z(B * kv_max), z(B * kv_max)
        self.act = z(B, cfg.intermediate_size)
        if moe:
            self.act_moe = z(B, cfg.top_k_experts, cfg.moe_intermediate_size)
            self.top_w = z(B, cfg.top_k_experts, dt=torch.float32)
            self.top_i = z(B, cfg.top_k_experts, dt=torch.int32)
        self.logits_bf = z(B, cfg.vocab_size)
        self.tok = z(B, dt=torch.int32)
        self.pos = z(B, dt=torch.int32)
        self.hist_len = hist_len if hist_len is not None else self.max_len + 1
        self.hist = z(B, self.hist_len, dt=torch.int32)
        self.rope = rope if rope is not None else {
            SLIDING: M.rope_table(cfg.head_dim, cfg.rope_theta_sliding, 1.0, self.max_len, dev),
            FULL: M.rope_table(cfg.global_head_dim, cfg.rope_theta_full, cfg.rope_partial_rotary_factor_full,
                               self.max_len, dev),
        }
        self.splits = {}
        ws = 0
        for lt in set(cfg.layer_types):
            kv = cfg.kv_heads_for(lt)
            span = min(cfg.sliding_window, self.max_len) if lt == SLIDING else self.max_len
            if lt == SLIDING:
                # 64-position splits: the 4-wave kernels, whose last block of a
                # head reduces the splits in order, so no reduce launch (8 rows
                # at a full 1,024 window: 6.34 -> 6.22 ms per step against 4
                # splits of 256 positions)
                ns = max(ops.attention_min_splits(span), (span + 63) // 64)
            else:
                ns = max(ops.attention_min_splits(span), min(max(1, 256 // (kv * B)), (span + 63) // 64))
            self.splits[lt] = ns
            ws = max(ws, ops._lib.lib().g4mi_decode_attention_workspace_bytes(
                B, cfg.num_attention_heads, cfg.head_dim_for(lt), self.max_len, ns))
        self.attn_ws = torch.zeros(ws, dtype=torch.uint8, device=dev)
        # the grouped experts (g4mi_moe_decode_grouped) read each selected expert
        # once per step; the per-pair kernels read it once per (row, slot) and
        # let the MALL serve the repeats.  Measured on the 26B shapes at ~8K
        # positions: 8 rows 1149 (per pair) vs 1128 tok/s (grouped: a sort and
        # a combine launch more), 16 rows 1414 vs 1604 tok/s.
        self.grouped_moe = B > 8

    def launch(self) -> None:
        ops, cfg, p = self.ops, self.cfg, self.params
        H, eps, NH, B = cfg.hidden_size, cfg.rms_norm_eps, cfg.num_attention_heads, self.B
        moe = cfg.enable_moe_block
        L = cfg.num_hidden_layers
        ops.rows_embed(self.tok, p["embed"], self.layers[0]["input_layernorm"], eps, self.x, self.xn)
        for i, lt in enumerate(cfg.layer_types):
            lp = self.layers[i]
            d, kv = cfg.head_dim_for(lt), cfg.kv_heads_for(lt)
            q = self.q[: B * NH * d].view(B, NH * d)
            k = self.k[: B * kv * d].view(B, kv * d)
            v = None if cfg.k_eq_v_for(lt) else self.v[: B * kv * d].view(B, kv * d)
            # q, k and v of the B rows in one launch (model.py:197-200)
            ws_ = [lp["q_proj"].reshape(NH * d, H), lp["k_proj"].reshape(kv * d, H)]
            outs = [q, k]
            if v is not None:
                ws_.append(lp["v_proj"].reshape(kv * d, H))
                outs.append(v)
            if B <= 16:
                ops.gemm_segments(self.xn, ws_, outs)
            else:
                for w_, o_ in zip(ws_, outs):
                    ops.prefill_gemm(self.xn, w_, o_)
            cos, sin = self.rope[lt]
            ctx = self.ctx[: B * NH * d].view(B, NH, d)
            ops.decode_attention(q.view(B, NH, d), k.view(B, kv, d), None if v is None else v.view(B, kv, d),
                                 lp["q_norm"], lp["k_norm"], cos, sin, self.cache["k"][i], self.cache["v"][i],
                                 self.cache["page_table"], self.pos, cfg.sliding_window if lt == SLIDING else 0,
                                 cfg.attn_logit_softcapping, eps, self.max_len, self.splits[lt], append=True, ctx=ctx,
                                 ws=self.attn_ws)
            ops.prefill_gemm(ctx.view(B, NH * d), lp["o_proj"].reshape(H, NH * d), self.o)
            ops.rows_post_attn(self.x, self.o, lp["post_attention_layernorm"], lp["pre_feedforward_layernorm"],
                               lp.get("pre_feedforward_layernorm_2"), eps, self.x1, self.xm, self.xe)
            gate, up = lp["mlp.gate_proj"], lp["mlp.up_proj"]
            ops.prefill_gemm(self.xm, gate, self.act, epilogue=ops.EP_GATED,
                             pair_offset=(up.data_ptr() - gate.data_ptr()) // 2, n=gate.shape[0])
            ops.prefill_gemm(self.act, lp["mlp.down_proj"], self.mlp_out)
            if moe:
                ops.moe_router_topk(self.xe, lp["router.scale"], lp["router.proj"], lp["router.per_expert_scale"],
                                    cfg.top_k_experts, eps, out=(self.top_w, self.top_i))
                if self.grouped_moe and B <= 16:  # each selected expert's rows once for all rows that chose it
                    ops.moe_decode_grouped(self.xe, self.top_w, self.top_i, lp["experts.gate_up_proj"],
                                           lp["experts.down_proj"], "bf16_running", out=self.moe_out)
                else:
                    ops.moe_gateup(self.xe, lp["experts.gate_up_proj"], self.top_w, self.top_i, act=self.act_moe)
                    ops.moe_down(self.act_moe, lp["experts.down_proj"], self.top_i, "bf16_running", out=self.moe_out)
            nxt = self.layers[i + 1]["input_layernorm"] if i + 1 < L else p["norm"]
            ops.rows_tail(self.x1, self.mlp_out, self.moe_out, lp.get("post_feedforward_layernorm_1"),
                          lp.get("post_feedforward_layernorm_2"), lp["post_feedforward_layernorm"],
                          lp["layer_scalar"], nxt, eps, self.x, self.xn)
        # xn is now the final norm's output: lm_head (model.py:381) + softcap + argmax
        ops.prefill_gemm(self.xn, p["embed"], self.logits_bf)
        ops.argmax_rows(self.logits_bf, cfg.final_logit_softcapping, self.tok, self.pos, self.hist)


class BatchEngine:
    """Greedy serving of up to `batch` sequences at once on one GPU.

    add(b, prompt) prefills sequence b into its own pages (the batched
    prefill) and samples its first token greedily; step() advances every
    sequence by one token; generate(prompts, n) does both for a list of
    prompts.  Pages come from a shared pool (pool_pages, default enough for
    every sequence to reach max_len)."""

    def __init__(self, cfg: TextConfig, params: dict, batch: int, max_len: int, device="cuda:0",
                 pool_pages: int | None = None):
        self.cfg, self.params = cfg, params
        self.device = torch.device(device)
        self.batch, self.max_len = batch, max_len
        page = M.PAGE_SIZE
        if pool_pages is None:
            pool_pages = batch * ((max_len + page - 1) // page)
        self.cache = M.init_cache(cfg, None, batch, max_len, device=self.device, num_pages=pool_pages)
        self.pool = PagePool(self.cache)
        self.runner = BatchDecodeRunner(cfg, params, self.cache, device=self.device)
        self._head = M.HeadRunner(cfg, params, self.device)
        self._prefill: M.PrefillRunner | None = None
        self._prompt = torch.zeros(max_len, dtype=torch.int32, device=self.device)
        self.pos_host = [0] * batch

    def add(self, b: int, prompt_ids) -> int:
        """Prefills sequence b (positions 0..n-1) and returns its first token."""
        n = len(prompt_ids)
        if not 1 <= n < self.max_len:
            raise ValueError(f"prompt of {n} tokens outside [1, {self.max_len - 1}]")
        self.pool.release(b)
        self.pool.ensure(b, n + 1)
        if self._prefill is None or self._prefill.capacity < n:
            cap = min(self.max_len, ((n + 255) // 256) * 256)
            self._prefill = None
            self._prefill = M.PrefillRunner(self.cfg, self.params, self.cache, cap, device=self.device,
                                            rope=self.runner.rope)
        self._prompt[:n].copy_(torch.as_tensor(list(prompt_ids), dtype=torch.int32))
        self._prefill.run(self._prompt, n, seq=b)
        r = self.runner
        r.hist[b, :n].copy_(self._prompt[:n])
        # the head on the last prompt row: the token after position n-1 -> tok[b], pos[b] = n, hist[b][n]
        h = self._head
        h.pos.fill_(n - 1)
        h.head(*self._prefill.last_row(n))
        r.tok[b:b + 1].copy_(h.tok)
        r.pos[b:b + 1].copy_(h.pos)
        r.hist[b, n:n + 1].copy_(h.tok)
        self.pos_host[b] = n
        return int(h.tok.item())

    def step(self) -> torch.Tensor:
        """One greedy token for every sequence; returns tok [B] (device)."""
        for b in range(self.batch):
            if self.pos_host[b] + 1 >= self.max_len:
                raise ValueError(f"sequence {b} reached max_len {self.max_len}")
            self.pool.ensure(b, self.pos_host[b] + 1)
        self.runner.launch()
        for b in range(self.batch):
            self.pos_host[b] += 1
        return self.runner.tok

    def generate(self, prompts: list, max_new_tokens: int) -> list[list[int]]:
        """Greedy tokens for each prompt: the first token after the prompt,
        then max_new_tokens - 1 batched steps (every sequence advances
        together; unused rows repeat the last prompt)."""
        if not 1 <= len(prompts) <= self.batch:
            raise ValueError(f"1 to {self.batch} prompts")
        rows = list(prompts) + [prompts[-1]] * (self.batch - len(prompts))
        for b, pr in enumerate(rows):
            self.add(b, pr)
        for _ in range(max_new_tokens - 1):
            self.step()
        torch.cuda.synchronize(self.device)
        out = []
        for b in range(len(prompts)):
            n = len(rows[b])
            out.append(self.runner.hist[b, n:n + max_new_tokens].cpu().tolist())
        return out
