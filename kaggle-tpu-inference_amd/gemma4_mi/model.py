"""Gemma-4 MoE text decoder on one MI355X (the model API of gemma4_tpu/model.py).

Parameter layout, cache, masks and sampling keep the reference's names and
signatures; the math runs in libg4mi's gfx950 kernels.
"""

from __future__ import annotations

import math
import os

import torch

from .config import FULL, SLIDING, TextConfig

NEG_INF = -1e30


# --------------------------------------------------------------------- primitives
def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """model.py:42-47 on a device tensor (bf16 or f32), through the library's
    row kernel: f32 normalisation with an exact sum of squares, optional
    weight (Gemma-4 multiplies by w, not 1 + w), cast back to x's dtype."""
    from . import ops

    return ops.rms_norm(x, weight, eps)


def gelu(x: torch.Tensor) -> torch.Tensor:
    """model.py:50-51: tanh-approximation GELU, computed in f32, x's dtype."""
    from . import ops

    return ops.gelu(x)


def rope_tables(positions, inv_freq) -> tuple[torch.Tensor, torch.Tensor]:
    """model.py:64-67: (cos, sin) f32 [T, D] of f32(pos) * inv_freq, halves
    duplicated, on the GPU (positions may be a host list or array)."""
    from . import ops

    pos = torch.as_tensor(positions)
    if not pos.is_cuda:
        pos = pos.to("cuda")
    return ops.rope_tables(pos, torch.as_tensor(inv_freq))


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """model.py:70-78: x [B, T, ..., D]; cos/sin [T, D] cast to x's dtype;
    x * c + rotate_half(x) * s with each op rounded to x's dtype."""
    from . import ops

    return ops.apply_rope(x, cos, sin)


class Mesh:
    """One-device stand-in for the reference's jax Mesh (model.py:159-161):
    the same attributes callers read (devices, axis_names, shape, size) and a
    no-op context manager, so `with mesh:` blocks run unchanged.  This build
    runs the model on one GPU; there is no tensor-parallel axis to shard."""

    def __init__(self, device: torch.device):
        import numpy as np

        self.devices = np.array([device], dtype=object)
        self.axis_names = ("tp",)
        self.shape = {"tp": 1}
        self.size = 1

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False

    def __repr__(self) -> str:
        return f"Mesh(devices={list(self.devices)}, axis_names={self.axis_names})"


def make_mesh() -> Mesh:
    """model.py:159-161: the mesh over the visible devices; here one GPU."""
    return Mesh(torch.device("cuda", 0))


# --------------------------------------------------------------------- layout
def param_shapes(cfg: TextConfig) -> dict[str, tuple[int, ...]]:
    """Canonical shapes of every parameter by flat name (model.py:84-117).

    q_proj [KV,G,D,H] puts query head j = kv*G + g (GQA map j -> j // G);
    experts.gate_up_proj [E,2,F,H] holds gate rows then up rows."""
    h = cfg.hidden_size
    shapes: dict[str, tuple[int, ...]] = {"embed": (cfg.vocab_size, h), "norm": (h,)}
    for i, lt in enumerate(cfg.layer_types):
        d = cfg.head_dim_for(lt)
        kv = cfg.kv_heads_for(lt)
        g = cfg.num_attention_heads // kv
        p = f"layers.{i}."
        for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                  "post_feedforward_layernorm"):
            shapes[p + n] = (h,)
        shapes[p + "layer_scalar"] = (1,)
        shapes[p + "q_proj"] = (kv, g, d, h)
        shapes[p + "k_proj"] = (kv, d, h)
        if not cfg.k_eq_v_for(lt):
            shapes[p + "v_proj"] = (kv, d, h)
        shapes[p + "o_proj"] = (h, kv, g, d)
        shapes[p + "q_norm"] = (d,)
        shapes[p + "k_norm"] = (d,)
        shapes[p + "mlp.gate_proj"] = (cfg.intermediate_size, h)
        shapes[p + "mlp.up_proj"] = (cfg.intermediate_size, h)
        shapes[p + "mlp.down_proj"] = (h, cfg.intermediate_size)
        if cfg.enable_moe_block:
            for n in ("pre_feedforward_layernorm_2", "post_feedforward_layernorm_1",
                      "post_feedforward_layernorm_2"):
                shapes[p + n] = (h,)
            shapes[p + "router.proj"] = (cfg.num_experts, h)
            shapes[p + "router.scale"] = (h,)
            shapes[p + "router.per_expert_scale"] = (cfg.num_experts,)
            shapes[p + "experts.gate_up_proj"] = (cfg.num_experts, 2, cfg.moe_intermediate_size, h)
            shapes[p + "experts.down_proj"] = (cfg.num_experts, h, cfg.moe_intermediate_size)
    return shapes


def cache_shapes(cfg: TextConfig, batch: int, max_len: int) -> list[tuple[int, ...]]:
    """Logical per-layer cache shape [B, max_len, KV, D] (model.py:174-175)."""
    return [(batch, max_len, cfg.kv_heads_for(lt), cfg.head_dim_for(lt)) for lt in cfg.layer_types]


def cache_bytes(cfg: TextConfig, batch: int, max_len: int) -> int:
    """bf16 bytes of the K and V caches (model.py:188-189)."""
    return sum(2 * 2 * math.prod(s) for s in cache_shapes(cfg, batch, max_len))


# --------------------------------------------------------------------- RoPE
def rope_inv_freq(head_dim: int, theta: float, partial_rotary_factor: float = 1.0):
    """Inverse frequencies (model.py:54-61): theta^(-2i/d) computed in f64 for
    the rotated pairs, zero for the NoPE tail of a partial rotation, as f32."""
    import numpy as np

    n_rot = int(partial_rotary_factor * head_dim // 2)
    inv = np.zeros(head_dim // 2, dtype=np.float64)
    if n_rot:
        inv[:n_rot] = 1.0 / (theta ** (np.arange(n_rot, dtype=np.float64) * 2.0 / head_dim))
    return inv.astype(np.float32)


def decode_splits(kv_heads: int, span: int) -> int:
    """Split count of the decode attention for a layer whose rows attend to at
    most `span` positions: ~256 blocks per KV pass at full length (one split
    per 64 positions below that), never fewer than the kernel's minimum."""
    from . import ops

    want = max(1, 256 // kv_heads)
    return max(ops.attention_min_splits(span), min(want, (span + 63) // 64))


def rope_table(head_dim: int, theta: float, partial: float, max_pos: int, device="cuda"):
    """(cos, sin) bf16 tables [max_pos, head_dim/2] of the angles
    f32(pos) * inv_freq (f32 product, model.py:65); each entry is the f64
    cosine/sine of that f32 angle rounded to f32, then to bf16 (the reference
    casts the tables to the activation dtype in apply_rope, model.py:76-77).
    The duplicated second half of the reference's table is not stored."""
    import numpy as np

    inv = rope_inv_freq(head_dim, theta, partial)
    ang = (np.arange(max_pos, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    cos = torch.from_numpy(np.cos(ang.astype(np.float64)).astype(np.float32))
    sin = torch.from_numpy(np.sin(ang.astype(np.float64)).astype(np.float32))
    return cos.to(torch.bfloat16).to(device), sin.to(torch.bfloat16).to(device)


# --------------------------------------------------------------------- cache
PAGE_SIZE = 64


def init_cache(cfg: TextConfig, mesh=None, batch: int = 1, max_len: int = 4096, dtype=torch.bfloat16,
               device="cuda", page_size: int = PAGE_SIZE, num_pages: int | None = None) -> dict:
    """Zero K and V caches, one pair per layer (model.py:178-185), stored as
    pages: k[i], v[i] are [num_pages, KV, PAGE, D] bf16 and
    cache["page_table"] [batch, max_pages] int32 maps position p of sequence
    b to page page_table[b, p // PAGE].  By default every sequence owns
    max_pages pages (num_pages = batch * max_pages, identity table); with a
    smaller shared pool the table starts unmapped (-1) and batch.PagePool
    hands pages out.  `mesh` is accepted for signature compatibility (one
    GPU, no mesh)."""
    if dtype != torch.bfloat16:
        raise ValueError("the cache is bf16")
    max_pages = (max_len + page_size - 1) // page_size
    pool = batch * max_pages if num_pages is None else int(num_pages)
    pools_k, pools_v = [], []
    for lt in cfg.layer_types:
        shape = (pool, cfg.kv_heads_for(lt), page_size, cfg.head_dim_for(lt))
        pools_k.append(torch.zeros(shape, dtype=torch.bfloat16, device=device))
        pools_v.append(torch.zeros(shape, dtype=torch.bfloat16, device=device))
    if num_pages is None:
        pt = torch.arange(batch * max_pages, dtype=torch.int32, device=device).reshape(batch, max_pages)
    else:
        pt = torch.full((batch, max_pages), -1, dtype=torch.int32, device=device)
    return {"k": pools_k, "v": pools_v, "page_table": pt, "page_size": page_size, "max_len": max_len,
            "batch": batch}


def cache_positions(cache: dict, layer: int, batch: int = 0, upto: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The logical [max_len, KV, D] K and V of one layer and sequence (for tests
    and inspection): pages gathered through the page table."""
    pt = cache["page_table"][batch].long()
    kp, vp = cache["k"][layer], cache["v"][layer]
    n, kv, page, d = kp.shape
    k = kp[pt].permute(0, 2, 1, 3).reshape(-1, kv, d)
    v = vp[pt].permute(0, 2, 1, 3).reshape(-1, kv, d)
    upto = cache["max_len"] if upto is None else upto
    return k[:upto], v[:upto]


# --------------------------------------------------------------------- masks
def prefill_masks(cfg: TextConfig, t: int, prompt_len) -> dict:
    """Causal masks of a t-token prefill (model.py:392-399): kv <= q, kv <
    prompt_len, and kv > q - window on sliding layers.  The kernels apply the
    same predicates implicitly; the dict also carries `prompt_len`."""
    q = torch.arange(t)[:, None]
    kv = torch.arange(t)[None, :]
    p = int(prompt_len)
    valid = (kv <= q) & (kv < p)
    return {FULL: valid[None, None, None], SLIDING: (valid & (kv > q - cfg.sliding_window))[None, None, None],
            "prompt_len": p}


def decode_masks(cfg: TextConfig, max_len: int, pos) -> dict:
    """Decode masks at position pos (model.py:402-408)."""
    kv = torch.arange(max_len)[None, :]
    p = int(pos)
    valid = kv <= p
    return {FULL: valid[None, None, None], SLIDING: (valid & (kv > p - cfg.sliding_window))[None, None, None],
            "pos": p}


# --------------------------------------------------------------------- sampling
def fold_in(key, data: int):
    """The per-step key of engine.py:66 and engine.py:80 (jax.random.fold_in):
    here the pair (seed, step).  sample() with it draws the uniform at
    Philox counter `step`, which is what the engine's decode step at
    position `step` draws (and step 0 after a prefill)."""
    seed = key[0] if isinstance(key, tuple) else int(key)
    return (int(seed), int(data))


def sample(logits: torch.Tensor, key, temperature, top_k: int, top_p) -> torch.Tensor:
    """model.py:414-424 on a device logits row [V] f32 -> int32 scalar (device).

    temperature <= 0: argmax, the first index of the maximum.  Otherwise the
    top_k of logits / max(T, 1e-6), softmax, the nucleus cut (exclusive
    prefix sum < top_p), renormalisation and one draw.  `key` is an integer
    seed or a (seed, step) pair from fold_in; the uniform comes from this
    library's Philox4x32-10 stream, not JAX's threefry, so stochastic draws
    match the reference in distribution, not bit for bit."""
    from . import ops

    lg = logits.reshape(-1)
    if lg.dtype != torch.float32 or not lg.is_contiguous():
        lg = lg.float().contiguous()
    dev = lg.device
    t = float(temperature.item()) if isinstance(temperature, torch.Tensor) else float(temperature)
    p = float(top_p.item()) if isinstance(top_p, torch.Tensor) else float(top_p)
    seed, step = key if isinstance(key, tuple) else (int(key), None)
    params = ops.sample_params(t, p, seed, dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    if step is None:
        ops.sample(lg, int(top_k), params, tok, counter_mode=0)
    else:
        ctr = torch.tensor([step], dtype=torch.int32, device=dev)
        ops.sample(lg, int(top_k), params, tok, counter_mode=1, pos=ctr)
    return tok.reshape(())


# --------------------------------------------------------------------- decode step
class DecodeRunner:
    """Launches one batch-1 token step of the model on the current stream.

    Per layer: layer_in (the previous layer's tail and this layer's input
    norm in every block's prologue, under its q/k/v row loads; the first
    layer embeds the token), decode attention (append + scores, then PV +
    the ordered split reduce), o_proj, ffn_in (post-attention norm, dense
    gate/up, router scores and the expert selection), routed expert gate/up,
    ffn_out (dense and expert down + combine); then lm_head (the last
    layer's tail and the final norm in its prologue) and the greedy argmax.
    All buffers are allocated once, so a step can be captured in a HIP graph
    and replayed; the token and position live in device memory (`tok`,
    `pos`)."""

    def __init__(self, cfg: TextConfig, params: dict, cache: dict, device="cuda", hist_len: int | None = None):
        from . import ops

        self.ops = ops
        self.cfg, self.params, self.cache = cfg, params, cache
        self.device = torch.device(device)
        dev = self.device
        H = cfg.hidden_size
        self.max_len = cache["max_len"]
        self.page_table = cache["page_table"][0:1].contiguous()
        self._bind_pages(0)
        self.layers = [{k[len(f"layers.{i}."):]: v for k, v in params.items() if k.startswith(f"layers.{i}.")}
                       for i in range(cfg.num_hidden_layers)]
        bf = torch.bfloat16
        qkv_max = max(cfg.num_attention_heads * cfg.head_dim_for(lt) + 2 * cfg.kv_heads_for(lt) * cfg.head_dim_for(lt)
                      for lt in cfg.layer_types)
        ctx_max = max(cfg.num_attention_heads * cfg.head_dim_for(lt) for lt in cfg.layer_types)
        z = lambda n, dt=bf: torch.zeros(n, dtype=dt, device=dev)  # noqa: E731
        self.x, self.x1, self.xe, self.o, self.xn = z(H), z(H), z(H), z(H), z(H)
        self.mlp_out, self.moe_out = z(H), z(H)
        self.qkv, self.ctx = z(qkv_max), z(ctx_max)
        self.act_mlp = z(cfg.intermediate_size)
        L = cfg.num_hidden_layers
        if cfg.enable_moe_block:
            self.act_moe = z(cfg.top_k_experts * cfg.moe_intermediate_size)
            self.scores = z(cfg.num_experts, torch.float32)
            self.top_w = z((L, cfg.top_k_experts), torch.float32)
            self.top_i = z((L, cfg.top_k_experts), torch.int32)
        self.logits = z(cfg.vocab_size, torch.float32)
        nb = ops.lm_head_blocks(cfg.vocab_size)
        self.blk_val, self.blk_idx = z(nb, torch.float32), z(nb, torch.int32)
        self.tok = z(1, torch.int32)
        self.pos = z(1, torch.int32)
        self.hist = z(hist_len if hist_len is not None else self.max_len + 1, torch.int32)
        # RoPE tables per layer type, and attention workspaces
        self.rope = {
            SLIDING: rope_table(cfg.head_dim, cfg.rope_theta_sliding, 1.0, self.max_len, dev),
            FULL: rope_table(cfg.global_head_dim, cfg.rope_theta_full, cfg.rope_partial_rotary_factor_full,
                             self.max_len, dev),
        }
        self.lmax = {SLIDING: min(cfg.sliding_window, self.max_len), FULL: self.max_len}
        self.splits = {}
        ws = 0
        for lt in set(cfg.layer_types):
            d = cfg.head_dim_for(lt)
            lmax = self.max_len  # positions are addressed up to max_len on every layer
            ns = self._splits(lt)
            self.splits[lt] = ns
            ws = max(ws, ops._lib.lib().g4mi_decode_attention_workspace_bytes(1, cfg.num_attention_heads, d, lmax, ns))
        self.attn_ws = torch.zeros(ws, dtype=torch.uint8, device=dev)
        # positions the full layers' attention is launched for (see set_full_span)
        self.full_span = self.max_len
        self.sample_ws = torch.zeros(ops.sample_workspace_bytes(cfg.vocab_size), dtype=torch.uint8, device=dev)
        self.ffn_ws = torch.zeros(int(ops._lib.lib().g4mi_ffn_in_workspace_bytes()), dtype=torch.uint8, device=dev)

    def _splits(self, lt: str) -> int:
        cfg = self.cfg
        span = min(cfg.sliding_window, self.max_len) if lt == SLIDING else self.max_len
        return decode_splits(cfg.kv_heads_for(lt), span)

    def set_full_span(self, span: int | None = None) -> None:
        """Steps launched from now on size the full-attention layers for
        positions below `span` (None: max_len).  A span up to 64 positions
        per split (8,192 at 128 splits) runs the attention kernels that take
        one K tile per wave; the full 32K span needs the long-range kernels
        and their split reduction.  A step at a position >= span attends to
        nothing on those layers, so a caller that captures a step with a
        short span replays it only below that position."""
        span = self.max_len if span is None else int(span)
        if not 1 <= span <= self.max_len:
            raise ValueError(f"span {span} outside [1, {self.max_len}]")
        self.full_span = span

    def launch(self, combine: str = "bf16_running", advance: bool = True, sampler=None, feed=None):
        """Enqueues one token step reading tok/pos.

        With `advance` the head writes the next token to tok, increments pos
        and records the token in hist[pos].  The head is the greedy argmax,
        or, with `sampler` = (params, top_k, counter_mode), the top-k/top-p
        sampler (model.py:414-424).  With `feed` (a device int32 prompt
        buffer) the step skips the lm_head and instead feeds the next prompt
        token: pos += 1, tok = feed[pos], hist[pos] = tok."""
        ops, cfg, p = self.ops, self.cfg, self.params
        H, eps, NH = cfg.hidden_size, cfg.rms_norm_eps, cfg.num_attention_heads
        moe = cfg.enable_moe_block
        for i, lt in enumerate(cfg.layer_types):
            lp = self.layers[i]
            d, kv = cfg.head_dim_for(lt), cfg.kv_heads_for(lt)
            q_rows, k_rows = NH * d, kv * d
            v_rows = 0 if cfg.k_eq_v_for(lt) else kv * d
            if i == 0:
                ops.layer_in(0, H, eps, lp["input_layernorm"], self.x, lp["q_proj"], lp["k_proj"], lp.get("v_proj"),
                             q_rows, k_rows, v_rows, self.qkv, tok=self.tok, embed=p["embed"])
            else:  # every block applies the previous layer's tail while its q/k/v rows stream in
                pl = self.layers[i - 1]
                ops.layer_in(1, H, eps, lp["input_layernorm"], self.x, lp["q_proj"], lp["k_proj"], lp.get("v_proj"),
                             q_rows, k_rows, v_rows, self.qkv, x1=self.x1, mlp_out=self.mlp_out,
                             moe_out=self.moe_out if moe else None, post_ff1=pl.get("post_feedforward_layernorm_1"),
                             post_ff2=pl.get("post_feedforward_layernorm_2"), post_ff=pl["post_feedforward_layernorm"],
                             layer_scalar=pl["layer_scalar"])
            q = self.qkv[:q_rows].view(1, NH, d)
            k = self.qkv[q_rows:q_rows + k_rows].view(1, kv, d)
            v = self.qkv[q_rows + k_rows:q_rows + k_rows + v_rows].view(1, kv, d) if v_rows else None
            cos, sin = self.rope[lt]
            ctx = self.ctx[:NH * d].view(1, NH, d)
            kp, vp = self.kv_pools[i]
            if lt == SLIDING or self.full_span == self.max_len:
                lmax, ns = self.max_len, self.splits[lt]
            else:
                lmax, ns = self.full_span, decode_splits(kv, self.full_span)
            ops.decode_attention(q, k, v, lp["q_norm"], lp["k_norm"], cos, sin, kp, vp,
                                 None if self.dense_pages else self.page_table, self.pos,
                                 cfg.sliding_window if lt == SLIDING else 0, cfg.attn_logit_softcapping, eps,
                                 lmax, ns, append=True, ctx=ctx, ws=self.attn_ws)
            ops.oproj(self.ctx, lp["o_proj"], H, NH * d, self.o)
            ops.ffn_in(self.x, self.o, lp["post_attention_layernorm"], lp["pre_feedforward_layernorm"],
                       lp.get("pre_feedforward_layernorm_2"), self.x1, self.xe, lp["mlp.gate_proj"],
                       lp["mlp.up_proj"], self.act_mlp, lp.get("router.scale"), lp.get("router.proj"),
                       self.scores if moe else None, H, eps,
                       per_expert_scale=lp["router.per_expert_scale"] if moe else None, k=cfg.top_k_experts,
                       route=(self.top_w[i], self.top_i[i]) if moe else None, ws=self.ffn_ws)
            if moe:
                ops.moe_gateup(self.xe.view(1, H), lp["experts.gate_up_proj"], self.top_w[i:i + 1],
                               self.top_i[i:i + 1], act=self.act_moe.view(1, cfg.top_k_experts, -1))
            ops.ffn_out(self.act_mlp, lp["mlp.down_proj"], self.mlp_out, self.act_moe if moe else None,
                        lp.get("experts.down_proj"), self.top_i[i] if moe else None, cfg.top_k_experts, combine,
                        self.moe_out if moe else None, H)
        if feed is not None:
            ops.advance_feed(feed, self.tok, self.pos, self.hist)
            return
        # the last layer's tail and the final norm run in the lm_head prologue
        pl = self.layers[-1]
        ops.lm_head(self.x1, self.mlp_out, self.moe_out if moe else None, pl.get("post_feedforward_layernorm_1"),
                    pl.get("post_feedforward_layernorm_2"), pl["post_feedforward_layernorm"], pl["layer_scalar"],
                    p["norm"], p["embed"], cfg.final_logit_softcapping, eps, self.logits, self.blk_val, self.blk_idx)
        if sampler is not None:
            params, top_k, counter_mode = sampler
            ops.sample(self.logits, top_k, params, self.tok, counter_mode, self.pos if advance else None,
                       self.hist if advance else None, ws=self.sample_ws)
        else:
            ops.argmax_finalize(self.blk_val, self.blk_idx, self.tok, self.pos if advance else None,
                                self.hist if advance else None)

    def head(self, x1, mlp_out, moe_out, sampler=None) -> None:
        """lm_head with the last layer's tail on (x1, mlp_out, moe_out) [H]
        (model.py:317-322, 373-385), then the argmax or the sampler: the
        token after position `pos` goes to tok and hist[pos + 1], pos += 1."""
        ops, cfg, p = self.ops, self.cfg, self.params
        pl = self.layers[-1]
        ops.lm_head(x1, mlp_out, moe_out, pl.get("post_feedforward_layernorm_1"),
                    pl.get("post_feedforward_layernorm_2"), pl["post_feedforward_layernorm"], pl["layer_scalar"],
                    p["norm"], p["embed"], cfg.final_logit_softcapping, cfg.rms_norm_eps, self.logits, self.blk_val,
                    self.blk_idx)
        if sampler is not None:
            params, top_k, counter_mode = sampler
            ops.sample(self.logits, top_k, params, self.tok, counter_mode, self.pos, self.hist, ws=self.sample_ws)
        else:
            ops.argmax_finalize(self.blk_val, self.blk_idx, self.tok, self.pos, self.hist)

    def set_state(self, token: int, pos: int) -> None:
        self.tok.fill_(int(token))
        self.pos.fill_(int(pos))

    def set_sequence(self, b: int) -> None:
        """Steps launched from now on use page-table row b of the cache (the
        runner's own buffers are shared).  Not for a runner whose steps are
        captured in graphs: a graph keeps the row it was captured with."""
        if not 0 <= b < self.cache["page_table"].shape[0]:
            raise ValueError(f"sequence {b} outside the cache's {self.cache['page_table'].shape[0]} rows")
        self.page_table = self.cache["page_table"][b:b + 1]
        self._bind_pages(b)

    def _bind_pages(self, b: int) -> None:
        """The K/V pools the attention kernels see.  When page-table row b is
        the identity on pages [b * max_pages, (b + 1) * max_pages) (the
        default cache: every sequence owns its pages in order), the kernels
        get that slice of each pool and no table, and compute page indices
        instead of loading them (one dependent memory round trip less per
        attention kernel).  The row is taken to stay so while bound."""
        pt = self.cache["page_table"]
        mp = pt.shape[1]
        ident = torch.arange(b * mp, (b + 1) * mp, dtype=pt.dtype, device=pt.device)
        self.dense_pages = bool(torch.equal(pt[b], ident)) and all(
            k.shape[0] >= (b + 1) * mp for k in self.cache["k"])
        if self.dense_pages:
            self.kv_pools = [(k[b * mp:(b + 1) * mp], v[b * mp:(b + 1) * mp])
                             for k, v in zip(self.cache["k"], self.cache["v"])]
        else:
            self.kv_pools = list(zip(self.cache["k"], self.cache["v"]))


class PrefillRunner:
    """Batched prefill of n prompt tokens at positions 0..n-1 (model.py:333-386
    over T = n rows, dense-MoE path), leaving the last row's layer-tail inputs
    for the head.  Per layer:

      q/k/v = xn . W^T                  MFMA GEMMs (model.py:197-201)
      kv_append                         k = rope(rms(k_raw)), v = rms(v_raw)
                                        written at positions 0..n-1 (model.py:202-206)
      q_norm_rope + prefill_attention   MFMA flash attention, query row t attends
                                        [max(0, t+1-W), t]: the causal / sliding
                                        prefill mask of model.py:392-399 on the
                                        real rows
      o = ctx . o_proj^T                MFMA GEMM (model.py:214)
      rows_post_attn                    x1, xm, xe (model.py:301-315)
      act = gelu(xm.g) * (xm.u)         MFMA GEMM, gated epilogue (model.py:218-220)
      mlp = act . down^T                MFMA GEMM (model.py:221)
      router top-k + moe_prefill        model.py:224-250 (selected experts only)
      rows_tail                         tail + next input norm (model.py:312-322)

    The first layer starts from rows_embed.  Rows beyond the prompt (the
    reference's bucket padding) are not computed: the reference never attends
    them and reads back only the last prompt row."""

    def __init__(self, cfg: TextConfig, params: dict, cache: dict, capacity: int, device="cuda", rope=None):
        from . import ops

        self.ops, self.cfg, self.params, self.cache = ops, cfg, params, cache
        self.device = dev = torch.device(device)
        self.capacity = cap = int(capacity)
        self.max_len = cache["max_len"]
        if not 1 <= cap <= self.max_len:
            raise ValueError(f"prefill capacity {cap} outside [1, {self.max_len}]")
        self.layers = [{k[len(f"layers.{i}."):]: v for k, v in params.items() if k.startswith(f"layers.{i}.")}
                       for i in range(cfg.num_hidden_layers)]
        H, bf = cfg.hidden_size, torch.bfloat16
        z = lambda *shape, dt=bf: torch.zeros(shape, dtype=dt, device=dev)  # noqa: E731
        self.x, self.x1, self.xn, self.xm, self.o = z(cap, H), z(cap, H), z(cap, H), z(cap, H), z(cap, H)
        self.mlp_out = z(cap, H)
        moe = cfg.enable_moe_block
        self.xe = z(cap, H) if moe else None
        self.moe_out = z(cap, H) if moe else None
        q_max = max(cfg.num_attention_heads * cfg.head_dim_for(lt) for lt in cfg.layer_types)
        kv_max = max(cfg.kv_heads_for(lt) * cfg.head_dim_for(lt) for lt in cfg.layer_types)
        self.q, self.ctx = z(cap * q_max), z(cap * q_max)
        self.k, self.v = z(cap * kv_max), z(cap * kv_max)
        self.act = z(cap, cfg.intermediate_size)
        if moe:
            self.top_w = z(cap, cfg.top_k_experts, dt=torch.float32)
            self.top_i = z(cap, cfg.top_k_experts, dt=torch.int32)
        self.pos = torch.arange(cap, dtype=torch.int32, device=dev)
        # a second stream (default priority) for the dense MLP beside the MoE
        # block (see run); G4MI_PREFILL_STREAMS=0 keeps one stream
        use_side = moe and os.environ.get("G4MI_PREFILL_STREAMS", "1") != "0"
        # the MoE combine inside the layer-tail kernel (G4MI_PREFILL_FUSED_TAIL=0:
        # the combine kernel, then the tail)
        self.fused_tail = os.environ.get("G4MI_PREFILL_FUSED_TAIL", "1") != "0"
        self.side = torch.cuda.Stream(device=dev) if use_side else None
        self.ev_fork = torch.cuda.Event() if use_side else None
        self.ev_join = torch.cuda.Event() if use_side else None
        self.rope = rope if rope is not None else {
            SLIDING: rope_table(cfg.head_dim, cfg.rope_theta_sliding, 1.0, self.max_len, dev),
            FULL: rope_table(cfg.global_head_dim, cfg.rope_theta_full, cfg.rope_partial_rotary_factor_full,
                             self.max_len, dev),
        }

    def run(self, tokens: torch.Tensor, n: int, seq: int = 0, p0: int = 0) -> None:
        """Runs the layers for tokens[:n] (device int32) of sequence `seq`
        (its page-table row) at positions p0 .. p0 + n - 1 on the current
        stream.  With p0 > 0 (a continued prefill) the rows also attend the
        positions < p0 already in the cache."""
        ops, cfg, p = self.ops, self.cfg, self.params
        if not 1 <= n <= self.capacity:
            raise ValueError(f"{n} prompt tokens outside [1, {self.capacity}]")
        if not 0 <= p0 <= self.max_len - n:
            raise ValueError(f"positions {p0}..{p0 + n - 1} outside the cache (max_len {self.max_len})")
        H, eps, NH = cfg.hidden_size, cfg.rms_norm_eps, cfg.num_attention_heads
        moe = cfg.enable_moe_block
        L = cfg.num_hidden_layers
        x, x1, xn, xm, o = self.x[:n], self.x1[:n], self.xn[:n], self.xm[:n], self.o[:n]
        mlp_out = self.mlp_out[:n]
        xe = self.xe[:n] if moe else None
        moe_out = self.moe_out[:n] if moe else None
        pos = self.pos[:n] if p0 == 0 else self.pos[:n] + p0
        page_row = self.cache["page_table"][seq]
        ops.rows_embed(tokens[:n], p["embed"], self.layers[0]["input_layernorm"], eps, x, xn)
        for i, lt in enumerate(cfg.layer_types):
            lp = self.layers[i]
            d, kv = cfg.head_dim_for(lt), cfg.kv_heads_for(lt)
            q = self.q[: n * NH * d].view(n, NH * d)
            k = self.k[: n * kv * d].view(n, kv * d)
            v = None if cfg.k_eq_v_for(lt) else self.v[: n * kv * d].view(n, kv * d)
            ops.prefill_gemm(xn, lp["q_proj"].reshape(NH * d, H), q)
            ops.prefill_gemm(xn, lp["k_proj"].reshape(kv * d, H), k)
            if v is not None:
                ops.prefill_gemm(xn, lp["v_proj"].reshape(kv * d, H), v)
            cos, sin = self.rope[lt]
            ops.kv_append(k.view(n, kv, d), None if v is None else v.view(n, kv, d), lp["k_norm"], cos, sin,
                          self.cache["k"][i], self.cache["v"][i], page_row, pos, self.max_len, eps)
            ctx = self.ctx[: n * NH * d].view(n, NH, d)
            window = cfg.sliding_window if lt == SLIDING else 0
            qh = ops.q_norm_rope(q.view(n, NH, d), lp["q_norm"], cos, sin, p0, eps)
            ops.prefill_attention(qh, self.cache["k"][i], self.cache["v"][i], page_row, p0, window,
                                  cfg.attn_logit_softcapping, ctx=ctx)
            ops.prefill_gemm(ctx.view(n, NH * d), lp["o_proj"].reshape(H, NH * d), o)
            ops.rows_post_attn(x, o, lp["post_attention_layernorm"], lp["pre_feedforward_layernorm"],
                               lp.get("pre_feedforward_layernorm_2"), eps, x1, xm, xe)
            gate, up = lp["mlp.gate_proj"], lp["mlp.up_proj"]
            act = self.act[:n]

            def dense_mlp(ws_key="gemm"):
                ops.prefill_gemm(xm, gate, act, epilogue=ops.EP_GATED,
                                 pair_offset=(up.data_ptr() - gate.data_ptr()) // 2, n=gate.shape[0], ws_key=ws_key)
                ops.prefill_gemm(act, lp["mlp.down_proj"], mlp_out, ws_key=ws_key)

            if moe and self.side is not None:
                # the dense MLP and the MoE block read the same normed rows and
                # meet only in the layer tail: the dense MLP (MFMA-bound) runs
                # on a second stream beside the router and the expert products
                # (bound by their weight stream)
                main = torch.cuda.current_stream()
                self.ev_fork.record(main)
                self.side.wait_event(self.ev_fork)
                with torch.cuda.stream(self.side):
                    dense_mlp("gemm_side")
                    self.ev_join.record(self.side)
            else:
                dense_mlp()
            fused_tail = moe and i + 1 < L and self.fused_tail
            if moe:
                tw, ti = self.top_w[:n], self.top_i[:n]
                ops.moe_router_topk(xe, lp["router.scale"], lp["router.proj"], lp["router.per_expert_scale"],
                                    cfg.top_k_experts, eps, out=(tw, ti))
                # with a tail to follow, the combine of the experts' outputs
                # runs inside the tail kernel
                moe_ws = ops.moe_prefill(xe, tw, ti, lp["experts.gate_up_proj"], lp["experts.down_proj"],
                                         out=moe_out, combine=not fused_tail)
                if self.side is not None:
                    torch.cuda.current_stream().wait_event(self.ev_join)
            if fused_tail:
                E, F = cfg.num_experts, cfg.moe_intermediate_size
                ops.rows_tail_experts(x1, mlp_out, moe_ws, cfg.top_k_experts, E, F,
                                      lp["post_feedforward_layernorm_1"], lp["post_feedforward_layernorm_2"],
                                      lp["post_feedforward_layernorm"], lp["layer_scalar"],
                                      self.layers[i + 1]["input_layernorm"], eps, x, xn)
            elif i + 1 < L:
                ops.rows_tail(x1, mlp_out, moe_out, lp.get("post_feedforward_layernorm_1"),
                              lp.get("post_feedforward_layernorm_2"), lp["post_feedforward_layernorm"],
                              lp["layer_scalar"], self.layers[i + 1]["input_layernorm"], eps, x, xn)

    def last_row(self, n: int) -> tuple:
        """(x1, mlp_out, moe_out) of prompt row n-1: the last layer's tail inputs."""
        return (self.x1[n - 1], self.mlp_out[n - 1], None if self.moe_out is None else self.moe_out[n - 1])


class HeadRunner:
    """The head of one row on its own: the last layer's tail and the final
    norm (model.py:317-322, 373), lm_head and the final softcap
    (model.py:381-385), then the greedy argmax or the sampler
    (model.py:414-424).  For callers that need the head of a prefill row
    without a decode step's buffers; tok/pos/hist are its own unless given."""

    def __init__(self, cfg: TextConfig, params: dict, device="cuda", tok=None, pos=None, hist=None,
                 hist_len: int = 8):
        from . import ops

        self.ops, self.cfg, self.params = ops, cfg, params
        dev = torch.device(device)
        z = lambda n, dt: torch.zeros(n, dtype=dt, device=dev)  # noqa: E731
        self.logits = z(cfg.vocab_size, torch.float32)
        nb = ops.lm_head_blocks(cfg.vocab_size)
        self.blk_val, self.blk_idx = z(nb, torch.float32), z(nb, torch.int32)
        self.tok = tok if tok is not None else z(1, torch.int32)
        self.pos = pos if pos is not None else z(1, torch.int32)
        self.hist = hist if hist is not None else z(hist_len, torch.int32)
        self.sample_ws = None
        self.last = {k[len(f"layers.{cfg.num_hidden_layers - 1}."):]: v for k, v in params.items()
                     if k.startswith(f"layers.{cfg.num_hidden_layers - 1}.")}

    def logits_of(self, x1, mlp_out, moe_out, out: torch.Tensor | None = None) -> torch.Tensor:
        """Softcapped f32 logits [V] of one row's tail inputs, into `out`."""
        cfg, pl = self.cfg, self.last
        out = self.logits if out is None else out
        self.ops.lm_head(x1, mlp_out, moe_out, pl.get("post_feedforward_layernorm_1"),
                         pl.get("post_feedforward_layernorm_2"), pl["post_feedforward_layernorm"],
                         pl["layer_scalar"], self.params["norm"], self.params["embed"], cfg.final_logit_softcapping,
                         cfg.rms_norm_eps, out, self.blk_val, self.blk_idx)
        return out

    def head(self, x1, mlp_out, moe_out, sampler=None) -> None:
        """logits_of, then the next token: the token after position `pos`
        goes to tok and hist[pos + 1], pos += 1."""
        self.logits_of(x1, mlp_out, moe_out)
        if sampler is not None:
            params, top_k, counter_mode = sampler
            if self.sample_ws is None:
                self.sample_ws = torch.zeros(self.ops.sample_workspace_bytes(self.cfg.vocab_size), dtype=torch.uint8,
                                             device=self.logits.device)
            self.ops.sample(self.logits, top_k, params, self.tok, counter_mode, self.pos, self.hist,
                            ws=self.sample_ws)
        else:
            self.ops.argmax_finalize(self.blk_val, self.blk_idx, self.tok, self.pos, self.hist)


def _runners_for(cfg: TextConfig, params: dict, cache: dict) -> dict:
    """The runners one forward() call uses for this (params, cache) pair: the
    decode runner and the head (the batched prefill is added when needed).
    They are built per call and dropped when it returns, so no module state
    keeps the caller's weights or cache alive after the caller lets go of
    them (the buffers come back from torch's caching allocator)."""
    dev = cache["k"][0].device
    return {"decode": DecodeRunner(cfg, params, cache, device=dev), "head": HeadRunner(cfg, params, dev),
            "prefill": None}


def runner_for(cfg: TextConfig, params: dict, cache: dict) -> DecodeRunner:
    """A DecodeRunner bound to this (params, cache) pair (a new one per call;
    it references both for as long as the caller keeps it)."""
    return DecodeRunner(cfg, params, cache, device=cache["k"][0].device)


def forward(cfg: TextConfig, mesh, params: dict, tokens, positions, cache: dict, write_at, masks: dict, kv_len: int,
            dense_moe: bool, last_index=None):
    """Logits for `tokens` [B, T] at `positions` [T] (model.py:333-386): every
    row b uses row b of the cache at the same positions, as the reference's
    batched forward does.  Returns (logits f32 [B, T or 1, V], cache); the
    cache is updated in place (the reference donates it) and returned.

    A multi-token call with the dense-MoE combine over consecutive positions
    (the engine's prefill, model.py:241-250 and 392-399) runs the batched
    prefill: MFMA GEMMs, the selected-expert grouped GEMMs and MFMA prefill
    attention, then the head of each requested row.  Single-token calls (the
    decode step, model.py:262-294) and any other call run the decode kernels
    one position at a time; row t of the reference's causal prefill attends
    exactly the cached positions <= t, so both equal the T x T masked form.
    dense_moe selects the dense-MoE f32 combine instead of the decode path's
    bf16 running sum.  Rows at or past the masks' prompt_len (the
    reference's bucket padding) are neither computed nor written to the
    cache: the reference never attends them and reads back only last_index
    (< prompt_len); their logits are returned as zeros.  kv_len is not
    needed: the kernels read only each row's attended positions."""
    tok = torch.as_tensor(tokens)
    if tok.ndim == 1:
        tok = tok[None]
    if tok.ndim != 2:
        raise ValueError(f"tokens must be [B, T], got {tuple(tok.shape)}")
    B, T = tok.shape
    pos = [int(v) for v in torch.as_tensor(positions).reshape(-1).tolist()]
    if len(pos) != T:
        raise ValueError(f"{len(pos)} positions for {T} tokens")
    if B > cache["page_table"].shape[0]:
        raise ValueError(f"{B} token rows for a cache of {cache['page_table'].shape[0]} sequences")
    if T and int(torch.as_tensor(write_at).item() if isinstance(write_at, torch.Tensor) else write_at) != pos[0]:
        raise ValueError("write_at must equal positions[0] (the cache rows are written at the token positions)")
    n = T
    if isinstance(masks, dict) and "prompt_len" in masks:
        n = min(n, int(masks["prompt_len"]))
    rs = _runners_for(cfg, params, cache)
    r, hr = rs["decode"], rs["head"]
    for t in range(n):
        if not 0 <= pos[t] < r.max_len:
            raise ValueError(f"position {pos[t]} outside the cache (max_len {r.max_len})")
    if last_index is not None and not 0 <= int(last_index) < max(n, 1):
        raise ValueError(f"last_index {int(last_index)} outside the {n} computed rows")
    keep = list(range(n)) if last_index is None else [int(last_index)]
    out = torch.zeros((B, T if last_index is None else 1, cfg.vocab_size), dtype=torch.float32, device=r.device)
    consecutive = all(pos[t] == pos[0] + t for t in range(n))
    if n > 1 and dense_moe and consecutive:
        pr = rs["prefill"]
        if pr is None or pr.capacity < n:
            rs["prefill"] = None
            pr = rs["prefill"] = PrefillRunner(cfg, params, cache, min(r.max_len, max(n, 256)), device=r.device,
                                               rope=r.rope)
        tok_dev = tok.to(device=r.device, dtype=torch.int32)
        for b in range(B):
            pr.run(tok_dev[b].contiguous(), n, seq=b, p0=pos[0])
            for j, t in enumerate(keep):
                hr.logits_of(pr.x1[t], pr.mlp_out[t], None if pr.moe_out is None else pr.moe_out[t], out=out[b, j])
        return out, cache
    combine = "f32" if dense_moe else "bf16_running"
    tok_host = tok.tolist()
    try:
        for b in range(B):
            r.set_sequence(b)
            j = 0
            for t in range(n):
                r.set_state(tok_host[b][t], pos[t])
                r.launch(combine, advance=False)
                if last_index is None or t == int(last_index):
                    out[b, j].copy_(r.logits)
                    j += 1
    finally:
        r.set_sequence(0)
    return out, cache
