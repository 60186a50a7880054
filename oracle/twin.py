"""torch-CPU restatement of gemma4_tpu/model.py — TEST INFRASTRUCTURE ONLY.

Each function cites the reference lines it restates.  Tensors are torch CPU
tensors; bf16 tensors hold values that the reference holds as bf16.  The
rounding recipe is described in oracle/__init__.py.

`precise=True` (default) accumulates every einsum in f64; `precise=False`
uses torch's native bf16 CPU GEMMs (f32 accumulation), which is how the
timed CPU baseline runs.  Both are restatements of the same program; they
differ only in accumulation order and precision, which the reference leaves
to XLA.

Parity pins (see tests/): rms_norm, gelu, rope, attention, MLP, softcap
against HF transformers Gemma-4 sub-modules and closed forms; router top-k
against a brute-force sort; MoE decode against the dense path (the
reference's own invariant, tests/test_parity.py:127-151) and brute force;
whole forward against committed HF fixtures (tests/golden/).
"""

from __future__ import annotations

import math

import numpy as np
import torch

FULL = "full_attention"
SLIDING = "sliding_attention"
NEG_INF = -1e30  # model.py:32
BF16 = torch.bfloat16


# ----------------------------------------------------------------- rounding
def rb(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (nearest even); f64 input is rounded through f32 first."""
    if x.dtype == torch.float64:
        x = x.float()
    return x.to(BF16)


def f32(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float32)


def ein(eq: str, a: torch.Tensor, b: torch.Tensor, precise: bool = True) -> torch.Tensor:
    """A bf16 x bf16 einsum with a bf16 result (XLA dot semantics)."""
    if precise:
        return rb(torch.einsum(eq, a.double(), b.double()))
    return torch.einsum(eq, a.to(BF16), b.to(BF16)).to(BF16)


# ----------------------------------------------------------------- primitives
def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """model.py:42-47: f32 normalisation, optional f32 weight, cast back."""
    x32 = f32(x)
    sumsq = (x32.double() * x32.double()).sum(-1, keepdim=True)
    mean = sumsq.float() / float(x.shape[-1])
    scale = (1.0 / torch.sqrt((mean + np.float32(eps)).double())).float()
    out = x32 * scale
    if weight is not None:
        out = out * f32(weight)
    return out.to(x.dtype)


def gelu(x: torch.Tensor) -> torch.Tensor:
    """model.py:50-51 (tanh approximation), computed in f32, one rounding."""
    x32 = f32(x)
    k0 = np.float32(math.sqrt(2.0 / math.pi))
    cdf = 0.5 * (1.0 + torch.tanh(k0 * (x32 + np.float32(0.044715) * (x32 * x32 * x32))))
    return (x32 * cdf).to(x.dtype)


def rope_inv_freq(head_dim: int, theta: float, partial_rotary_factor: float = 1.0) -> np.ndarray:
    """model.py:54-61: f64 inverse frequencies of the rotated pairs, zero for the
    NoPE tail, cast to f32."""
    n_rot = int(partial_rotary_factor * head_dim // 2)
    half = head_dim // 2
    inv = np.zeros(half, np.float64)
    exps = np.arange(0, 2 * n_rot, 2, dtype=np.float64) / head_dim
    inv[:n_rot] = 1.0 / (theta**exps)
    return inv.astype(np.float32)


def rope_tables(positions, inv_freq: np.ndarray) -> tuple[torch.Tensor, torch.Tensor]:
    """model.py:64-67: angles pos*inv_freq in f32, halves duplicated; cos/sin f32."""
    pos = torch.as_tensor(np.asarray(positions), dtype=torch.float32).reshape(-1)
    freqs = pos[:, None] * torch.as_tensor(inv_freq, dtype=torch.float32)[None, :]
    emb = torch.cat([freqs, freqs], dim=-1).double()
    return torch.cos(emb).float(), torch.sin(emb).float()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """model.py:70-78: x [B,T,...,D] bf16; cos/sin [T,D] cast to bf16;
    x*c + rotate_half(x)*s with each bf16 op rounded."""
    d = x.shape[-1]
    rot = torch.cat([-x[..., d // 2 :], x[..., : d // 2]], dim=-1)
    shape = (1, cos.shape[0]) + (1,) * (x.ndim - 3) + (d,)
    c = f32(rb(cos).reshape(shape))
    s = f32(rb(sin).reshape(shape))
    return rb(f32(rb(f32(x) * c)) + f32(rb(f32(rot) * s)))


# ----------------------------------------------------------------- layout
def param_shapes(cfg) -> dict[str, tuple[int, ...]]:
    """model.py:84-117: canonical shapes, keyed by flat name, in this order."""
    h = cfg.hidden_size
    out: dict[str, tuple[int, ...]] = {"embed": (cfg.vocab_size, h), "norm": (h,)}
    for i, lt in enumerate(cfg.layer_types):
        d, kv = cfg.head_dim_for(lt), cfg.kv_heads_for(lt)
        g = cfg.num_attention_heads // kv
        p = f"layers.{i}."
        for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                  "post_feedforward_layernorm"):
            out[p + n] = (h,)
        out[p + "layer_scalar"] = (1,)
        out[p + "q_proj"] = (kv, g, d, h)
        out[p + "k_proj"] = (kv, d, h)
        if not cfg.k_eq_v_for(lt):
            out[p + "v_proj"] = (kv, d, h)
        out[p + "o_proj"] = (h, kv, g, d)
        out[p + "q_norm"] = (d,)
        out[p + "k_norm"] = (d,)
        out[p + "mlp.gate_proj"] = (cfg.intermediate_size, h)
        out[p + "mlp.up_proj"] = (cfg.intermediate_size, h)
        out[p + "mlp.down_proj"] = (h, cfg.intermediate_size)
        if cfg.enable_moe_block:
            for n in ("pre_feedforward_layernorm_2", "post_feedforward_layernorm_1",
                      "post_feedforward_layernorm_2"):
                out[p + n] = (h,)
            out[p + "router.proj"] = (cfg.num_experts, h)
            out[p + "router.scale"] = (h,)
            out[p + "router.per_expert_scale"] = (cfg.num_experts,)
            out[p + "experts.gate_up_proj"] = (cfg.num_experts, 2, cfg.moe_intermediate_size, h)
            out[p + "experts.down_proj"] = (cfg.num_experts, h, cfg.moe_intermediate_size)
    return out


def random_params(cfg, seed: int, std: float = 0.02, ones: tuple[str, ...] = ("layer_scalar",)) -> dict:
    """bf16 CPU tensors from the numpy restatement of the weight generator.
    Names ending in any of `ones` are filled with 1.0."""
    from .philox import normal_bf16_bits, tensor_key

    out = {}
    for name, shape in param_shapes(cfg).items():
        n = int(np.prod(shape))
        if any(name.endswith(s) for s in ones):
            out[name] = torch.ones(shape, dtype=BF16)
            continue
        bits = normal_bf16_bits(n, tensor_key(seed, name), std)
        out[name] = torch.from_numpy(bits.view(np.int16).copy()).view(BF16).reshape(shape)
    return out


def layer_params(params: dict, i: int) -> dict:
    p = f"layers.{i}."
    return {k[len(p):]: v for k, v in params.items() if k.startswith(p)}


# ----------------------------------------------------------------- cache
def cache_shapes(cfg, batch: int, max_len: int) -> list[tuple[int, ...]]:
    """model.py:174-175."""
    return [(batch, max_len, cfg.kv_heads_for(lt), cfg.head_dim_for(lt)) for lt in cfg.layer_types]


def init_cache(cfg, batch: int, max_len: int) -> dict:
    """model.py:178-185: zero K and V per layer."""
    shapes = cache_shapes(cfg, batch, max_len)
    return {"k": [torch.zeros(s, dtype=BF16) for s in shapes], "v": [torch.zeros(s, dtype=BF16) for s in shapes]}


# ----------------------------------------------------------------- blocks
def attention_core(q, k_raw, v_raw, q_norm, k_norm, cos, sin, cache_k, cache_v, write_at, mask, kv_len, eps,
                   softcap=None, precise=True, inplace=False):
    """model.py:198-213 from the raw projections on: q [B,T,KV,G,D], k_raw/v_raw
    [B,T,KV,D] bf16 (v_raw is k_raw on k==v layers).  Returns (ctx
    [B,T,KV,G,D] bf16, cache_k, cache_v).  With `inplace` the caches are
    updated in place (the reference donates them), else copied first."""
    q = apply_rope(rms_norm(q, q_norm, eps), cos, sin)
    k = apply_rope(rms_norm(k_raw, k_norm, eps), cos, sin)
    v = rms_norm(v_raw, None, eps)
    t = q.shape[1]
    if not inplace:
        cache_k = cache_k.clone()
        cache_v = cache_v.clone()
    cache_k[:, write_at : write_at + t] = k
    cache_v[:, write_at : write_at + t] = v
    kk, vv = cache_k[:, :kv_len], cache_v[:, :kv_len]
    scores = f32(ein("btkgd,bskd->bkgts", q, kk, precise))
    if softcap:
        scores = torch.tanh(scores / np.float32(softcap)) * np.float32(softcap)
    scores = torch.where(torch.as_tensor(mask), scores, torch.tensor(NEG_INF, dtype=torch.float32))
    probs = rb(torch.softmax(scores, dim=-1))
    ctx = ein("bkgts,bskd->btkgd", probs, vv, precise)
    return ctx, cache_k, cache_v


def attention(cfg, lp, x, layer_type, cos, sin, cache_k, cache_v, write_at, mask, kv_len, precise=True,
              inplace=False):
    """model.py:195-215.  x [B,T,H] bf16 (input_layernorm output); mask bool
    broadcastable to [B,KV,G,T,kv_len].  Returns (out [B,T,H], cache_k, cache_v)."""
    q = ein("bth,kgdh->btkgd", x, lp["q_proj"], precise)
    k_raw = ein("bth,kdh->btkd", x, lp["k_proj"], precise)
    v_raw = k_raw if cfg.k_eq_v_for(layer_type) else ein("bth,kdh->btkd", x, lp["v_proj"], precise)
    ctx, cache_k, cache_v = attention_core(q, k_raw, v_raw, lp["q_norm"], lp["k_norm"], cos, sin, cache_k, cache_v,
                                           write_at, mask, kv_len, cfg.rms_norm_eps,
                                           getattr(cfg, "attn_logit_softcapping", None), precise, inplace)
    out = ein("btkgd,hkgd->bth", ctx, lp["o_proj"], precise)
    return out, cache_k, cache_v


def dense_mlp(lp, x, precise=True):
    """model.py:218-221."""
    g = ein("bth,ih->bti", x, lp["mlp.gate_proj"], precise)
    u = ein("bth,ih->bti", x, lp["mlp.up_proj"], precise)
    a = rb(f32(gelu(g)) * f32(u))
    return ein("bti,hi->bth", a, lp["mlp.down_proj"], precise)


def router(cfg, lp, flat, precise=True):
    """model.py:224-232.  flat [N,H] bf16 -> (top_w [N,k] f32, top_i [N,k] int64).

    The router's dot is always exact (f64) and its softmax exponent is taken in
    f64 and rounded to f32; top-k is a stable descending sort on the
    probabilities (ties to the lower index, as jax.lax.top_k)."""
    h = cfg.hidden_size
    x = rms_norm(flat, None, cfg.rms_norm_eps)
    c = float(rb(torch.tensor(h**-0.5, dtype=torch.float32)))
    x = rb(f32(rb(f32(x) * f32(lp["router.scale"]))) * np.float32(c))
    scores = f32(rb(torch.einsum("nh,eh->ne", x.double(), lp["router.proj"].double())))
    m = scores.max(dim=-1, keepdim=True).values
    ex = torch.exp((scores - m).double()).float()
    total = ex.double().sum(-1, keepdim=True).float()
    probs = ex / total
    order = torch.sort(probs, dim=-1, descending=True, stable=True).indices
    top_i = order[:, : cfg.top_k_experts]
    top_w = torch.gather(probs, 1, top_i)
    top_w = top_w / top_w.double().sum(-1, keepdim=True).float()
    top_w = top_w * f32(lp["router.per_expert_scale"])[top_i]
    return top_w, top_i


def moe_dense_selected(cfg, flat, top_w, top_i, gate_up, down, precise=True):
    """model.py:241-250 (the dense-MoE contraction) evaluated on the selected
    (token, expert) pairs only.  An unselected expert's routing weight is 0,
    so its activation is bf16(x * 0) = 0 exactly and it adds exact zeros to
    the contraction over experts: the result is the dense path's (up to the
    order of the f64 sum before its rounding), at k/E of the products.
    flat [N,H] bf16, top_w [N,k] f32, top_i [N,k] int -> [N,H] bf16."""
    n_tok, k = top_i.shape
    f = gate_up.shape[2]
    acts = torch.zeros((n_tok, k, f), dtype=BF16)
    ti = top_i.long()
    experts = torch.unique(ti).tolist()
    for e in experts:
        rows, slots = (ti == e).nonzero(as_tuple=True)
        gu = ein("nh,cfh->ncf", flat[rows], gate_up[e], precise)
        act = rb(f32(gelu(gu[:, 0])) * f32(gu[:, 1]))
        acts[rows, slots] = rb(f32(act) * f32(rb(top_w[rows, slots]))[:, None])
    acc = torch.zeros((n_tok, down.shape[1]), dtype=torch.float64 if precise else torch.float32)
    for e in experts:
        rows, slots = (ti == e).nonzero(as_tuple=True)
        a = acts[rows, slots]
        if precise:
            acc.index_add_(0, rows, a.double() @ down[e].double().T)
        else:
            acc.index_add_(0, rows, (a @ down[e].to(BF16).T).float())
    return rb(acc)


def moe(cfg, lp, flat, dense, precise=True, return_route=False):
    """model.py:235-294.  flat [N,H] bf16 (pre_feedforward_layernorm_2 output).

    dense=True: all experts for every token as one contraction masked by the
    routing weight (model.py:241-250).  dense="selected": the same
    contraction restricted to the selected experts (moe_dense_selected).
    dense=False: the default "slice" decode path, a bf16 running sum over the
    selected experts in top-k order (model.py:262-294)."""
    top_w, top_i = router(cfg, lp, flat, precise)
    gate_up, down = lp["experts.gate_up_proj"], lp["experts.down_proj"]
    n_tok = flat.shape[0]
    if isinstance(dense, str):
        if dense != "selected":
            raise ValueError(f"dense={dense!r}")
        out = moe_dense_selected(cfg, flat, top_w, top_i, gate_up, down, precise)
    elif dense:
        w_full = torch.zeros((n_tok, cfg.num_experts), dtype=torch.float32)
        w_full.scatter_(1, top_i, top_w)
        gu = ein("nh,ecfh->necf", flat, gate_up, precise)
        act = rb(f32(gelu(gu[:, :, 0])) * f32(gu[:, :, 1]))
        act = rb(f32(act) * f32(rb(w_full))[:, :, None])
        out = ein("nef,ehf->nh", act, down, precise)
    else:
        rows = []
        for n in range(n_tok):
            acc = None
            for kk in range(cfg.top_k_experts):
                e = int(top_i[n, kk])
                gu = ein("h,cfh->cf", flat[n], gate_up[e], precise)
                a = rb(f32(rb(f32(gelu(gu[0])) * f32(gu[1]))) * f32(rb(top_w[n, kk])))
                part = ein("f,hf->h", a, down[e], precise)
                acc = part if acc is None else rb(f32(acc) + f32(part))
            rows.append(acc)
        out = torch.stack(rows, 0)
    return (out, top_w, top_i) if return_route else out


def layer(cfg, lp, x, layer_type, cos, sin, ck, cv, write_at, mask, kv_len, dense_moe, precise=True, trace=None,
          inplace=False):
    """model.py:297-322.  `trace`, if a list, receives this layer's (top_w, top_i)."""
    eps = cfg.rms_norm_eps
    residual = x
    h = rms_norm(x, lp["input_layernorm"], eps)
    h, ck, cv = attention(cfg, lp, h, layer_type, cos, sin, ck, cv, write_at, mask, kv_len, precise, inplace)
    h = rms_norm(h, lp["post_attention_layernorm"], eps)
    x = rb(f32(residual) + f32(h))

    residual = x
    h = dense_mlp(lp, rms_norm(x, lp["pre_feedforward_layernorm"], eps), precise)
    if cfg.enable_moe_block:
        h1 = rms_norm(h, lp["post_feedforward_layernorm_1"], eps)
        b, t, hid = residual.shape
        h2 = rms_norm(residual.reshape(-1, hid), lp["pre_feedforward_layernorm_2"], eps)
        h2, top_w, top_i = moe(cfg, lp, h2, dense_moe, precise, return_route=True)
        if trace is not None:
            trace.append((top_w.reshape(b, t, -1), top_i.reshape(b, t, -1)))
        h2 = rms_norm(h2.reshape(b, t, hid), lp["post_feedforward_layernorm_2"], eps)
        h = rb(f32(h1) + f32(h2))
    h = rms_norm(h, lp["post_feedforward_layernorm"], eps)
    x = rb(f32(residual) + f32(h))
    return rb(f32(x) * f32(lp["layer_scalar"])), ck, cv


def forward(cfg, params, tokens, positions, cache, write_at, masks, kv_len, dense_moe, last_index=None,
            precise=True, trace=None, inplace=False):
    """model.py:333-386 without sharding.  tokens [B,T] int; returns
    (logits f32 [B,T or 1,V], cache).  `trace`, if a list, receives per-layer
    routing (top_w, top_i)."""
    embed = params["embed"]
    tok = torch.as_tensor(np.asarray(tokens), dtype=torch.long)
    c = f32(rb(torch.tensor(np.float32(math.sqrt(cfg.hidden_size)))))
    x = rb(f32(embed[tok]) * c)
    inv_sl = rope_inv_freq(cfg.head_dim, cfg.rope_theta_sliding)
    inv_fu = rope_inv_freq(cfg.global_head_dim, cfg.rope_theta_full, cfg.rope_partial_rotary_factor_full)
    rope = {SLIDING: rope_tables(positions, inv_sl), FULL: rope_tables(positions, inv_fu)}
    ks, vs = list(cache["k"]), list(cache["v"])
    for i, lt in enumerate(cfg.layer_types):
        cos, sin = rope[lt]
        x, ks[i], vs[i] = layer(cfg, layer_params(params, i), x, lt, cos, sin, ks[i], vs[i], write_at,
                                masks[lt], kv_len, dense_moe, precise, trace, inplace)
    x = rms_norm(x, params["norm"], cfg.rms_norm_eps)
    if last_index is not None:
        x = x[:, int(last_index) : int(last_index) + 1]
    logits = f32(ein("bth,vh->btv", x, embed, precise))
    if cfg.final_logit_softcapping:
        cap = np.float32(cfg.final_logit_softcapping)
        logits = torch.tanh(logits / cap) * cap
    return logits, {"k": ks, "v": vs}


# ----------------------------------------------------------------- masks
def prefill_masks(cfg, t: int, prompt_len: int) -> dict:
    """model.py:392-399: causal, kv < prompt_len, plus the window on sliding layers."""
    q = torch.arange(t)[:, None]
    kv = torch.arange(t)[None, :]
    valid = (kv <= q) & (kv < prompt_len)
    return {FULL: valid[None, None, None], SLIDING: (valid & (kv > q - cfg.sliding_window))[None, None, None]}


def decode_masks(cfg, max_len: int, pos: int) -> dict:
    """model.py:402-408."""
    kv = torch.arange(max_len)[None, :]
    valid = kv <= pos
    return {FULL: valid[None, None, None], SLIDING: (valid & (kv > pos - cfg.sliding_window))[None, None, None]}


# ----------------------------------------------------------------- sampling
def greedy(logits: torch.Tensor) -> int:
    """model.py:416 with temperature <= 0: first index of the maximum."""
    return int(torch.argmax(logits))


# ----------------------------------------------------------------- drivers
def prefill_then_decode(cfg, params, prompt, n_decode: int, max_len: int, precise=True, trace=None,
                        all_logits: bool = True, prefill_dense=True, forced=None):
    """The engine's call pattern (engine.py:149-221) with greedy sampling and no
    bucket padding (padded positions are never attended): dense-MoE prefill of
    the whole prompt with every position's logits (only the last prompt
    row's with all_logits=False), then n_decode greedy steps.  prefill_dense
    is passed to moe() as `dense` for the prompt rows.  With `forced` (a
    token list of length >= n_decode) decode step s is fed forced[s]
    instead of the previous greedy token (teacher forcing), and the greedy
    tokens are still returned.
    Returns (logits [P or 1, + n_decode, V] f32, tokens generated [n_decode + 1])."""
    p = len(prompt)
    cache = init_cache(cfg, 1, max_len)
    toks = np.asarray(prompt, np.int64)[None]
    logits, cache = forward(cfg, params, toks, np.arange(p), cache, 0, prefill_masks(cfg, p, p), p, prefill_dense,
                            None if all_logits else p - 1, precise, trace)
    out = [logits[0]]
    nxt = greedy(logits[0, -1])
    gen = [nxt]
    for step in range(n_decode):
        pos = p + step
        feed = nxt if forced is None else int(forced[step])
        lg, cache = forward(cfg, params, np.array([[feed]]), np.array([pos]), cache, pos,
                            decode_masks(cfg, max_len, pos), max_len, False, None, precise, trace)
        out.append(lg[0])
        nxt = greedy(lg[0, 0])
        gen.append(nxt)
    return torch.cat(out, 0), gen
