"""torch-facing wrappers over the libg4mi C ABI.

Each wrapper checks dtypes, devices and contiguity on the host, passes raw
device pointers plus the current HIP stream, and raises ``G4miError`` when the
library rejects a call.  Scratch buffers come from :class:`Workspace`, which
allocates once per (device, purpose) and zero-fills on allocation: the kernels
leave their completion counters at zero, so a workspace is reusable (also
across HIP-graph replays) without any further clearing.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

BF16 = torch.bfloat16


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream_handle(device: torch.device | None = None) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need(t: torch.Tensor, dtype: torch.dtype, name: str, shape: tuple | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU (got {t.device}); libg4mi has no CPU path")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


class Workspace:
    """Grow-only per-device scratch buffers, zero-filled when (re)allocated."""

    def __init__(self) -> None:
        self._bufs: dict[tuple[int, str], torch.Tensor] = {}

    def get(self, device: torch.device, purpose: str, nbytes: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        key = (idx, purpose)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


WORKSPACE = Workspace()


# ------------------------------------------------------------------------- init
def fill_normal_(t: torch.Tensor, key: int, std: float) -> torch.Tensor:
    """In-place N(0, std) bf16 fill from the library's Philox generator."""
    _need(t, BF16, "t")
    _lib.call(
        "g4mi_fill_normal_bf16", _ptr(t), t.numel(), ctypes.c_uint64(key & (2**64 - 1)), float(std),
        stream_handle(t.device),
    )
    return t


def philox4x32_10(ctr: torch.Tensor, key: int) -> torch.Tensor:
    """Raw Philox4x32-10 blocks: ctr [n, 4] int32 (uint32 bit patterns) -> [n, 4]."""
    _need(ctr, torch.int32, "ctr")
    out = torch.empty_like(ctr)
    _lib.call(
        "g4mi_philox4x32_10", _ptr(ctr), ctypes.c_uint64(key & (2**64 - 1)), _ptr(out), ctr.numel() // 4,
        stream_handle(ctr.device),
    )
    return out


# -------------------------------------------------------------------------- MoE
def moe_router_topk(
    x: torch.Tensor,
    router_scale: torch.Tensor,
    router_proj: torch.Tensor,
    per_expert_scale: torch.Tensor,
    k: int,
    eps: float,
    pre_norm_w: torch.Tensor | None = None,
    out: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Router + top-k (model.py:224-232).  x [N, H] bf16 -> (top_w [N,k] f32, top_i [N,k] i32).

    With ``pre_norm_w`` the pre_feedforward_layernorm_2 RMSNorm (model.py:315)
    is applied to x first."""
    n, h = x.shape
    e = router_proj.shape[0]
    _need(x, BF16, "x")
    _need(router_scale, BF16, "router_scale", (h,))
    _need(router_proj, BF16, "router_proj", (e, h))
    _need(per_expert_scale, BF16, "per_expert_scale", (e,))
    if pre_norm_w is not None:
        _need(pre_norm_w, BF16, "pre_norm_w", (h,))
    if out is None:
        top_w = torch.empty((n, k), dtype=torch.float32, device=x.device)
        top_i = torch.empty((n, k), dtype=torch.int32, device=x.device)
    else:
        top_w, top_i = out
        _need(top_w, torch.float32, "top_w", (n, k))
        _need(top_i, torch.int32, "top_i", (n, k))
    lib = _lib.lib()
    nbytes = lib.g4mi_moe_router_workspace_bytes(n, e)
    ws = WORKSPACE.get(x.device, "router", nbytes)
    _lib.call(
        "g4mi_moe_router_topk", _ptr(x), _ptr(pre_norm_w), _ptr(router_scale), _ptr(router_proj),
        _ptr(per_expert_scale), n, h, e, k, float(eps), _ptr(top_w), _ptr(top_i), _ptr(ws), ws.numel(),
        stream_handle(x.device),
    )
    return top_w, top_i


def moe_experts(
    xn: torch.Tensor,
    gate_up: torch.Tensor,
    down: torch.Tensor,
    top_w: torch.Tensor,
    top_i: torch.Tensor,
    combine: str = "bf16_running",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Selected-expert gate/up + down GEMVs and the weighted combine.

    combine="bf16_running" is the decode path (model.py:262-294); "f32" is the
    dense-MoE contraction used by prefill (model.py:241-250)."""
    n, h = xn.shape
    e, two, f, h2 = gate_up.shape
    k = top_i.shape[1]
    if two != 2 or h2 != h:
        raise ValueError(f"gate_up shape {tuple(gate_up.shape)} does not match hidden {h}")
    _need(xn, BF16, "xn")
    _need(gate_up, BF16, "gate_up")
    _need(down, BF16, "down", (e, h, f))
    _need(top_w, torch.float32, "top_w", (n, k))
    _need(top_i, torch.int32, "top_i", (n, k))
    mode = {"bf16_running": _lib.COMBINE_BF16_RUNNING, "f32": _lib.COMBINE_F32}[combine]
    if out is None:
        out = torch.empty((n, h), dtype=BF16, device=xn.device)
    else:
        _need(out, BF16, "out", (n, h))
    lib = _lib.lib()
    nbytes = lib.g4mi_moe_experts_workspace_bytes(n, f, k)
    ws = WORKSPACE.get(xn.device, "experts", nbytes)
    _lib.call(
        "g4mi_moe_experts_decode", _ptr(xn), _ptr(gate_up), _ptr(down), _ptr(top_w), _ptr(top_i), n, h, f, e,
        k, mode, _ptr(out), _ptr(ws), ws.numel(), stream_handle(xn.device),
    )
    return out


def moe_gateup(xn, gate_up, top_w, top_i, act=None):
    """Selected-expert gate/up GEMV + activation: act [N, k, F] bf16."""
    n, h = xn.shape
    e, _, f, _ = gate_up.shape
    k = top_i.shape[1]
    _need(xn, BF16, "xn")
    _need(gate_up, BF16, "gate_up", (e, 2, f, h))
    _need(top_w, torch.float32, "top_w", (n, k))
    _need(top_i, torch.int32, "top_i", (n, k))
    if act is None:
        act = torch.empty((n, k, f), dtype=BF16, device=xn.device)
    _need(act, BF16, "act", (n, k, f))
    _lib.call("g4mi_moe_gateup", _ptr(xn), _ptr(gate_up), _ptr(top_w), _ptr(top_i), n, h, f, e, k, _ptr(act),
              stream_handle(xn.device))
    return act


def moe_down(act, down, top_i, combine="bf16_running", out=None):
    """Selected-expert down GEMV + combine: out [N, H] bf16."""
    n, k, f = act.shape
    e, h, _ = down.shape
    _need(act, BF16, "act")
    _need(down, BF16, "down", (e, h, f))
    _need(top_i, torch.int32, "top_i", (n, k))
    mode = {"bf16_running": _lib.COMBINE_BF16_RUNNING, "f32": _lib.COMBINE_F32}[combine]
    if out is None:
        out = torch.empty((n, h), dtype=BF16, device=act.device)
    _need(out, BF16, "out", (n, h))
    _lib.call("g4mi_moe_down", _ptr(act), _ptr(down), _ptr(top_i), n, h, f, e, k, mode, _ptr(out),
              stream_handle(act.device))
    return out


def moe_router_scores(x, router_scale, router_proj, eps, pre_norm_w=None, out=None):
    """Router logits (bf16-rounded, as f32) [N, E] (model.py:225-227)."""
    n, h = x.shape
    e = router_proj.shape[0]
    _need(x, BF16, "x")
    _need(router_scale, BF16, "router_scale", (h,))
    _need(router_proj, BF16, "router_proj", (e, h))
    if pre_norm_w is not None:
        _need(pre_norm_w, BF16, "pre_norm_w", (h,))
    if out is None:
        out = torch.empty((n, e), dtype=torch.float32, device=x.device)
    _need(out, torch.float32, "out", (n, e))
    _lib.call("g4mi_moe_router_scores", _ptr(x), _ptr(pre_norm_w), _ptr(router_scale), _ptr(router_proj), n, h, e,
              float(eps), _ptr(out), stream_handle(x.device))
    return out


def moe_block(xn, router_scale, router_proj, per_expert_scale, gate_up, down, k, eps, combine="bf16_running",
              out=None, route=None):
    """The whole MoE decode block (model.py:235-294) on xn [N, H]; returns
    (out [N, H] bf16, top_w [N, k] f32, top_i [N, k] int32)."""
    n, h = xn.shape
    e, _, f, _ = gate_up.shape
    _need(xn, BF16, "xn")
    _need(router_scale, BF16, "router_scale", (h,))
    _need(router_proj, BF16, "router_proj", (e, h))
    _need(per_expert_scale, BF16, "per_expert_scale", (e,))
    _need(gate_up, BF16, "gate_up", (e, 2, f, h))
    _need(down, BF16, "down", (e, h, f))
    mode = {"bf16_running": _lib.COMBINE_BF16_RUNNING, "f32": _lib.COMBINE_F32}[combine]
    if out is None:
        out = torch.empty((n, h), dtype=BF16, device=xn.device)
    _need(out, BF16, "out", (n, h))
    if route is None:
        route = (torch.empty((n, k), dtype=torch.float32, device=xn.device),
                 torch.empty((n, k), dtype=torch.int32, device=xn.device))
    top_w, top_i = route
    _need(top_w, torch.float32, "top_w", (n, k))
    _need(top_i, torch.int32, "top_i", (n, k))
    nbytes = _lib.lib().g4mi_moe_block_workspace_bytes(n, e, f, k)
    ws = WORKSPACE.get(xn.device, "moe_block", nbytes)
    _lib.call("g4mi_moe_block_decode", _ptr(xn), _ptr(router_scale), _ptr(router_proj), _ptr(per_expert_scale),
              _ptr(gate_up), _ptr(down), n, h, f, e, k, float(eps), mode, _ptr(out), _ptr(top_w), _ptr(top_i),
              _ptr(ws), ws.numel(), stream_handle(xn.device))
    return out, top_w, top_i


def moe_gateup_routed(xn, scores, per_expert_scale, gate_up, k, act=None, route=None):
    """gate/up with the softmax + top-k selection fused (model.py:228-231, 267-271)."""
    n, h = xn.shape
    e, _, f, _ = gate_up.shape
    _need(xn, BF16, "xn")
    _need(scores, torch.float32, "scores", (n, e))
    _need(per_expert_scale, BF16, "per_expert_scale", (e,))
    _need(gate_up, BF16, "gate_up", (e, 2, f, h))
    if act is None:
        act = torch.empty((n, k, f), dtype=BF16, device=xn.device)
    _need(act, BF16, "act", (n, k, f))
    if route is None:
        route = (torch.empty((n, k), dtype=torch.float32, device=xn.device),
                 torch.empty((n, k), dtype=torch.int32, device=xn.device))
    top_w, top_i = route
    _need(top_w, torch.float32, "top_w", (n, k))
    _need(top_i, torch.int32, "top_i", (n, k))
    _lib.call("g4mi_moe_gateup_routed", _ptr(xn), _ptr(scores), _ptr(per_expert_scale), _ptr(gate_up), n, h, f, e,
              k, _ptr(act), _ptr(top_w), _ptr(top_i), stream_handle(xn.device))
    return act, top_w, top_i


# -------------------------------------------------------------------- attention
def attention_min_splits(lmax: int) -> int:
    return int(_lib.lib().g4mi_attention_min_splits(lmax))


def decode_attention(q_raw, k_raw, v_raw, q_norm, k_norm, rope_cos, rope_sin, k_pages, v_pages, page_table, pos,
                     window, softcap, eps, lmax, n_split_max=None, append=True, ctx=None, ws=None):
    """Split-K decode attention over the paged cache (model.py:197-213) for B
    sequences: q_raw [B, NH, D], k_raw / v_raw [B, KV, D] (v_raw None on k==v
    layers), pages [num_pages, KV, PAGE, D], page_table [B, max_pages],
    pos [B] int32 (device).  page_table None: sequence b owns pages
    [b * max_pages, (b + 1) * max_pages) of the pool in order, max_pages =
    num_pages // B (the kernels compute page indices instead of loading
    them).  Appends the new K/V at pos when `append`.  Returns ctx [B, NH, D]
    bf16."""
    b, nh, d = q_raw.shape
    num_pages, kv, page, d2 = k_pages.shape
    if d2 != d:
        raise ValueError("head_dim mismatch between q and the cache")
    _need(q_raw, BF16, "q_raw")
    if append:
        _need(k_raw, BF16, "k_raw", (b, kv, d))
        if v_raw is not None:
            _need(v_raw, BF16, "v_raw", (b, kv, d))
    _need(q_norm, BF16, "q_norm", (d,))
    _need(k_norm, BF16, "k_norm", (d,))
    _need(rope_cos, BF16, "rope_cos")
    _need(rope_sin, BF16, "rope_sin", tuple(rope_cos.shape))
    _need(k_pages, BF16, "k_pages")
    _need(v_pages, BF16, "v_pages", tuple(k_pages.shape))
    _need(pos, torch.int32, "pos", (b,))
    if rope_cos.shape[1] != d // 2 or rope_cos.shape[0] < lmax:
        raise ValueError("rope tables must be [>= lmax, head_dim/2]")
    if page_table is None:
        max_pages = num_pages // b
    else:
        _need(page_table, torch.int32, "page_table")
        max_pages = page_table.shape[1]
        if page_table.shape[0] != b:
            raise ValueError("page_table must have one row per sequence")
    if n_split_max is None:
        n_split_max = max(attention_min_splits(lmax), 1)
    if ctx is None:
        ctx = torch.empty((b, nh, d), dtype=BF16, device=q_raw.device)
    _need(ctx, BF16, "ctx", (b, nh, d))
    nbytes = _lib.lib().g4mi_decode_attention_workspace_bytes(b, nh, d, lmax, n_split_max)
    if ws is None:
        # the shared scratch buffer may have held another layout (other B or
        # NH put data where this call's arrival counters sit): zero it
        ws = WORKSPACE.get(q_raw.device, "attention", nbytes)
        ws[:nbytes].zero_()
    _lib.call("g4mi_decode_attention", _ptr(q_raw), _ptr(k_raw), _ptr(v_raw), _ptr(q_norm), _ptr(k_norm),
              _ptr(rope_cos), _ptr(rope_sin), _ptr(k_pages), _ptr(v_pages), num_pages, _ptr(page_table), max_pages,
              _ptr(pos), b, nh, kv, d, page, int(window), float(softcap or 0.0), float(eps), 1 if append else 0,
              int(lmax), int(n_split_max), _ptr(ctx), _ptr(ws), ws.numel(), stream_handle(q_raw.device))
    return ctx


def kv_append(k_raw, v_raw, k_norm, rope_cos, rope_sin, k_pages, v_pages, page_table_row, pos, lmax, eps):
    """Writes rope(rms_norm(k_raw, k_norm)) and rms_norm(v_raw) of T tokens of
    one sequence at positions pos [T] (model.py:202-206).  k_raw [T, KV, D]."""
    t, kv, d = k_raw.shape
    num_pages, kv2, page, d2 = k_pages.shape
    if (kv2, d2) != (kv, d):
        raise ValueError("cache geometry does not match k_raw")
    _need(k_raw, BF16, "k_raw")
    if v_raw is not None:
        _need(v_raw, BF16, "v_raw", (t, kv, d))
    _need(k_norm, BF16, "k_norm", (d,))
    _need(k_pages, BF16, "k_pages")
    _need(v_pages, BF16, "v_pages", tuple(k_pages.shape))
    _need(page_table_row, torch.int32, "page_table_row")
    _need(pos, torch.int32, "pos", (t,))
    _lib.call("g4mi_kv_append", _ptr(k_raw), _ptr(v_raw), _ptr(k_norm), _ptr(rope_cos), _ptr(rope_sin),
              _ptr(k_pages), _ptr(v_pages), num_pages, _ptr(page_table_row), page_table_row.numel(), _ptr(pos), t, kv,
              d, page, int(lmax), float(eps), stream_handle(k_raw.device))


# ------------------------------------------------------------------- layer ops
def layer_in(mode, H, eps, input_ln, x_out, wq, wk, wv, q_rows, k_rows, v_rows, qkv_out, tok=None, embed=None,
             x_in=None, x1=None, mlp_out=None, moe_out=None, post_ff1=None, post_ff2=None, post_ff=None,
             layer_scalar=None):
    """q/k/v projection of rms_norm(x, input_ln) with x from the embedding
    (mode 0), the previous layer's tail (mode 1) or x_in (mode 2); mode 3
    takes x_in as the already-normalised input."""
    vocab = embed.shape[0] if embed is not None else 0
    _lib.call("g4mi_layer_in", int(mode), _ptr(tok), _ptr(embed), vocab, _ptr(x_in), _ptr(x1), _ptr(mlp_out),
              _ptr(moe_out), _ptr(post_ff1), _ptr(post_ff2), _ptr(post_ff), _ptr(layer_scalar), _ptr(input_ln),
              _ptr(x_out), _ptr(wq), q_rows, _ptr(wk), k_rows, _ptr(wv), v_rows, _ptr(qkv_out), H, float(eps),
              stream_handle(qkv_out.device))


def oproj(ctx, w, rows, K, out):
    _lib.call("g4mi_oproj", _ptr(ctx), _ptr(w), rows, K, _ptr(out), stream_handle(out.device))


def ffn_in(x, o, post_attn_ln, pre_ff_ln, pre_ff2_ln, x1_out, xe_out, gate, up, act_mlp, router_scale, router_proj,
           scores, H, eps, per_expert_scale=None, k=0, route=None, ws=None):
    """Post-attention residual, pre-FFN norms, dense gate/up and router scores
    (model.py:218-227, 301-315); with per_expert_scale and route = (top_w [k],
    top_i [k]) also the expert selection (model.py:228-231)."""
    I = gate.shape[0]
    E = router_proj.shape[0] if router_proj is not None else 0
    top_w, top_i = route if route is not None else (None, None)
    if per_expert_scale is not None and ws is None:
        ws = WORKSPACE.get(x.device, "ffn_in", int(_lib.lib().g4mi_ffn_in_workspace_bytes()))
    _lib.call("g4mi_ffn_in", _ptr(x), _ptr(o), _ptr(post_attn_ln), _ptr(pre_ff_ln), _ptr(pre_ff2_ln), _ptr(x1_out),
              _ptr(xe_out), _ptr(gate), _ptr(up), I, _ptr(act_mlp), _ptr(router_scale), _ptr(router_proj), E,
              _ptr(scores), _ptr(per_expert_scale), int(k), _ptr(top_w), _ptr(top_i), _ptr(ws),
              0 if ws is None else ws.numel(), H, float(eps), stream_handle(x.device))


def ffn_out(act_mlp, down, mlp_out, act_moe, experts_down, top_i, k, combine, moe_out, H, tail=None, eps=1e-6,
            ws=None):
    """Dense and expert down projections + combine (model.py:221, 272-294).
    With tail = dict(x1, post_ff1, post_ff2, post_ff, layer_scalar, next_ln,
    x_out, xn_out) the last block also applies the layer tail and the next
    norm (model.py:312-322, 298)."""
    I = down.shape[1]
    E = experts_down.shape[0] if experts_down is not None else 0
    F = experts_down.shape[2] if experts_down is not None else 0
    mode = {"bf16_running": _lib.COMBINE_BF16_RUNNING, "f32": _lib.COMBINE_F32}[combine]
    t = tail or {}
    if tail is not None and ws is None:
        ws = WORKSPACE.get(mlp_out.device, "ffn_out", int(_lib.lib().g4mi_ffn_out_workspace_bytes()))
    _lib.call("g4mi_ffn_out", _ptr(act_mlp), _ptr(down), I, _ptr(mlp_out), _ptr(act_moe), _ptr(experts_down),
              _ptr(top_i), E, k, F, mode, _ptr(moe_out), _ptr(t.get("x1")), _ptr(t.get("post_ff1")),
              _ptr(t.get("post_ff2")), _ptr(t.get("post_ff")), _ptr(t.get("layer_scalar")), _ptr(t.get("next_ln")),
              _ptr(t.get("x_out")), _ptr(t.get("xn_out")), float(eps), _ptr(ws), 0 if ws is None else ws.numel(), H,
              stream_handle(mlp_out.device))


def lm_head_normed(xn, embed, softcap, logits, blk_val, blk_idx):
    V, H = embed.shape
    _lib.call("g4mi_lm_head_normed", _ptr(xn), _ptr(embed), V, H, float(softcap or 0.0), _ptr(logits),
              _ptr(blk_val), _ptr(blk_idx), stream_handle(embed.device))


def lm_head_blocks(V: int) -> int:
    return int(_lib.lib().g4mi_lm_head_blocks(V))


def lm_head(x1, mlp_out, moe_out, post_ff1, post_ff2, post_ff, layer_scalar, final_norm, embed, softcap, eps,
            logits, blk_val, blk_idx):
    V, H = embed.shape
    _lib.call("g4mi_lm_head", _ptr(x1), _ptr(mlp_out), _ptr(moe_out), _ptr(post_ff1), _ptr(post_ff2),
              _ptr(post_ff), _ptr(layer_scalar), _ptr(final_norm), _ptr(embed), V, H, float(softcap or 0.0),
              float(eps), _ptr(logits), _ptr(blk_val), _ptr(blk_idx), stream_handle(embed.device))


def advance_feed(feed, tok, pos, hist=None):
    """pos += 1; tok = feed[pos]; hist[pos] = tok (teacher forcing through a prompt)."""
    _need(feed, torch.int32, "feed")
    _lib.call("g4mi_advance_feed", _ptr(feed), feed.numel(), _ptr(tok), _ptr(pos), _ptr(hist),
              0 if hist is None else hist.numel(), stream_handle(tok.device))


def argmax_finalize(blk_val, blk_idx, tok, pos=None, hist=None):
    _lib.call("g4mi_argmax_finalize", _ptr(blk_val), _ptr(blk_idx), blk_val.numel(), _ptr(tok), _ptr(pos),
              _ptr(hist), 0 if hist is None else hist.numel(), stream_handle(tok.device))


# ------------------------------------------------------------------------- sampling
def sample_params(temperature: float, top_p: float, seed: int, device, out: torch.Tensor | None = None):
    """A device g4mi_sample_params {f32 temperature, f32 top_p, u64 seed} (16 bytes).
    With `out`, the existing buffer is overwritten (stream-ordered copy)."""
    import struct

    raw = struct.pack("<ffQ", float(temperature), float(top_p), int(seed) & (2**64 - 1))
    host = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
    if out is None:
        out = torch.empty(16, dtype=torch.uint8, device=device)
    out.copy_(host)
    return out


def sample_workspace_bytes(V: int) -> int:
    return int(_lib.lib().g4mi_sample_workspace_bytes(V))


def sample(logits, top_k: int, params, tok, counter_mode: int = 1, pos=None, hist=None, ws=None):
    """model.py:414-424 on a device logits row [V] f32 -> tok [1] int32 (and
    pos/hist advanced when given).  `params` from sample_params()."""
    _need(logits, torch.float32, "logits")
    V = logits.numel()
    need = sample_workspace_bytes(V)
    if ws is None:
        ws = WORKSPACE.get(logits.device, "sample", need)
    _lib.call("g4mi_sample", _ptr(logits), V, int(top_k), _ptr(params), int(counter_mode), _ptr(tok), _ptr(pos),
              _ptr(hist), 0 if hist is None else hist.numel(), _ptr(ws), ws.numel(), stream_handle(logits.device))
    return tok


# ------------------------------------------------------------------------- prefill GEMMs
EP_BF16, EP_F32, EP_GATED = 0, 1, 2


def gemm(a, b, out=None, a_rows=None, epilogue=EP_BF16, pair_offset=0, n=None, row_scale=None, k_slices=1,
         lda=None, ldc=None, tiles=None, ntiles=None, m=None, ws_key="gemm"):
    """C = A[a_rows] . B^T on MFMA (bf16 in, f32 accumulate).

    a [*, K] bf16; b [N, K] bf16, or [G, ..., N, K] groups selected per
    64-row tile by `tiles` (int32 [T, 3] of (group, m0, m1), live count in
    `ntiles`, int32 [1]).  epilogue EP_BF16, EP_F32, or EP_GATED with the up
    rows at b + pair_offset elements and row_scale [M] f32 (n = gate rows).
    out [M, N] (row stride ldc).  ws_key names the split-K workspace (calls
    that may run at the same time on different streams need their own)."""
    K = a.shape[-1]
    M = m if m is not None else (a_rows.numel() if a_rows is not None else a.shape[0])
    N = n if n is not None else b.shape[-2]
    _need(a, BF16, "a")
    _need(b, BF16, "b")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32 if epilogue == EP_F32 else BF16, device=a.device)
    ws = None
    nbytes = int(_lib.lib().g4mi_gemm_workspace_bytes(M, N, k_slices))
    if nbytes:
        ws = WORKSPACE.get(a.device, ws_key, nbytes)
    group_stride = b.stride(0) if (tiles is not None and b.dim() >= 3) else 0
    _lib.call("g4mi_gemm_bf16", _ptr(a), a.stride(0) if lda is None else lda, _ptr(a_rows), _ptr(b), b.stride(-2),
              group_stride, int(pair_offset), M, N, K, _ptr(tiles), _ptr(ntiles),
              0 if tiles is None else tiles.shape[0], int(epilogue), _ptr(out),
              out.stride(0) if ldc is None else ldc, _ptr(row_scale), int(k_slices), _ptr(ws),
              0 if ws is None else ws.numel(), stream_handle(a.device))
    return out


def gemm_segments(a, bs, outs):
    """outs[s] = A . bs[s]^T (bf16) for up to 4 weight matrices sharing A, in
    one launch: a [M <= 16, K], bs[s] [N_s, K] contiguous, outs[s] [M, N_s]
    contiguous, N_s multiples of 16 (model.py:197-200 for B decode rows)."""
    M, K = a.shape
    _need(a, BF16, "a")
    if not 1 <= len(bs) == len(outs) <= 4:
        raise ValueError("gemm_segments takes 1 to 4 (weight, output) pairs")
    for b, c in zip(bs, outs):
        _need(b, BF16, "b")
        _need(c, BF16, "out", (M, b.shape[0]))
        if b.shape[1] != K or not b.is_contiguous() or not c.is_contiguous():
            raise ValueError("segments need contiguous [N_s, K] weights and [M, N_s] outputs")
    nseg = len(bs)
    bp = (ctypes.c_void_p * nseg)(*[b.data_ptr() for b in bs])
    cp = (ctypes.c_void_p * nseg)(*[c.data_ptr() for c in outs])
    nn = (ctypes.c_int64 * nseg)(*[b.shape[0] for b in bs])
    _lib.call("g4mi_gemm_bf16_segments", _ptr(a), a.stride(0), M, K, nseg, bp, nn, cp, stream_handle(a.device))
    return outs


def moe_decode_grouped(xn, top_w, top_i, gate_up, down, combine="bf16_running", out=None, ws=None):
    """The experts of a decode step of n <= 16 tokens (model.py:262-294 per
    token) with each selected expert's rows read once for all the tokens
    that chose it: xn [n, H], top_w/top_i [n, K] -> out [n, H] bf16."""
    n, H = xn.shape
    E, _, F, _ = gate_up.shape
    K = top_i.shape[1]
    _need(xn, BF16, "xn")
    _need(top_w, torch.float32, "top_w", (n, K))
    _need(top_i, torch.int32, "top_i", (n, K))
    _need(gate_up, BF16, "gate_up", (E, 2, F, H))
    _need(down, BF16, "down", (E, H, F))
    if out is None:
        out = torch.empty((n, H), dtype=BF16, device=xn.device)
    _need(out, BF16, "out", (n, H))
    nbytes = int(_lib.lib().g4mi_moe_prefill_workspace_bytes(n, K, E, F, H))
    if ws is None:
        ws = WORKSPACE.get(xn.device, "moe_decode_grouped", nbytes)
    mode = {"bf16_running": _lib.COMBINE_BF16_RUNNING, "f32": _lib.COMBINE_F32}[combine]
    _lib.call("g4mi_moe_decode_grouped", _ptr(xn), _ptr(top_w), _ptr(top_i), _ptr(gate_up), _ptr(down), n, H, F, E,
              K, mode, _ptr(out), _ptr(ws), ws.numel(), stream_handle(xn.device))
    return out


def moe_prefill(xn, top_w, top_i, gate_up, down, out=None, ws=None, combine=True):
    """model.py:241-250 for xn [n, H]: out [n, H] bf16 (selected experts only,
    grouped MFMA GEMMs).  combine=False leaves the per-slot f32 outputs in the
    workspace for rows_tail_experts and returns the workspace."""
    n, H = xn.shape
    E, _, F, _ = gate_up.shape
    K = top_i.shape[1]
    _need(xn, BF16, "xn")
    _need(top_w, torch.float32, "top_w", (n, K))
    _need(top_i, torch.int32, "top_i", (n, K))
    _need(gate_up, BF16, "gate_up", (E, 2, F, H))
    _need(down, BF16, "down", (E, H, F))
    if out is None and combine:
        out = torch.empty((n, H), dtype=BF16, device=xn.device)
    nbytes = int(_lib.lib().g4mi_moe_prefill_workspace_bytes(n, K, E, F, H))
    if ws is None:
        ws = WORKSPACE.get(xn.device, "moe_prefill", nbytes)
    _lib.call("g4mi_moe_prefill", _ptr(xn), _ptr(top_w), _ptr(top_i), _ptr(gate_up), _ptr(down), n, H, F, E, K,
              _ptr(out if combine else None), _ptr(ws), ws.numel(), stream_handle(xn.device))
    return out if combine else ws


# ------------------------------------------------------------------ prefill rows
def rows_embed(tok, embed, input_ln, eps, x_out, xn_out):
    """x = bf16(embed[tok] * bf16(sqrt(H))), xn = rms_norm(x, input_ln) for
    n token rows (model.py:355-357, 298)."""
    n = tok.numel()
    V, H = embed.shape
    _lib.call("g4mi_rows_embed", _ptr(tok), n, _ptr(embed), V, _ptr(input_ln), H, float(eps), _ptr(x_out),
              _ptr(xn_out), stream_handle(embed.device))


def rows_post_attn(x, o, post_attn_ln, pre_ff_ln, pre_ff2_ln, eps, x1_out, xm_out, xe_out=None):
    """x1 = bf16(x + rms_norm(o, post_attn_ln)), xm = rms_norm(x1, pre_ff_ln),
    xe = rms_norm(x1, pre_ff2_ln) for n rows (model.py:301-315)."""
    n, H = x.shape
    _lib.call("g4mi_rows_post_attn", _ptr(x), _ptr(o), n, _ptr(post_attn_ln), _ptr(pre_ff_ln), _ptr(pre_ff2_ln), H,
              float(eps), _ptr(x1_out), _ptr(xm_out), _ptr(xe_out), stream_handle(x.device))


def rows_tail(x1, mlp_out, moe_out, post_ff1, post_ff2, post_ff, layer_scalar, next_ln, eps, x_out, xn_out):
    """The layer tail of n rows (model.py:312-322) and the next input norm."""
    n, H = x1.shape
    _lib.call("g4mi_rows_tail", _ptr(x1), _ptr(mlp_out), _ptr(moe_out), n, _ptr(post_ff1), _ptr(post_ff2),
              _ptr(post_ff), _ptr(layer_scalar), _ptr(next_ln), H, float(eps), _ptr(x_out), _ptr(xn_out),
              stream_handle(x1.device))


def rows_tail_experts(x1, mlp_out, moe_ws, K, E, F, post_ff1, post_ff2, post_ff, layer_scalar, next_ln, eps, x_out,
                      xn_out):
    """rows_tail with the MoE output combined from the per-slot outputs that
    moe_prefill(combine=False) left in moe_ws (model.py:250, 312-322), in one
    launch; identical to moe_prefill + rows_tail."""
    n, H = x1.shape
    _lib.call("g4mi_rows_tail_experts", _ptr(x1), _ptr(mlp_out), n, K, E, F, _ptr(post_ff1), _ptr(post_ff2),
              _ptr(post_ff), _ptr(layer_scalar), _ptr(next_ln), H, float(eps), _ptr(x_out), _ptr(xn_out), _ptr(moe_ws),
              moe_ws.numel(), stream_handle(x1.device))


def prefill_gemm(a, w, out, epilogue=EP_BF16, pair_offset=0, n=None, blocks=256, ws_key="gemm"):
    """gemm() for the batched prefill: activations a [M, K] times the weight
    rows w [N, K] on the MFMA kernels (M <= 16: the skinny kernel; more rows:
    the tile kernel, split over K when there are fewer tiles than `blocks`);
    the gated epilogue takes the gate rows w and the up rows at w +
    pair_offset elements."""
    M, K = a.shape
    N = n if n is not None else w.shape[0]
    k_slices = 1
    if epilogue != EP_GATED and M > 16:  # M <= 16 runs the skinny kernel (K split inside the block)
        tm = 64 if M <= 64 else 128
        tiles = ((M + tm - 1) // tm) * ((N + 127) // 128)
        if tiles < blocks:
            k_slices = max(1, min((blocks + tiles - 1) // tiles, K // 128, 16))
    return gemm(a, w, out=out, epilogue=epilogue, pair_offset=pair_offset, n=N, k_slices=k_slices, ws_key=ws_key)


def q_norm_rope(q, q_norm, rope_cos, rope_sin, p0, eps):
    """q [T, NH, D] = rope(rms_norm(q, q_norm)) in place at positions p0 + t
    (model.py:198-199)."""
    T, NH, D = q.shape
    _need(q, BF16, "q")
    _need(q_norm, BF16, "q_norm", (D,))
    _lib.call("g4mi_q_norm_rope", _ptr(q), _ptr(q_norm), _ptr(rope_cos), _ptr(rope_sin), T, NH, D, int(p0),
              rope_cos.shape[0], float(eps), stream_handle(q.device))
    return q


def prefill_attention(q, k_pages, v_pages, page_table_row, p0, window, softcap, ctx=None):
    """Causal prefill attention of T query rows q [T, NH, D] (normed and
    rotated, positions p0 + t) over the paged cache (model.py:207-213, T > 1).
    Returns ctx [T, NH, D] bf16."""
    T, NH, D = q.shape
    num_pages, KV, page, D2 = k_pages.shape
    if D2 != D:
        raise ValueError("head_dim mismatch between q and the cache")
    _need(q, BF16, "q")
    _need(k_pages, BF16, "k_pages")
    _need(v_pages, BF16, "v_pages", tuple(k_pages.shape))
    _need(page_table_row, torch.int32, "page_table_row")
    if ctx is None:
        ctx = torch.empty((T, NH, D), dtype=BF16, device=q.device)
    _need(ctx, BF16, "ctx", (T, NH, D))
    _lib.call("g4mi_prefill_attention", _ptr(q), _ptr(k_pages), _ptr(v_pages), num_pages, _ptr(page_table_row),
              page_table_row.numel(), page, T, int(p0), NH, KV, D, int(window), float(softcap or 0.0), _ptr(ctx),
              stream_handle(q.device))
    return ctx


def argmax_rows(logits_bf16, softcap, tok, pos=None, hist=None, logits_f32=None):
    """Greedy head for B rows of bf16 logits [B, V] (model.py:381-385, 416):
    softcap, first index of the maximum -> tok [B]; with pos [B] / hist
    [B, L] the positions advance and the tokens are recorded."""
    B, V = logits_bf16.shape
    _need(logits_bf16, BF16, "logits")
    _need(tok, torch.int32, "tok", (B,))
    hist_len = 0
    if hist is not None:
        _need(hist, torch.int32, "hist")
        hist_len = hist.shape[1]
    ws = WORKSPACE.get(logits_bf16.device, "argmax_rows", int(_lib.lib().g4mi_argmax_rows_workspace_bytes(B)))
    _lib.call("g4mi_argmax_rows", _ptr(logits_bf16), B, V, float(softcap or 0.0), _ptr(logits_f32), _ptr(tok),
              _ptr(pos), _ptr(hist), hist_len, _ptr(ws), ws.numel(), stream_handle(logits_bf16.device))


# ------------------------------------------------------------------------- model primitives
def _dtype_code(t: torch.Tensor, name: str) -> int:
    if t.dtype == torch.bfloat16:
        return 0
    if t.dtype == torch.float32:
        return 1
    raise TypeError(f"{name}: bf16 or f32 expected, got {t.dtype}")


def _on_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name}: a device tensor is expected (the kernels have no CPU path)")


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """model.py:42-47 over the last axis of x (bf16 or f32) -> x's dtype."""
    _on_device(x, "rms_norm x")
    x = x.contiguous()
    dim = x.shape[-1]
    w_code = 0
    if weight is not None:
        weight = weight.contiguous()
        w_code = _dtype_code(weight, "rms_norm weight")
        if weight.numel() != dim:
            raise ValueError(f"rms_norm: weight has {weight.numel()} elements, x's last axis {dim}")
    out = torch.empty_like(x)
    _lib.call("g4mi_rms_norm", _ptr(x), _dtype_code(x, "rms_norm x"), _ptr(weight), w_code, x.numel() // max(dim, 1),
              dim, float(eps), _ptr(out), stream_handle(x.device))
    return out


def gelu(x: torch.Tensor) -> torch.Tensor:
    """model.py:50-51: tanh-approximation GELU, x's dtype."""
    _on_device(x, "gelu x")
    x = x.contiguous()
    out = torch.empty_like(x)
    _lib.call("g4mi_gelu_tanh", _ptr(x), _dtype_code(x, "gelu x"), x.numel(), _ptr(out), stream_handle(x.device))
    return out


def rope_tables(positions: torch.Tensor, inv_freq: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """model.py:64-67: (cos, sin) f32 [T, 2 * len(inv_freq)] on positions' device."""
    _on_device(positions, "rope_tables positions")
    pos = positions.reshape(-1).to(torch.int32).contiguous()
    inv = inv_freq.to(device=pos.device, dtype=torch.float32).contiguous()
    T, half = pos.numel(), inv.numel()
    cos = torch.empty((T, 2 * half), dtype=torch.float32, device=pos.device)
    sin = torch.empty_like(cos)
    _lib.call("g4mi_rope_tables", _ptr(pos), T, _ptr(inv), half, _ptr(cos), _ptr(sin), stream_handle(pos.device))
    return cos, sin


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """model.py:70-78: x [B, T, ..., D]; cos/sin [T, D] broadcast over B and
    the head axes."""
    _on_device(x, "apply_rope x")
    if x.ndim < 3:
        raise ValueError("apply_rope: x must be [B, T, ..., D]")
    x = x.contiguous()
    B, T, D = x.shape[0], x.shape[1], x.shape[-1]
    inner = x.numel() // max(B * T * D, 1)
    c = cos.to(device=x.device, dtype=torch.float32).reshape(-1, D).contiguous()
    s = sin.to(device=x.device, dtype=torch.float32).reshape(-1, D).contiguous()
    if c.shape[0] != T or s.shape[0] != T:
        raise ValueError(f"apply_rope: tables hold {c.shape[0]} positions, x {T}")
    out = torch.empty_like(x)
    _lib.call("g4mi_apply_rope", _ptr(x), _dtype_code(x, "apply_rope x"), _ptr(c), _ptr(s), B, T, inner, D, _ptr(out),
              stream_handle(x.device))
    return out


def decode_attention_noalloc(q_raw, k_raw, v_raw, q_norm, k_norm, rope_cos, rope_sin, k_pages, v_pages, page_table,
                             pos, window, softcap, eps, lmax, n_split_max, ctx, append=True):
    """decode_attention through g4mi_decode_attention_noalloc: the same
    kernels with the split-K scratch in the library's per-device array (no
    workspace argument, nothing allocated here: ctx is the caller's)."""
    b, nh, d = q_raw.shape
    num_pages, kv, page, _ = k_pages.shape
    _need(ctx, BF16, "ctx", (b, nh, d))
    _need(pos, torch.int32, "pos", (b,))
    if page_table is not None:
        _need(page_table, torch.int32, "page_table")
    max_pages = num_pages // b if page_table is None else page_table.shape[1]
    _lib.call("g4mi_decode_attention_noalloc", _ptr(q_raw), _ptr(k_raw), _ptr(v_raw), _ptr(q_norm), _ptr(k_norm),
              _ptr(rope_cos), _ptr(rope_sin), _ptr(k_pages), _ptr(v_pages), num_pages, _ptr(page_table),
              max_pages, _ptr(pos), b, nh, kv, d, page, int(window), float(softcap or 0.0), float(eps),
              1 if append else 0, int(lmax), int(n_split_max), _ptr(ctx), stream_handle(q_raw.device))
    return ctx
