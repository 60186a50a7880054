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
