"""Weights: layout, byte accounting, seeded random init on the GPU, and the
safetensors loader (gemma4_tpu/weights.py).

All parameters live in HBM as bf16 torch tensors in the reference's canonical
shapes (model.param_shapes, model.py:84-117): every GEMV row is contiguous, so
the kernels read 16-byte vectors straight out of it.
"""

from __future__ import annotations

import glob
import json
import os
from typing import Callable

import torch

from .config import TextConfig


# ------------------------------------------------------------------ accounting
def param_bytes(cfg: TextConfig) -> int:
    """weights.py:138-139: bf16 bytes of every parameter."""
    from .model import param_shapes

    total = 0
    for s in param_shapes(cfg).values():
        n = 1
        for d in s:
            n *= d
        total += 2 * n
    return total


def active_params_per_token(cfg: TextConfig) -> int:
    """weights.py:142-159: parameters one decode token reads (q, k, [v], o,
    dense MLP, router, k experts, tied lm_head)."""
    h = cfg.hidden_size
    total = 0
    for lt in cfg.layer_types:
        d, kv = cfg.head_dim_for(lt), cfg.kv_heads_for(lt)
        qo = 2 * cfg.num_attention_heads * d * h
        kvp = (1 if cfg.k_eq_v_for(lt) else 2) * kv * d * h
        total += qo + kvp + 3 * cfg.intermediate_size * h
        if cfg.enable_moe_block:
            total += cfg.num_experts * h + cfg.top_k_experts * 3 * cfg.moe_intermediate_size * h
    return total + cfg.vocab_size * h


def kv_bytes_per_token(cfg: TextConfig) -> int:
    """session.py:49-50: bf16 K and V bytes one cached position costs over all layers."""
    return sum(2 * 2 * cfg.kv_heads_for(lt) * cfg.head_dim_for(lt) for lt in cfg.layer_types)


def decode_bytes(cfg: TextConfig, pos: int) -> int:
    """Algorithmic HBM bytes of one batch-1 decode step at position `pos`:
    active weights plus the K/V each layer must read (window-clamped on
    sliding layers)."""
    kv = 0
    for lt in cfg.layer_types:
        n = pos + 1 if lt != "sliding_attention" else min(pos + 1, cfg.sliding_window)
        kv += 2 * 2 * cfg.kv_heads_for(lt) * cfg.head_dim_for(lt) * n
    return 2 * active_params_per_token(cfg) + kv


# ------------------------------------------------------------------ random init
def _fnv1a64(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def tensor_key(seed: int, name: str) -> int:
    """Philox key of one named tensor: FNV-1a 64 of the name, xor seed * golden ratio."""
    return _fnv1a64(name.encode()) ^ ((seed * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)


def init_random_params(
    cfg: TextConfig,
    seed: int,
    std: float = 0.02,
    device: str | torch.device = "cuda",
    ones: tuple[str, ...] = ("layer_scalar",),
    progress: Callable[[int, int, str], None] | None = None,
) -> dict[str, torch.Tensor]:
    """Every parameter of param_shapes ~ N(0, std) in bf16, generated on the GPU
    by the library's Philox generator (per-tensor key from `seed` and the name).

    Names ending with an entry of `ones` are set to 1.0.  The default keeps
    `layer_scalar` at 1: HF Gemma-4 holds it as a buffer, so the reference's
    parity test (which re-draws every *parameter*, tests/test_parity.py:70-72)
    leaves it at one, and a random scalar of scale 0.02 per layer would shrink
    the residual stream below bf16 range within ~25 layers."""
    from . import ops
    from .model import param_shapes

    shapes = param_shapes(cfg)
    params: dict[str, torch.Tensor] = {}
    for i, (name, shape) in enumerate(shapes.items()):
        t = torch.empty(shape, dtype=torch.bfloat16, device=device)
        if any(name.endswith(s) for s in ones):
            t.fill_(1.0)
        else:
            ops.fill_normal_(t, tensor_key(seed, name), std)
        params[name] = t
        if progress:
            progress(i + 1, len(shapes), name)
    return params


# ------------------------------------------------------------------ checkpoints
def checkpoint_key_map(cfg: TextConfig, prefix: str = "model.language_model.") -> dict[str, str]:
    """Checkpoint tensor name -> flat parameter name (weights.py:30-58)."""
    out = {prefix + "embed_tokens.weight": "embed", prefix + "norm.weight": "norm"}
    norms = (
        "input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm", "post_feedforward_layernorm",
        "pre_feedforward_layernorm_2", "post_feedforward_layernorm_1", "post_feedforward_layernorm_2",
    )
    for i in range(cfg.num_hidden_layers):
        src, dst = f"{prefix}layers.{i}.", f"layers.{i}."
        out.update({f"{src}{n}.weight": dst + n for n in norms})
        out[src + "layer_scalar"] = dst + "layer_scalar"
        out.update({f"{src}self_attn.{n}.weight": dst + n
                    for n in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm")})
        out.update({f"{src}mlp.{n}.weight": f"{dst}mlp.{n}" for n in ("gate_proj", "up_proj", "down_proj")})
        out[src + "router.proj.weight"] = dst + "router.proj"
        for n in ("router.scale", "router.per_expert_scale", "experts.gate_up_proj", "experts.down_proj"):
            out[src + n] = dst + n
    return out


def _reshape(cfg: TextConfig, flat: str, t: torch.Tensor) -> torch.Tensor:
    from .model import param_shapes

    want = tuple(param_shapes(cfg)[flat])
    if tuple(t.shape) == want:
        return t
    n = 1
    for d in want:
        n *= d
    if t.numel() != n:
        raise ValueError(f"{flat}: checkpoint shape {tuple(t.shape)} != expected {want}")
    return t.reshape(want)


def params_from_arrays(cfg: TextConfig, get, names, mesh=None, prefix: str = "model.language_model.",
                       device: str | torch.device = "cuda") -> dict[str, torch.Tensor]:
    """Builds device params from any ``name -> array`` accessor (weights.py:70-83).
    Arrays may be torch tensors or numpy arrays (bf16 numpy arrays are accepted
    as uint16 bit patterns).  `mesh` is accepted for signature compatibility."""
    from .model import param_shapes

    shapes = param_shapes(cfg)
    key_map = checkpoint_key_map(cfg, prefix)
    params: dict[str, torch.Tensor] = {}
    for ck in names:
        flat = key_map.get(ck)
        if flat is None or flat not in shapes or flat in params:
            continue
        arr = get(ck)
        if not isinstance(arr, torch.Tensor):
            import numpy as np

            a = np.asarray(arr)
            arr = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16) if a.dtype.itemsize == 2 and \
                a.dtype.kind in "uV" else torch.from_numpy(a)
        params[flat] = _reshape(cfg, flat, arr.to(torch.bfloat16)).contiguous().to(device)
    return params


def load_params(cfg: TextConfig, model_dir: str, mesh=None,
                progress: Callable[[int, int, str], None] | None = None,
                device: str | torch.device = "cuda") -> dict[str, torch.Tensor]:
    """Streams every safetensors tensor of `model_dir` into HBM (weights.py:86-135).
    Raises FileNotFoundError without safetensors and KeyError for missing params."""
    from safetensors import safe_open

    from .model import param_shapes

    shapes = param_shapes(cfg)
    key_map = checkpoint_key_map(cfg)
    files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no safetensors under {model_dir}")
    index = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            wmap = json.load(f)["weight_map"]
        by_file: dict[str, list[str]] = {}
        for ck in key_map:
            if ck in wmap:
                by_file.setdefault(os.path.join(model_dir, wmap[ck]), []).append(ck)
    else:
        by_file = {f: list(key_map) for f in files}
    params: dict[str, torch.Tensor] = {}
    for path, keys in by_file.items():
        with safe_open(path, framework="pt", device="cpu") as f:
            have = set(f.keys())
            for ck in keys:
                flat = key_map[ck]
                if ck not in have or flat not in shapes:
                    continue
                t = _reshape(cfg, flat, f.get_tensor(ck).to(torch.bfloat16))
                params[flat] = t.contiguous().to(device)
                if progress:
                    progress(len(params), len(shapes), flat)
    missing = sorted(set(shapes) - set(params))
    if missing:
        raise KeyError(f"missing {len(missing)} params, e.g. {missing[:5]}")
    return params
