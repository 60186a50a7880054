"""Gemma-4 MoE text decoder on one MI355X (the model API of gemma4_tpu/model.py).

Parameter layout, cache, masks and sampling keep the reference's names and
signatures; the math runs in libg4mi's gfx950 kernels.
"""

from __future__ import annotations

import math

import torch

from .config import FULL, SLIDING, TextConfig

NEG_INF = -1e30


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
