"""Gemma-4 MoE text-stack configuration (the fields of gemma4_tpu/config.py).

``TextConfig`` keeps the reference's field names and per-layer-type helpers
(config.py:11-49) so callers written against it run unchanged.  One field is
added with a default: ``attn_logit_softcapping`` (None = off, the reference's
behaviour; the isolated-attention workload sets it to 50).
"""

from __future__ import annotations

import dataclasses
import json
import math
import os

FULL = "full_attention"
SLIDING = "sliding_attention"


@dataclasses.dataclass(frozen=True)
class TextConfig:
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    head_dim: int
    global_head_dim: int
    num_key_value_heads: int
    num_global_key_value_heads: int
    intermediate_size: int
    moe_intermediate_size: int
    num_experts: int
    top_k_experts: int
    sliding_window: int
    rms_norm_eps: float
    vocab_size: int
    final_logit_softcapping: float | None
    attention_k_eq_v: bool
    enable_moe_block: bool
    layer_types: tuple[str, ...]
    rope_theta_sliding: float
    rope_theta_full: float
    rope_partial_rotary_factor_full: float
    eos_token_ids: tuple[int, ...]
    attn_logit_softcapping: float | None = None

    @property
    def embed_scale(self) -> float:
        return math.sqrt(self.hidden_size)

    def head_dim_for(self, layer_type: str) -> int:
        """config.py:40-41: full layers use global_head_dim."""
        return self.global_head_dim if layer_type == FULL else self.head_dim

    def kv_heads_for(self, layer_type: str) -> int:
        """config.py:43-46: the global KV-head count applies to k==v full layers only."""
        if layer_type == FULL and self.attention_k_eq_v:
            return self.num_global_key_value_heads
        return self.num_key_value_heads

    def k_eq_v_for(self, layer_type: str) -> bool:
        """config.py:48-49: full layers share the K projection as V."""
        return layer_type == FULL and self.attention_k_eq_v

    def replace(self, **kw) -> "TextConfig":
        return dataclasses.replace(self, **kw)


def _eos_ids(raw: dict, text: dict, gen_path: str) -> tuple[int, ...]:
    ids: list[int] = []
    if os.path.exists(gen_path):
        with open(gen_path) as f:
            eos = json.load(f).get("eos_token_id", [])
        ids = [eos] if isinstance(eos, int) else list(eos)
    if not ids:
        eos = raw.get("eos_token_id", text.get("eos_token_id", 1))
        ids = [eos] if isinstance(eos, int) else list(eos)
    return tuple(int(i) for i in ids)


def load_text_config(model_dir: str) -> TextConfig:
    """Reads ``config.json["text_config"]`` (+ generation_config.json EOS ids),
    as config.py:52-92 does.  Also accepts the per-layer-type layout newer
    transformers versions write (``per_layer_config``)."""
    with open(os.path.join(model_dir, "config.json")) as f:
        raw = json.load(f)
    tc = raw.get("text_config", raw)
    per = tc.get("per_layer_config") or {}
    full = per.get(FULL, {}) if isinstance(per, dict) else {}
    rope = tc["rope_parameters"]
    head_dim = tc["head_dim"]
    return TextConfig(
        hidden_size=tc["hidden_size"],
        num_hidden_layers=tc["num_hidden_layers"],
        num_attention_heads=tc["num_attention_heads"],
        head_dim=head_dim,
        global_head_dim=tc.get("global_head_dim") or full.get("head_dim") or head_dim,
        num_key_value_heads=tc["num_key_value_heads"],
        num_global_key_value_heads=(
            tc.get("num_global_key_value_heads")
            or full.get("num_key_value_heads")
            or tc["num_key_value_heads"]
        ),
        intermediate_size=tc["intermediate_size"],
        moe_intermediate_size=tc["moe_intermediate_size"],
        num_experts=tc["num_experts"],
        top_k_experts=tc["top_k_experts"],
        sliding_window=tc["sliding_window"],
        rms_norm_eps=tc["rms_norm_eps"],
        vocab_size=tc["vocab_size"],
        final_logit_softcapping=tc.get("final_logit_softcapping"),
        attention_k_eq_v=bool(tc.get("attention_k_eq_v", False)),
        enable_moe_block=bool(tc.get("enable_moe_block", False)),
        layer_types=tuple(tc["layer_types"]),
        rope_theta_sliding=rope[SLIDING]["rope_theta"],
        rope_theta_full=rope[FULL]["rope_theta"],
        rope_partial_rotary_factor_full=rope[FULL].get("partial_rotary_factor", 1.0),
        eos_token_ids=_eos_ids(raw, tc, os.path.join(model_dir, "generation_config.json")),
        attn_logit_softcapping=tc.get("attn_logit_softcapping"),
    )


def write_text_config(cfg: TextConfig, model_dir: str) -> str:
    """Writes a config.json that :func:`load_text_config` reads back to ``cfg``."""
    os.makedirs(model_dir, exist_ok=True)
    tc = {
        "hidden_size": cfg.hidden_size,
        "num_hidden_layers": cfg.num_hidden_layers,
        "num_attention_heads": cfg.num_attention_heads,
        "head_dim": cfg.head_dim,
        "global_head_dim": cfg.global_head_dim,
        "num_key_value_heads": cfg.num_key_value_heads,
        "num_global_key_value_heads": cfg.num_global_key_value_heads,
        "intermediate_size": cfg.intermediate_size,
        "moe_intermediate_size": cfg.moe_intermediate_size,
        "num_experts": cfg.num_experts,
        "top_k_experts": cfg.top_k_experts,
        "sliding_window": cfg.sliding_window,
        "rms_norm_eps": cfg.rms_norm_eps,
        "vocab_size": cfg.vocab_size,
        "final_logit_softcapping": cfg.final_logit_softcapping,
        "attention_k_eq_v": cfg.attention_k_eq_v,
        "enable_moe_block": cfg.enable_moe_block,
        "layer_types": list(cfg.layer_types),
        "rope_parameters": {
            SLIDING: {"rope_type": "default", "rope_theta": cfg.rope_theta_sliding},
            FULL: {
                "rope_type": "proportional",
                "rope_theta": cfg.rope_theta_full,
                "partial_rotary_factor": cfg.rope_partial_rotary_factor_full,
            },
        },
        "attn_logit_softcapping": cfg.attn_logit_softcapping,
    }
    path = os.path.join(model_dir, "config.json")
    with open(path, "w") as f:
        json.dump({"text_config": tc, "eos_token_id": list(cfg.eos_token_ids)}, f, indent=1)
    return path


def tiny_parity_config() -> TextConfig:
    """4 layers (3 sliding window 64, 1 full k==v), hidden 256, 4 q / 2 KV heads
    at head_dim 64, dense MLP 512 beside 16 experts top-4 of width 128, vocab
    4096, final softcap 30.  The last layer is the full one, as the Gemma-4
    layer pattern requires."""
    return TextConfig(
        hidden_size=256,
        num_hidden_layers=4,
        num_attention_heads=4,
        head_dim=64,
        global_head_dim=64,
        num_key_value_heads=2,
        num_global_key_value_heads=2,
        intermediate_size=512,
        moe_intermediate_size=128,
        num_experts=16,
        top_k_experts=4,
        sliding_window=64,
        rms_norm_eps=1e-6,
        vocab_size=4096,
        final_logit_softcapping=30.0,
        attention_k_eq_v=True,
        enable_moe_block=True,
        layer_types=(SLIDING, SLIDING, SLIDING, FULL),
        rope_theta_sliding=10000.0,
        rope_theta_full=1000000.0,
        rope_partial_rotary_factor_full=0.25,
        eos_token_ids=(1,),
    )


def gemma4_26b_a4b_config() -> TextConfig:
    """The google/gemma-4-26B-A4B text stack: 30 layers (full attention at every
    sixth, i = 5, 11, 17, 23, 29), hidden 2816, 16 query heads, sliding layers
    8 KV heads x 256 (window 1024), full layers 2 KV heads x 512 with k==v,
    dense MLP 2112 beside 128 experts top-8 of width 704, vocab 262,144."""
    types = tuple(FULL if i % 6 == 5 else SLIDING for i in range(30))
    return TextConfig(
        hidden_size=2816,
        num_hidden_layers=30,
        num_attention_heads=16,
        head_dim=256,
        global_head_dim=512,
        num_key_value_heads=8,
        num_global_key_value_heads=2,
        intermediate_size=2112,
        moe_intermediate_size=704,
        num_experts=128,
        top_k_experts=8,
        sliding_window=1024,
        rms_norm_eps=1e-6,
        vocab_size=262144,
        final_logit_softcapping=30.0,
        attention_k_eq_v=True,
        enable_moe_block=True,
        layer_types=types,
        rope_theta_sliding=10000.0,
        rope_theta_full=1000000.0,
        rope_partial_rotary_factor_full=0.25,
        eos_token_ids=(1, 106),
    )
