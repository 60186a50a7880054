"""Writes tests/golden/hf_tiny_c1.npz: HF transformers Gemma-4 logits for the
tiny parity model, the oracle's independent cross-check.

This follows the reference's own parity procedure (tests/test_parity.py:29-159:
a tiny random HF Gemma4ForCausalLM, eager attention and eager experts, compared
on logits), with two changes:
  * the weights are the seeded values of the library's generator (the numpy
    restatement in oracle/philox.py), so the same model runs on the GPU;
  * the HF router is fed pre_feedforward_layernorm_2(residual), as the
    reference's model.py:315 does, instead of the raw residual HF 5.x uses.

Run from the repo root in a container that has transformers (no network):
    python tests/golden/make_hf_fixtures.py
The model is built locally from a config object; nothing is downloaded.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "kaggle-tpu-inference_amd"))

from gemma4_mi.config import tiny_parity_config  # noqa: E402
from oracle import twin  # noqa: E402

SEED = 0
PROMPT_SEED = 0
PROMPT_LEN = 128
N_DECODE = 32
KEEP_ROWS = (0, 1, 2, 31, 63, 64, 65, 100, 127, 128, 129, 140, 150, 159)


def build_hf(cfg, params):
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM

    hf_cfg = Gemma4TextConfig(
        vocab_size=cfg.vocab_size,
        hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size,
        num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads,
        head_dim=cfg.head_dim,
        global_head_dim=cfg.global_head_dim,
        num_global_key_value_heads=cfg.num_global_key_value_heads,
        sliding_window=cfg.sliding_window,
        layer_types=list(cfg.layer_types),
        num_experts=cfg.num_experts,
        top_k_experts=cfg.top_k_experts,
        moe_intermediate_size=cfg.moe_intermediate_size,
        enable_moe_block=True,
        attention_k_eq_v=True,
        final_logit_softcapping=cfg.final_logit_softcapping,
        tie_word_embeddings=True,
        hidden_size_per_layer_input=0,
        num_kv_shared_layers=0,
        rms_norm_eps=cfg.rms_norm_eps,
        hidden_activation="gelu_pytorch_tanh",
        rope_parameters={
            "full_attention": {
                "rope_type": "proportional",
                "rope_theta": cfg.rope_theta_full,
                "partial_rotary_factor": cfg.rope_partial_rotary_factor_full,
            },
            "sliding_attention": {"rope_type": "default", "rope_theta": cfg.rope_theta_sliding},
        },
        use_bidirectional_attention="vision",
        attn_implementation="eager",
        max_position_embeddings=4096,
    )
    hf_cfg._experts_implementation = "eager"
    model = Gemma4ForCausalLM(hf_cfg).to(torch.bfloat16).eval()

    sd = {}
    sd["model.embed_tokens.weight"] = params["embed"]
    sd["model.norm.weight"] = params["norm"]
    for i in range(cfg.num_hidden_layers):
        s, d = f"model.layers.{i}.", f"layers.{i}."
        for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                  "post_feedforward_layernorm", "pre_feedforward_layernorm_2", "post_feedforward_layernorm_1",
                  "post_feedforward_layernorm_2"):
            sd[s + n + ".weight"] = params[d + n]
        for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
            if d + n in params:
                t = params[d + n]
                sd[s + "self_attn." + n + ".weight"] = t.reshape(t.shape[0], -1) if n == "o_proj" else t.reshape(-1, cfg.hidden_size)
        sd[s + "self_attn.q_norm.weight"] = params[d + "q_norm"]
        sd[s + "self_attn.k_norm.weight"] = params[d + "k_norm"]
        for n in ("gate_proj", "up_proj", "down_proj"):
            sd[s + "mlp." + n + ".weight"] = params[d + "mlp." + n]
        sd[s + "router.proj.weight"] = params[d + "router.proj"]
        sd[s + "router.scale"] = params[d + "router.scale"]
        sd[s + "router.per_expert_scale"] = params[d + "router.per_expert_scale"]
        gu = params[d + "experts.gate_up_proj"]
        sd[s + "experts.gate_up_proj"] = gu.reshape(gu.shape[0], -1, gu.shape[-1])
        sd[s + "experts.down_proj"] = params[d + "experts.down_proj"]
        sd[s + "layer_scalar"] = params[d + "layer_scalar"]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    missing = [m for m in missing if not m.endswith("lm_head.weight")]
    assert not missing and not unexpected, (missing, unexpected)

    # Route on pre_feedforward_layernorm_2(residual), as model.py:315 does.
    routes = []
    for layer in model.model.layers:
        orig = layer.router.forward
        pre = layer.pre_feedforward_layernorm_2

        def fwd(h, orig=orig, pre=pre):
            probs, w, idx = orig(pre(h))
            routes.append(idx.detach().clone())
            return probs, w, idx

        layer.router.forward = fwd
    return model, routes


def main() -> int:
    cfg = tiny_parity_config()
    params = twin.random_params(cfg, SEED)
    model, routes = build_hf(cfg, params)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg.vocab_size, size=PROMPT_LEN).astype(np.int64)

    # greedy continuation with HF itself, then one causal pass over all 160 ids
    ids = torch.tensor(prompt)[None]
    with torch.no_grad():
        for _ in range(N_DECODE):
            routes.clear()
            lg = model(input_ids=ids).logits[0, -1].float()
            ids = torch.cat([ids, torch.tensor([[int(torch.argmax(lg))]])], 1)
        routes.clear()
        logits = model(input_ids=ids).logits[0].float().numpy()
    top_i = torch.stack([r.reshape(-1, cfg.top_k_experts) for r in routes], 0).numpy().astype(np.int16)

    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hf_tiny_c1.npz")
    np.savez_compressed(
        out,
        ids=ids[0].numpy().astype(np.int32),
        prompt_len=np.int32(PROMPT_LEN),
        rows=np.asarray(KEEP_ROWS, np.int32),
        logits_rows=logits[list(KEEP_ROWS)].astype(np.float32),
        argmax=logits.argmax(-1).astype(np.int32),
        top2_gap=np.sort(logits, -1)[:, -1] - np.sort(logits, -1)[:, -2],
        top_i=top_i,
        seed=np.int32(SEED),
    )
    print(f"wrote {out}: ids {ids.shape[1]}, logits rows {len(KEEP_ROWS)}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
