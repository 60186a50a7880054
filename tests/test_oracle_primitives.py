"""CPU: the oracle's primitives and blocks (oracle/twin.py) against closed
forms, HF transformers sub-modules, brute force and invariants.

Each check is chosen so that a plausible slip in the restatement fails it: a
`1 + w` RMSNorm weight, a missing 1/H, a wrong RoPE half, a scaled or
uncapped score, a wrong GQA head map, a window off by one, a router tie
broken the wrong way, the routing weight applied after `down` instead of
before, a dense/sparse combine mismatch.
"""

import math

import numpy as np
import pytest
import torch

from gemma4_mi.config import tiny_parity_config
from oracle import twin

BF = torch.bfloat16


def _bf(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(BF)


def _ulps(a, b):
    """Distance in bf16 units of the larger magnitude."""
    a, b = a.float(), b.float()
    scale = torch.maximum(a.abs(), b.abs()).clamp_min(1e-30)
    return ((a - b).abs() / (scale * 2.0 ** -8)).max().item()


# ----------------------------------------------------------------- rms_norm
def test_rms_norm_closed_form_f64():
    x = _bf((5, 256), 1, 3.0)
    w = _bf((256,), 2, 0.5)
    got = twin.rms_norm(x, w, 1e-6).double()
    xd = x.double()
    exp = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert _ulps(got, exp) <= 1.0  # one bf16 rounding of the f64 value
    # no weight: unit root-mean-square
    y = twin.rms_norm(x, None, 1e-6).double()
    assert torch.allclose((y * y).mean(-1), torch.ones(5, dtype=torch.float64), rtol=2e-2)


def test_rms_norm_matches_hf_gemma4():
    from transformers.models.gemma4.modeling_gemma4 import Gemma4RMSNorm

    x = _bf((7, 2816), 3, 2.0)
    w = _bf((2816,), 4, 0.3)
    hf = Gemma4RMSNorm(2816, eps=1e-6)
    with torch.no_grad():
        hf.weight.copy_(w.float())
        ref = hf(x)
    got = twin.rms_norm(x, w, 1e-6)
    assert _ulps(got, ref) <= 1.0
    assert (got == ref).float().mean().item() >= 0.99


# ----------------------------------------------------------------- gelu
def test_gelu_matches_torch_tanh_approximation():
    x = torch.linspace(-8, 8, 20001).to(BF)
    exp = torch.nn.functional.gelu(x.double(), approximate="tanh")
    got = twin.gelu(x).double()
    # one bf16 rounding, plus the f32 cancellation of 1 + tanh(.) for x << 0
    assert torch.all((got - exp).abs() <= 2.0 ** -8 * exp.abs() + 4.0 * 2.0 ** -24 * x.double().abs())
    assert twin.gelu(torch.zeros(1, dtype=BF)).item() == 0.0


# ----------------------------------------------------------------- rope
def test_rope_inv_freq_known_answers():
    inv = twin.rope_inv_freq(256, 1e4)
    assert inv.dtype == np.float32 and inv.shape == (128,)
    assert inv[0] == 1.0
    assert abs(float(inv[1]) - 0.9305720409) < 1e-7  # 1e4^(-2/256)
    assert abs(float(inv[127]) - 1.0e-4 ** (254 / 256)) < 1e-10
    prop = twin.rope_inv_freq(512, 1e6, 0.25)  # proportional: 64 rotated, 192 NoPE
    assert prop.shape == (256,)
    assert np.count_nonzero(prop) == 64 and np.all(prop[64:] == 0) and prop[0] == 1.0
    assert abs(float(prop[63]) - 1e6 ** (-126 / 512)) < 1e-9


def test_rope_is_the_complex_rotation():
    d = 64
    x = _bf((1, 3, 2, d), 5)
    inv = twin.rope_inv_freq(d, 1e4)
    pos = [0, 17, 4000]
    cos, sin = twin.rope_tables(pos, inv)
    got = twin.apply_rope(x, cos, sin).double()
    # (x1 + i x2) * exp(i * pos * f) per frequency, with bf16 cos/sin as the reference casts them
    c = cos.to(BF).double()[None, :, None, : d // 2]
    s = sin.to(BF).double()[None, :, None, : d // 2]
    x1, x2 = x.double()[..., : d // 2], x.double()[..., d // 2:]
    exp = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1)
    assert (got - exp).abs().max().item() <= 3 * 2.0 ** -8 * x.double().abs().max().item()
    # position 0 is the identity
    assert torch.equal(got[:, 0], x.double()[:, 0])


def test_rope_tables_angles():
    inv = twin.rope_inv_freq(512, 1e6, 0.25)
    cos, sin = twin.rope_tables([12345], inv)
    ang = np.float32(12345) * inv
    assert np.allclose(cos[0, :256].numpy(), np.cos(ang.astype(np.float64)), atol=1e-7)
    assert np.array_equal(cos[0, :256].numpy(), cos[0, 256:].numpy())
    assert np.all(cos[0, 64:256].numpy() == 1.0) and np.all(sin[0, 64:256].numpy() == 0.0)


# ----------------------------------------------------------------- attention
def _brute_attention(q, kk, vv, lo, hi, softcap):
    """Textbook softmax(q . k) v over positions [lo, hi], scale 1, GQA j -> j // G,
    in f64 without intermediate rounding.  q [KV,G,D], kk/vv [S,KV,D]."""
    kv, g, _ = q.shape
    out = torch.zeros(q.shape, dtype=torch.float64)
    for h in range(kv * g):
        kvh, gi = h // g, h % g
        s = torch.stack([q[kvh, gi].double() @ kk[p, kvh].double() for p in range(lo, hi + 1)])
        if softcap:
            s = torch.tanh(s / softcap) * softcap
        p_ = torch.softmax(s, 0)
        out[kvh, gi] = (p_[:, None] * vv[lo:hi + 1, kvh].double()).sum(0)
    return out


@pytest.mark.parametrize("window,softcap", [(0, None), (8, None), (0, 50.0), (8, 20.0)])
def test_attention_core_against_brute_force(window, softcap):
    kv, g, d, lmax, pos = 2, 2, 16, 24, 19
    q = _bf((1, 1, kv, g, d), 10)
    k_raw = _bf((1, 1, kv, d), 11)
    v_raw = _bf((1, 1, kv, d), 12)
    qn, kn = _bf((d,), 13, 0.5), _bf((d,), 14, 0.5)
    ck, cv = _bf((1, lmax, kv, d), 15), _bf((1, lmax, kv, d), 16)
    cos, sin = twin.rope_tables([pos], twin.rope_inv_freq(d, 1e4))

    class C:
        sliding_window = window if window else 10**9

    mk = twin.decode_masks(C, lmax, pos)
    mask = mk[twin.SLIDING] if window else mk[twin.FULL]
    ctx, nk, nv = twin.attention_core(q, k_raw, v_raw, qn, kn, cos, sin, ck, cv, pos, mask, lmax, 1e-6, softcap)
    # the new K/V row: normalised (K with k_norm and RoPE), the rest untouched
    assert torch.equal(nk[0, pos], twin.apply_rope(twin.rms_norm(k_raw, kn, 1e-6), cos, sin)[0, 0])
    assert torch.equal(nv[0, pos], twin.rms_norm(v_raw, None, 1e-6)[0, 0])
    keep = [p for p in range(lmax) if p != pos]
    assert torch.equal(nk[0, keep], ck[0, keep]) and torch.equal(nv[0, keep], cv[0, keep])
    qr = twin.apply_rope(twin.rms_norm(q, qn, 1e-6), cos, sin)[0, 0]
    lo = max(0, pos + 1 - window) if window else 0
    exp = _brute_attention(qr, nk[0], nv[0], lo, pos, softcap)
    # scores, probabilities and ctx are each rounded to bf16 in the reference
    err = (ctx[0, 0].double() - exp).abs().max().item()
    assert err <= 2.0 ** -6 * exp.abs().max().item(), err


def test_sliding_window_covering_everything_equals_full():
    cfg = tiny_parity_config()
    kv, g, d, lmax, pos = 2, 2, 64, 40, 30
    args = (_bf((1, 1, kv, g, d), 20), _bf((1, 1, kv, d), 21), _bf((1, 1, kv, d), 22), _bf((d,), 23),
            _bf((d,), 24))
    cos, sin = twin.rope_tables([pos], twin.rope_inv_freq(d, 1e4))
    ck, cv = _bf((1, lmax, kv, d), 25), _bf((1, lmax, kv, d), 26)
    wide = cfg.replace(sliding_window=pos + 1)
    m_s = twin.decode_masks(wide, lmax, pos)[twin.SLIDING]
    m_f = twin.decode_masks(wide, lmax, pos)[twin.FULL]
    a = twin.attention_core(*args, cos, sin, ck, cv, pos, m_s, lmax, 1e-6)[0]
    b = twin.attention_core(*args, cos, sin, ck, cv, pos, m_f, lmax, 1e-6)[0]
    assert torch.equal(a, b)
    narrow = cfg.replace(sliding_window=pos)  # one position fewer: must differ
    m_n = twin.decode_masks(narrow, lmax, pos)[twin.SLIDING]
    assert int(m_n.sum()) == pos and int(m_f.sum()) == pos + 1


def test_masks_closed_form():
    cfg = tiny_parity_config().replace(sliding_window=4)
    pm = twin.prefill_masks(cfg, 8, 6)
    for q in range(8):
        for kv in range(8):
            assert bool(pm[twin.FULL][0, 0, 0, q, kv]) == (kv <= q and kv < 6)
            assert bool(pm[twin.SLIDING][0, 0, 0, q, kv]) == (kv <= q and kv < 6 and kv > q - 4)
    dm = twin.decode_masks(cfg, 8, 5)
    assert dm[twin.FULL][0, 0, 0, 0].tolist() == [True] * 6 + [False] * 2
    assert dm[twin.SLIDING][0, 0, 0, 0].tolist() == [False, False, True, True, True, True, False, False]


def test_decode_row_equals_prefill_row():
    """The logits of position p from a T-token prefill equal a decode step at p
    after a prefill of p tokens (the causal mask is the only difference)."""
    cfg = tiny_parity_config()
    params = twin.random_params(cfg, 0)
    toks = np.random.default_rng(1).integers(0, cfg.vocab_size, size=(1, 12))
    t = 12
    full, _ = twin.forward(cfg, params, toks, np.arange(t), twin.init_cache(cfg, 1, t), 0,
                           twin.prefill_masks(cfg, t, t), t, False)
    cache = twin.init_cache(cfg, 1, 32)
    _, cache = twin.forward(cfg, params, toks[:, : t - 1], np.arange(t - 1), cache, 0,
                            twin.prefill_masks(cfg, t - 1, t - 1), t - 1, False)
    dec, _ = twin.forward(cfg, params, toks[:, t - 1:], np.array([t - 1]), cache, t - 1,
                          twin.decode_masks(cfg, 32, t - 1), 32, False)
    assert torch.equal(full[0, t - 1], dec[0, 0])


# ----------------------------------------------------------------- router / MoE
def _router_inputs(n, seed):
    cfg = tiny_parity_config()
    params = twin.random_params(cfg, seed)
    lp = twin.layer_params(params, 0)
    flat = _bf((n, cfg.hidden_size), seed + 100)
    return cfg, lp, flat


def test_router_against_brute_force():
    cfg, lp, flat = _router_inputs(64, 1)
    # unit-scale router weights so that the probabilities are well separated
    lp = dict(lp, **{"router.scale": torch.ones(cfg.hidden_size, dtype=BF),
                     "router.proj": _bf((cfg.num_experts, cfg.hidden_size), 7)})
    top_w, top_i = twin.router(cfg, lp, flat)
    checked = 0
    h = cfg.hidden_size
    for n in range(flat.shape[0]):
        x = flat[n].double()
        x = x / math.sqrt(float((x * x).mean()) + cfg.rms_norm_eps)
        x = x * lp["router.scale"].double() * h ** -0.5
        s = (lp["router.proj"].double() @ x)
        p = torch.softmax(s, 0)
        order = sorted(range(cfg.num_experts), key=lambda e: (-float(p[e]), e))[: cfg.top_k_experts]
        # the reference rounds x and the scores to bf16, so compare where the
        # brute-force probabilities are separated by more than that rounding
        sp = sorted(p.tolist(), reverse=True)
        if sp[cfg.top_k_experts - 1] - sp[cfg.top_k_experts] > 0.02 * sp[0]:
            assert set(top_i[n].tolist()) == set(order)
            checked += 1
        # within the top k, order follows the brute-force probabilities where
        # neighbours are separated by more than the bf16 score rounding
        for a, b in zip(top_i[n][:-1].tolist(), top_i[n][1:].tolist()):
            if abs(float(p[a]) - float(p[b])) > 0.02 * sp[0]:
                assert float(p[a]) > float(p[b])
        w = p[top_i[n]] / p[top_i[n]].sum() * lp["router.per_expert_scale"].double()[top_i[n]]
        assert torch.allclose(top_w[n].double(), w, rtol=0.05, atol=1e-6)
    assert checked >= 32


def test_router_ties_go_to_lower_index():
    cfg, lp, flat = _router_inputs(1, 2)
    lp = dict(lp)
    lp["router.proj"] = torch.zeros_like(lp["router.proj"])  # all scores equal
    lp["router.per_expert_scale"] = torch.ones_like(lp["router.per_expert_scale"])
    top_w, top_i = twin.router(cfg, lp, flat)
    assert top_i[0].tolist() == list(range(cfg.top_k_experts))
    assert torch.allclose(top_w, torch.full_like(top_w, 1.0 / cfg.top_k_experts))


def test_sparse_moe_matches_dense_moe():
    """The reference's invariant (tests/test_parity.py:127-151): the top-k slice
    decode path and the dense all-experts path agree."""
    cfg, lp, flat = _router_inputs(6, 3)
    sp, w1, i1 = twin.moe(cfg, lp, flat, dense=False, return_route=True)
    de, w2, i2 = twin.moe(cfg, lp, flat, dense=True, return_route=True)
    assert torch.equal(i1, i2) and torch.equal(w1, w2)
    a, b = sp.double().ravel(), de.double().ravel()
    assert np.corrcoef(a.numpy(), b.numpy())[0, 1] >= 0.9999
    # bf16 running sum of k terms vs one f32 contraction: a few ulps of the output scale
    assert (a - b).abs().max().item() <= 4 * 2.0 ** -8 * b.abs().max().item()


def test_dense_moe_on_selected_experts_equals_all_experts():
    """The dense-MoE contraction restricted to the selected (token, expert)
    pairs (moe_dense_selected, what the 26B-shaped parity tests run) equals
    the all-experts contraction of model.py:241-250 bit for bit: the masked
    experts add exact zeros, and only the f64 summation order differs before
    the single rounding.  Also at 64 tokens with routing ties."""
    for n_tok, seed in ((6, 3), (64, 8)):
        cfg, lp, flat = _router_inputs(n_tok, seed)
        full, w1, i1 = twin.moe(cfg, lp, flat, dense=True, return_route=True)
        sel, w2, i2 = twin.moe(cfg, lp, flat, dense="selected", return_route=True)
        assert torch.equal(i1, i2) and torch.equal(w1, w2)
        assert torch.equal(full.view(torch.int16), sel.view(torch.int16))
    with pytest.raises(ValueError):
        twin.moe(cfg, lp, flat, dense="all")


def test_teacher_forced_decode_feeds_the_given_tokens():
    """prefill_then_decode with `forced` feeds the given tokens; fed the
    oracle's own greedy stream it reproduces the free-running logits, and
    all_logits=False returns the last prompt row only."""
    cfg = tiny_parity_config()
    params = twin.random_params(cfg, 0)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab_size, size=12)
    lg, gen = twin.prefill_then_decode(cfg, params, prompt, 3, 32)
    lg2, gen2 = twin.prefill_then_decode(cfg, params, prompt, 3, 32, all_logits=False, prefill_dense="selected",
                                         forced=gen)
    assert lg.shape[0] == 12 + 3 and lg2.shape[0] == 1 + 3
    assert torch.equal(lg[11:], lg2) and gen2 == gen
    other = [(t + 1) % cfg.vocab_size for t in gen]
    lg3, _ = twin.prefill_then_decode(cfg, params, prompt, 3, 32, all_logits=False, forced=other)
    assert torch.equal(lg3[0], lg2[0]) and not torch.equal(lg3[1], lg2[1])


def test_moe_against_brute_force_selected_experts():
    """Routing weight applied before down (model.py:271), f64 brute force over
    the selected experts only."""
    cfg, lp, flat = _router_inputs(3, 4)
    out, top_w, top_i = twin.moe(cfg, lp, flat, dense=False, return_route=True)
    for n in range(flat.shape[0]):
        acc = torch.zeros(cfg.hidden_size, dtype=torch.float64)
        for k in range(cfg.top_k_experts):
            e = int(top_i[n, k])
            gu = lp["experts.gate_up_proj"][e].double() @ flat[n].double()  # [2, F]
            g, u = gu[0], gu[1]
            act = 0.5 * g * (1 + torch.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3))) * u * float(top_w[n, k])
            acc += lp["experts.down_proj"][e].double() @ act
        err = (out[n].double() - acc).abs().max().item()
        assert err <= 2.0 ** -5 * acc.abs().max().item(), err


# ----------------------------------------------------------------- head
def test_lm_head_softcap_bound_and_greedy_first_index():
    cfg = tiny_parity_config()
    params = twin.random_params(cfg, 0)
    params = dict(params)
    params["norm"] = torch.full_like(params["norm"], 40.0)  # push logits into the cap
    lg, _ = twin.forward(cfg, params, np.array([[5, 6]]), np.arange(2), twin.init_cache(cfg, 1, 2), 0,
                         twin.prefill_masks(cfg, 2, 2), 2, False)
    assert lg.dtype == torch.float32 and lg.abs().max().item() < 30.0
    assert lg.abs().max().item() > 10.0
    assert twin.greedy(torch.tensor([1.0, 3.0, 3.0, 2.0])) == 1
    assert twin.greedy(torch.tensor([-1.0, -1.0])) == 0
