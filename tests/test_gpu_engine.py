"""GPU: the Engine API (engine.py:26-221) and the device sampler
(model.py:414-424) on the tiny parity model.

* generate() at temperature 0 yields the oracle's greedy tokens (prefill
  event first, then decode events with the reference's fields), through the
  captured feed/head/decode graphs with lookahead 3;
* prompts of 1, 37, 256 and 300 tokens (one and two prefill buckets) give
  the oracle's greedy tokens, or declared near ties, teacher-forced;
* prefill_fn / decode_fn keep the reference's calling convention
  ((tok [1,1], cache, pos) returns, cache updated in place);
* stop ids end the stream; a prompt that fills the context raises ValueError;
* sampling: greedy at temperature <= 0, top_k = 1 or a tiny top_p;
  ties go to the lower index; and the empirical distribution of 6000 draws
  matches the top-k / nucleus distribution computed in numpy (chi-square,
  p > 1e-4).  The draws are this library's Philox stream, not JAX's, so
  only the distribution is pinned (parity unpinned bit for bit).
"""

import numpy as np
import pytest
import torch
from scipy import stats

from gemma4_mi import ops
from gemma4_mi.config import tiny_parity_config
from gemma4_mi.engine import Engine
from greedy_check import check_stream
from oracle import twin

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
P, N_DEC, MAX_LEN = 128, 32, 256


@pytest.fixture(scope="module")
def setup():
    cfg = tiny_parity_config()
    eng = Engine.random(cfg, seed=0, max_len=MAX_LEN, top_k=64, device=DEV)
    prompt = np.random.default_rng(0).integers(0, cfg.vocab_size, size=P).astype(np.int64)
    _, gen_o = twin.prefill_then_decode(cfg, twin.random_params(cfg, 0), prompt, N_DEC, MAX_LEN)
    return cfg, eng, prompt, gen_o


def test_generate_greedy_matches_oracle(setup):
    cfg, eng, prompt, gen_o = setup
    events = list(eng.generate(prompt.tolist(), max_new_tokens=N_DEC + 1, temperature=0.0, stop_ids=()))
    assert events[0]["kind"] == "prefill" and events[0]["prompt_tokens"] == P
    assert events[0]["prefill_bucket"] == 256 and events[0]["ttft"] > 0
    assert [e["kind"] for e in events[1:]] == ["decode"] * N_DEC
    assert [e["index"] for e in events[1:]] == list(range(1, N_DEC + 1))
    assert events[-1]["total_tokens"] == N_DEC + 1
    toks = [e["token"] for e in events]
    print("engine", toks[:8], "oracle", gen_o[:8])
    assert toks == list(gen_o[: N_DEC + 1])


def test_stepwise_prefill_engine_matches_oracle(setup):
    """prefill="stepwise" (the prompt fed one position at a time through the
    decode kernels, "feed" then "head" graphs) gives the same greedy tokens."""
    cfg, eng, prompt, gen_o = setup
    eng2 = Engine(None, MAX_LEN, 1, 64, cfg=cfg, params=eng.params, device=DEV, prefill="stepwise")
    toks = [e["token"] for e in eng2.generate(prompt.tolist(), max_new_tokens=9, temperature=0.0, stop_ids=())]
    assert toks == list(gen_o[:9])


@pytest.mark.parametrize("plen", [1, 37, 256, 300])
def test_prompt_lengths_across_prefill_buckets(setup, plen):
    """Prompts of 1, 37, 256 (one whole bucket) and 300 tokens (two buckets)
    through the batched prefill, then 5 greedy decode steps: the bucket is the
    reference's (multiples of 256), and every token is the oracle's greedy
    choice given the same history, or a declared near tie."""
    cfg, eng, _, _ = setup
    max_len = 640
    eng2 = Engine(None, max_len, 1, 64, cfg=cfg, params=eng.params, device=DEV)
    prompt = np.random.default_rng(100 + plen).integers(0, cfg.vocab_size, size=plen).astype(np.int64)
    events = list(eng2.generate(prompt.tolist(), max_new_tokens=6, temperature=0.0, stop_ids=()))
    assert events[0]["prompt_tokens"] == plen and events[0]["prefill_bucket"] == max(256, -(-plen // 256) * 256)
    gen = [e["token"] for e in events]
    assert len(gen) == 6
    check_stream(cfg, twin.random_params(cfg, 0), prompt, gen, max_len, what=f"prompt of {plen}")


@pytest.mark.parametrize("mode", ["batched", "stepwise"])
def test_prompt_in_the_last_page_on_a_fresh_engine(setup, mode):
    """A prompt of max_len - 10 tokens on a fresh Engine: its decode (and, when
    stepwise, head) graphs are first captured while the prompt's K/V rows sit
    in the cache's last page, and the capture's warm step (run at the scratch
    position max_len - 1) must leave those rows intact.  The tokens equal
    those of an engine whose graphs were captured on a short prompt, and
    every one is the teacher-forced oracle's greedy choice."""
    cfg, eng, _, _ = setup
    plen = MAX_LEN - 10
    prompt = np.random.default_rng(7).integers(0, cfg.vocab_size, size=plen).astype(np.int64)
    warm = Engine(None, MAX_LEN, 1, 64, cfg=cfg, params=eng.params, device=DEV, prefill=mode)
    list(warm.generate([1, 2, 3], max_new_tokens=3, temperature=0.0, stop_ids=()))
    want = [e["token"] for e in warm.generate(prompt.tolist(), max_new_tokens=9, temperature=0.0, stop_ids=())]
    fresh = Engine(None, MAX_LEN, 1, 64, cfg=cfg, params=eng.params, device=DEV, prefill=mode)
    got = [e["token"] for e in fresh.generate(prompt.tolist(), max_new_tokens=9, temperature=0.0, stop_ids=())]
    print(f"{mode}: fresh {got} warmed {want}")
    assert got == want
    check_stream(cfg, twin.random_params(cfg, 0), prompt, got, MAX_LEN, what=f"{mode} prompt of {plen}")


def test_step_functions_calling_convention(setup):
    cfg, eng, prompt, gen_o = setup
    eng.reset_cache()
    toks = torch.zeros((1, 256), dtype=torch.int32)
    toks[0, :P] = torch.as_tensor(prompt)
    tok, cache, pos = eng.prefill_fn(256)(eng.params, toks, eng.cache, P, 0, 0.0, 1.0)
    assert cache is eng.cache and tuple(tok.shape) == (1, 1) and int(pos) == P
    got = [int(tok.item())]
    dec = eng.decode_fn()
    for _ in range(4):
        tok, cache, pos = dec(eng.params, tok, cache, pos, 0, 0.0, 1.0)
        got.append(int(tok.item()))
    assert int(pos) == P + 4
    assert got == list(gen_o[:5])
    # a host-supplied token at an explicit position (teacher forcing) is accepted
    tok2, _, pos2 = dec(eng.params, torch.tensor([[gen_o[5]]], dtype=torch.int32), cache, P + 5, 0, 0.0, 1.0)
    assert int(pos2) == P + 6 and int(tok2.item()) == gen_o[6]


def test_stop_ids_and_limits(setup):
    cfg, eng, prompt, gen_o = setup
    stop = gen_o[3]
    first = next(i for i, t in enumerate(gen_o) if t == stop)
    events = list(eng.generate(prompt.tolist(), max_new_tokens=20, temperature=0.0, stop_ids=(stop,)))
    assert [e["token"] for e in events] == list(gen_o[: first + 1])
    with pytest.raises(ValueError):
        list(eng.generate(list(range(MAX_LEN)), max_new_tokens=4, temperature=0.0))


def test_compile_all_reports_times(setup):
    cfg, eng, prompt, gen_o = setup
    out = eng.compile_all(bucket=256)
    assert set(out) == {"prefill_compile_s", "decode_compile_s", "decode_step_s"}
    assert 0 < out["decode_step_s"] < 1.0 and eng.decode_step_seconds == out["decode_step_s"]
    assert eng.n_devices == 1 and eng.param_bytes > 0 and eng.cache_bytes > 0


def test_sampled_generation_is_seeded(setup):
    cfg, eng, prompt, gen_o = setup
    a = [e["token"] for e in eng.generate(prompt.tolist(), max_new_tokens=12, temperature=1.0, top_p=0.95,
                                          seed=7, stop_ids=())]
    b = [e["token"] for e in eng.generate(prompt.tolist(), max_new_tokens=12, temperature=1.0, top_p=0.95,
                                          seed=7, stop_ids=())]
    c = [e["token"] for e in eng.generate(prompt.tolist(), max_new_tokens=12, temperature=1.0, top_p=0.95,
                                          seed=8, stop_ids=())]
    assert a == b and len(a) == 12
    assert a != c


# ----------------------------------------------------------------- the sampler kernel
def _expected(logits, t, top_k, top_p):
    v = (logits / np.float32(max(t, 1e-6))).astype(np.float32)
    order = sorted(range(len(v)), key=lambda i: (-float(v[i]), i))[:top_k]
    vals = v[order].astype(np.float64)
    p = np.exp(vals - vals.max())
    p /= p.sum()
    keep = (np.cumsum(p) - p) < top_p
    q = np.where(keep, p, 0.0)
    return np.array(order), q / q.sum()


def _draws(logits_np, t, top_p, top_k, n, seed=11):
    logits = torch.tensor(logits_np, dtype=torch.float32, device=DEV)
    prm = ops.sample_params(t, top_p, seed, DEV)
    tok = torch.zeros(1, dtype=torch.int32, device=DEV)
    pos = torch.zeros(1, dtype=torch.int32, device=DEV)
    hist = torch.zeros(n + 1, dtype=torch.int32, device=DEV)
    for _ in range(n):
        ops.sample(logits, top_k, prm, tok, 1, pos, hist)
    torch.cuda.synchronize()
    assert int(pos.item()) == n
    return hist[1:].cpu().numpy()


def test_sampler_distribution_matches_top_k_top_p():
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal(5000) * 2.0).astype(np.float32)
    for t, top_p, top_k in ((1.0, 0.9, 64), (0.7, 1.0, 16)):
        idx, q = _expected(logits, t, top_k, top_p)
        d = _draws(logits, t, top_p, top_k, 6000)
        assert set(np.unique(d)) <= set(idx[q > 0].tolist())
        counts = np.array([(d == i).sum() for i in idx])
        exp = q * len(d)
        big = exp >= 5
        obs = np.append(counts[big], counts[~big].sum())
        ex = np.append(exp[big], exp[~big].sum())
        if ex[-1] == 0:
            obs, ex = obs[:-1], ex[:-1]
        pv = stats.chisquare(obs, ex).pvalue
        print(f"T={t} top_p={top_p} top_k={top_k}: {len(idx[q > 0])} kept, chi2 p={pv:.3g}")
        assert pv > 1e-4


def test_sampler_greedy_cases_and_ties():
    rng = np.random.default_rng(4)
    logits = rng.standard_normal(70000).astype(np.float32)
    logits[12345] = logits[54321] = 9.0  # exact tie: the lower index wins
    am = 12345
    assert (_draws(logits, 0.0, 0.95, 64, 3) == am).all()           # temperature <= 0
    assert (_draws(logits, -1.0, 0.95, 64, 3) == am).all()
    assert (_draws(logits, 1.0, 0.95, 1, 3) == am).all()            # top_k = 1
    assert (_draws(logits, 1.0, 1e-9, 64, 3) == am).all()           # nucleus keeps only the first
    two = _draws(logits, 1.0, 1.0, 2, 400)
    assert set(np.unique(two)) == {12345, 54321}                      # the tie pair, nothing else


@pytest.mark.parametrize("kind", ["decode_short", "decode_tiny"])
def test_decode_crosses_the_short_span_graph_boundary(kind):
    """Below SHORT_SPAN (TINY_SPAN) the engine replays a decode graph whose
    full-attention layers are sized for SHORT_SPAN (TINY_SPAN) positions;
    from there on, the max_len-sized graph.  Decoding 8 steps across the
    boundary from a context prefilled to 5 positions before it must give,
    step for step, the greedy tokens and logits of the same steps replayed
    with the max_len-sized graph only: the attention configurations differ
    only in their f32 summation order (logits within 2^-8 of their largest
    magnitude, corr >= 0.99999)."""
    from gemma4_mi.engine import SHORT_SPAN, TINY_SPAN
    cfg = tiny_parity_config()
    span = SHORT_SPAN if kind == "decode_short" else TINY_SPAN
    max_len, n0, steps = 2 * span, span - 5, 8
    eng = Engine.random(cfg, seed=1, max_len=max_len, top_k=64, device=DEV)
    r = eng._runner
    prompt = torch.as_tensor(np.random.default_rng(1).integers(0, cfg.vocab_size, size=(1, n0)), dtype=torch.int32)
    tok, cache, pos = eng.prefill_fn(n0)(eng.params, prompt, eng.cache, n0, 0, 0.0, 1.0)
    torch.cuda.synchronize()
    saved = ([t.clone() for t in cache["k"] + cache["v"]], r.tok.clone(), r.pos.clone(), r.hist.clone())

    def run(force_full):
        for t, s in zip(cache["k"] + cache["v"], saved[0]):
            t.copy_(s)
        r.tok.copy_(saved[1]); r.pos.copy_(saved[2]); r.hist.copy_(saved[3])
        eng._pos_host = n0
        dec = eng.decode_fn()
        t, p = r.hist[n0:n0 + 1].view(1, 1), torch.tensor(n0, dtype=torch.int32)
        toks, logits = [], []
        for i in range(steps):
            if force_full:
                eng._graph("decode", True).replay()
                p = torch.tensor(n0 + i + 1, dtype=torch.int32)
                eng._pos_host = n0 + i + 1
            else:
                t, cache_, p = dec(eng.params, t, cache, p, 0, 0.0, 1.0)
            torch.cuda.synchronize()
            toks.append(int(r.hist[n0 + i + 1].item()))
            logits.append(r.logits.clone())
        return toks, logits

    toks_a, log_a = run(False)
    assert (kind, True) in eng._graphs and ("decode", True) in eng._graphs
    toks_b, log_b = run(True)
    for i in range(steps):
        a, b = log_a[i].double(), log_b[i].double()
        scale = b.abs().max().item()
        err = (a - b).abs().max().item()
        corr = float(np.corrcoef(a.cpu().numpy(), b.cpu().numpy())[0, 1])
        print(f"step at position {n0 + i}: max|d|={err:.3e} scale={scale:.3e} corr={corr:.7f}")
        assert err <= scale * 2.0 ** -8 and corr >= 0.99999, f"logits differ at position {n0 + i}"
        if toks_a[i] != toks_b[i]:  # only a near-tie may flip the greedy token
            top2 = torch.topk(b, 2).values
            assert (top2[0] - top2[1]).item() <= 2 * err, f"greedy token differs at position {n0 + i}"
