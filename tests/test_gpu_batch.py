"""GPU: batched decode of several sequences at their own positions
(gemma4_mi.batch) on the tiny parity model.

Three prompts of 40, 77 and 128 tokens (rng 0, 1, 2) share one page pool; a
fourth row repeats the last prompt.  Each sequence is prefilled into its own
pages, then all advance together for 12 greedy tokens.  Each sequence's
tokens are checked against the oracle run on that prompt alone, teacher
forced on the GPU's tokens (oracle.twin.prefill_then_decode): every token is
the oracle's greedy choice or a declared near tie (top-two oracle logits
within 2.5e-4; the batched path's GEMMs accumulate in another order than the
single-sequence GEMVs and the oracle's f64).
"""

import numpy as np
import pytest
import torch

from gemma4_mi.batch import BatchEngine
from gemma4_mi.config import tiny_parity_config
from gemma4_mi.weights import init_random_params
from greedy_check import check_stream
from oracle import twin

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_batched_decode_matches_single_sequence_oracle():
    cfg = tiny_parity_config()
    params = init_random_params(cfg, 0, device=DEV)
    params_cpu = twin.random_params(cfg, 0)
    lens = (40, 77, 128)
    prompts = [np.random.default_rng(i).integers(0, cfg.vocab_size, size=n).tolist() for i, n in enumerate(lens)]
    eng = BatchEngine(cfg, params, batch=4, max_len=256, device=DEV)
    got = eng.generate(prompts, 12)
    used = sum(len(o) for o in eng.pool.owned)
    assert used == sum((n + 12 + 63) // 64 for n in list(lens) + [lens[-1]])
    for b, pr in enumerate(prompts):
        print(f"sequence {b} ({len(pr)} tokens): gpu {got[b][:6]}")
        check_stream(cfg, params_cpu, pr, got[b], 256, what=f"sequence {b}")


def test_batched_decode_above_eight_rows_uses_grouped_experts():
    """Ten rows (the grouped expert path, each selected expert read once per
    step): rows holding the same prompt produce the same tokens, and each
    distinct prompt's tokens follow the single-sequence oracle (greedy
    choices or declared near ties)."""
    cfg = tiny_parity_config()
    params = init_random_params(cfg, 0, device=DEV)
    params_cpu = twin.random_params(cfg, 0)
    base = [np.random.default_rng(20 + i).integers(0, cfg.vocab_size, size=n).tolist()
            for i, n in enumerate((33, 64, 95))]
    prompts = [base[i % 3] for i in range(10)]
    eng = BatchEngine(cfg, params, batch=10, max_len=192, device=DEV)
    assert eng.runner.grouped_moe
    got = eng.generate(prompts, 10)
    for b in range(10):
        assert got[b] == got[b % 3], b
    for i, pr in enumerate(base):
        check_stream(cfg, params_cpu, pr, got[i], 192, what=f"prompt {i}")


def test_batched_rows_are_independent():
    """Row b's tokens do not depend on what the other rows hold: a batch of
    [A, B, A] yields the same stream for both A rows."""
    cfg = tiny_parity_config()
    params = init_random_params(cfg, 0, device=DEV)
    a = np.random.default_rng(5).integers(0, cfg.vocab_size, size=50).tolist()
    b = np.random.default_rng(6).integers(0, cfg.vocab_size, size=90).tolist()
    eng = BatchEngine(cfg, params, batch=3, max_len=192, device=DEV)
    got = eng.generate([a, b, a], 10)
    assert got[0] == got[2]
    torch.cuda.synchronize()


def test_argmax_rows_softcap_ties_and_history():
    """The batched greedy head: softcap 30 in f32, the first index of the
    maximum per row (an exact tie goes to the lower index), pos += 1 and the
    token recorded in that row's history."""
    from gemma4_mi import ops

    rng = np.random.default_rng(7)
    B, V = 5, 70001
    lg = torch.tensor(rng.standard_normal((B, V)) * 8.0, dtype=torch.bfloat16)
    lg[1, 100] = lg[1, 60000] = 120.0  # tie after the softcap
    lg[3, 69999] = 200.0
    d = lg.to(DEV)
    tok = torch.zeros(B, dtype=torch.int32, device=DEV)
    pos = torch.arange(B, dtype=torch.int32, device=DEV) * 3
    hist = torch.zeros((B, 32), dtype=torch.int32, device=DEV)
    f32 = torch.empty((B, V), dtype=torch.float32, device=DEV)
    ops.argmax_rows(d, 30.0, tok, pos, hist, logits_f32=f32)
    torch.cuda.synchronize()
    v = torch.tanh(lg.float() / 30.0) * 30.0
    exp = [int(np.argmax(v[b].numpy())) for b in range(B)]  # numpy argmax: first maximal index
    assert tok.cpu().tolist() == exp and exp[1] == 100 and exp[3] == 69999
    assert pos.cpu().tolist() == [3 * b + 1 for b in range(B)]
    assert [int(hist[b, 3 * b + 1]) for b in range(B)] == exp
    assert torch.allclose(f32.cpu(), v, rtol=0, atol=2e-6)
