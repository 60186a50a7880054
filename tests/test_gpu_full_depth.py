"""Full-depth parity of the decode path on the 26B-A4B-shaped model.

The whole 30-layer model (seed 3; 25 sliding layers and 5 full k==v layers
at 5, 11, 17, 23, 29; 47 GiB of bf16 weights) runs through the Engine API on
a 32,768-position cache: the batched prefill, then greedy decode_fn steps,
each a replay of one captured HIP graph (engine.py:57-93; the layer loop of
model.py:365-371).  Two prompts:

  * 54 tokens (the decode benchmark's prompt): 4 decode steps at positions
    54-57 through the graph whose full layers are sized for 1,024 positions
    (182 kernels per token: one attention launch on every layer);
  * 8,190 tokens: 4 decode steps at positions 8,190-8,193, from the graph
    sized for 8,192 positions (187 kernels per token) into the one sized for
    the whole cache at 8,192 (192 kernels per token: the long-range
    attention kernels and their split reduction).

For each prompt the oracle takes the GPU's K/V rows of positions 0..P-2,
then runs the prompt's last token and the GPU's tokens itself (torch-CPU,
bf16 GEMMs with f32 accumulation: oracle/twin.py with precise=False, as in
the benchmark's CPU leg), teacher-forced.  Every step: logits corr >= 0.9999
and max |d| <= LOGIT_TOL, and the GPU token is the oracle's greedy choice or
within TIE of it (a flip needs the oracle's top-two gap <= 2 max |d|); the
teacher-forced agreement count is printed and asserted.
"""

import os

import numpy as np
import pytest
import torch

from gemma4_mi import model as gm
from gemma4_mi.config import gemma4_26b_a4b_config
from gemma4_mi.engine import Engine
from gemma4_mi.weights import init_random_params
from oracle import twin

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
MAX_LEN = 32768
N_DEC = 4
LOGIT_TOL = 1e-3  # measured 26B-shaped decode error ~5e-4: one bf16 ulp of the largest logits
TIE = LOGIT_TOL   # an excused flip needs the oracle's top-two gap within this


@pytest.fixture(scope="module")
def full26():
    cfg = gemma4_26b_a4b_config()
    params = init_random_params(cfg, 3, device=DEV)
    torch.cuda.synchronize()
    eng = Engine(None, MAX_LEN, 1, cfg=cfg, params=params, device=DEV)
    torch.set_num_threads(max(1, len(os.sched_getaffinity(0))))
    cpu = {k: v.cpu() for k, v in params.items()}
    yield cfg, eng, cpu
    del eng, params
    torch.cuda.empty_cache()


def _gpu_steps(eng, prompt):
    """prefill_fn on the prompt, then N_DEC greedy decode_fn steps; the token
    and the f32 logits of every step (the prefill head's first)."""
    p = len(prompt)
    bucket = -(-p // 256) * 256
    eng.reset_cache()
    toks = torch.zeros((1, bucket), dtype=torch.int32)
    toks[0, :p] = torch.tensor(prompt, dtype=torch.int32)
    tok, cache, pos = eng.prefill_fn(bucket)(eng.params, toks, eng.cache, p, 0, 0.0, 1.0)
    gen, rows = [int(tok.item())], [eng._runner.logits.cpu().clone()]
    dec = eng.decode_fn()
    for _ in range(N_DEC):
        tok, cache, pos = dec(eng.params, tok, cache, pos, 0, 0.0, 1.0)
        gen.append(int(tok.item()))
        rows.append(eng._runner.logits.cpu().clone())
    assert int(pos) == p + N_DEC
    return gen, torch.stack(rows).numpy()


def _oracle_steps(cfg, cpu, eng, prompt, gen):
    """The oracle from the GPU's cache rows 0..P-2: positions P-1 (the prompt's
    last token) to P-1+N_DEC (the GPU's tokens), over the whole cache as the
    reference's decode attends it (engine.py:78)."""
    p = len(prompt)
    oc = {"k": [], "v": []}
    for i in range(cfg.num_hidden_layers):
        k, v = gm.cache_positions(eng.cache, i, upto=p - 1)
        kk = torch.zeros((1, MAX_LEN) + tuple(k.shape[1:]), dtype=torch.bfloat16)
        vv = torch.zeros_like(kk)
        kk[0, :p - 1] = k.cpu()
        vv[0, :p - 1] = v.cpu()
        oc["k"].append(kk)
        oc["v"].append(vv)
    rows = []
    for s, t in enumerate([prompt[-1]] + gen[:N_DEC]):
        pos = p - 1 + s
        lg, oc = twin.forward(cfg, cpu, np.array([[t]]), np.array([pos]), oc, pos,
                              twin.decode_masks(cfg, MAX_LEN, pos), MAX_LEN, False, None, precise=False,
                              inplace=True)
        rows.append(lg[0, 0])
    return torch.stack(rows).numpy()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("plen", [54, 8190])
def test_full_depth_decode_matches_oracle(full26, plen):
    cfg, eng, cpu = full26
    prompt = np.random.default_rng(3 if plen == 54 else 13).integers(0, cfg.vocab_size, size=plen).tolist()
    gen, got = _gpu_steps(eng, prompt)
    exp = _oracle_steps(cfg, cpu, eng, prompt, gen)
    agree, near = 0, 0
    for s, t in enumerate(gen):
        err = float(np.abs(got[s] - exp[s]).max())
        corr = float(np.corrcoef(got[s], exp[s])[0, 1])
        best = int(np.argmax(exp[s]))
        top2 = np.sort(exp[s])[-2:]
        gap = float(top2[1] - top2[0])
        near += gap <= TIE
        print(f"prompt {plen}, position {plen - 1 + s}: token {t} oracle {best} max|d| {err:.3e} "
              f"corr {corr:.7f} oracle top-2 gap {gap:.3e}")
        assert corr >= 0.9999 and err <= LOGIT_TOL, (s, err, corr)
        assert t == int(np.argmax(got[s]))  # the head's token is the argmax of its own logits
        if t == best:
            agree += 1
        else:
            assert exp[s][best] - exp[s][t] <= TIE, f"position {plen - 1 + s}: not a near tie"
    print(f"prompt {plen}: teacher-forced agreement {agree}/{len(gen)} ({near} oracle near ties)")
    assert agree >= len(gen) - near
