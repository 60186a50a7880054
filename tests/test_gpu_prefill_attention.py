"""GPU parity of the MFMA prefill attention (g4mi_q_norm_rope +
g4mi_prefill_attention, model.py:195-215 at T > 1) against the CPU oracle's
attention_core over the same cache: query row t at position p0 + t attends
the keys [max(0, p0 + t + 1 - W), p0 + t].

Cases: a small full layer with separate V; a small sliding layer with k==v
and softcap 50 continuing a 70-position cached prefix (p0 = 70) over a
shuffled page table; the 26B sliding shape (16 q / 8 KV heads, head_dim 256)
with a 100-position window; the 26B full shape (16 q / 2 KV heads,
head_dim 512, k==v, partial RoPE 0.25) over 300 rows; 70 rows after a
16,448-position cached prefix (key pages past the 256 whose table entries a
block stages in LDS).

Tolerances: ctx (bf16) corr >= 0.9999, >= 95% of elements bit-identical,
every element within 2^-6 of the output's max magnitude.  The GPU accumulates
the dots in f32 on MFMA, the oracle in f64, so a probability that sits on a
bf16 rounding boundary can round the other way; in the first rows (few keys,
probabilities near 1/2) that moves ctx by up to |v| * 2^-9 before ctx's own
rounding, which can reach 1.5 bf16 ulps of a large element.
"""

import numpy as np
import pytest
import torch

from gemma4_mi import model as gm
from gemma4_mi import ops
from gemma4_mi.weights import tensor_key
from oracle import twin

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _gen(shape, seed, name, std=1.0):
    t = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
    ops.fill_normal_(t, tensor_key(seed, name), std)
    return t


def _check(got, exp, what, min_same=0.95):
    g = got.float().cpu().numpy().ravel()
    e = exp.float().cpu().numpy().ravel()
    scale = float(np.abs(e).max())
    err = np.abs(g - e)
    corr = float(np.corrcoef(g, e)[0, 1])
    same = float(np.mean(got.cpu().view(torch.int16).numpy().ravel() == exp.cpu().view(torch.int16).numpy().ravel()))
    print(f"{what}: max|d|={err.max():.3e} scale={scale:.3e} corr={corr:.7f} bit-identical={same:.4f}")
    assert corr >= 0.9999, what
    assert err.max() <= scale * 2.0 ** -6, what
    assert same >= min_same, what


def _prefill_case(T, NH, KV, D, window, softcap, k_eq_v, theta, partial, seed, p0=0, page=64):
    G, eps = NH // KV, 1e-6
    lmax = ((p0 + T + page - 1) // page) * page
    max_pages = lmax // page
    num_pages = max_pages + 3
    q_raw = _gen((T, NH, D), seed, "q")
    k_raw = _gen((T, KV, D), seed, "k")
    v_raw = None if k_eq_v else _gen((T, KV, D), seed, "v")
    q_norm = _gen((D,), seed, "q_norm", 0.5)
    k_norm = _gen((D,), seed, "k_norm", 0.5)
    cos, sin = gm.rope_table(D, theta, partial, lmax, DEV)
    perm = torch.randperm(num_pages, generator=torch.Generator().manual_seed(seed))[:max_pages]
    pt = perm.to(torch.int32).to(DEV)
    # cached prefix (positions < p0), already normalised values
    ck = torch.zeros((lmax, KV, D), dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    if p0:
        ck[:p0] = _gen((p0, KV, D), seed, "prefix_k")
        cv[:p0] = _gen((p0, KV, D), seed, "prefix_v")
    kp = torch.zeros((num_pages, KV, page, D), dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros_like(kp)
    for i in range(max_pages):
        kp[perm[i]] = ck[i * page:(i + 1) * page].permute(1, 0, 2)
        vp[perm[i]] = cv[i * page:(i + 1) * page].permute(1, 0, 2)
    pos = torch.arange(p0, p0 + T, dtype=torch.int32, device=DEV)
    ops.kv_append(k_raw, v_raw, k_norm, cos, sin, kp, vp, pt, pos, lmax, eps)
    q = ops.q_norm_rope(q_raw.clone(), q_norm, cos, sin, p0, eps)
    ctx = ops.prefill_attention(q, kp, vp, pt, p0, window, softcap)
    torch.cuda.synchronize()

    inv = twin.rope_inv_freq(D, theta, partial)
    c, s = twin.rope_tables(list(range(p0, p0 + T)), inv)
    qo = q_raw.cpu().reshape(1, T, KV, G, D)
    ko = k_raw.cpu()[None]
    vo = ko if k_eq_v else v_raw.cpu()[None]
    qp = torch.arange(p0, p0 + T)[:, None]
    kk = torch.arange(lmax)[None, :]
    mask = kk <= qp
    if window:
        mask &= kk > qp - window
    ectx, _, _ = twin.attention_core(qo, ko, vo, q_norm.cpu(), k_norm.cpu(), c, s, ck.cpu()[None], cv.cpu()[None],
                                     p0, mask[None, None, None], lmax, eps, softcap)
    _check(ctx, ectx.reshape(T, NH, D), f"prefill ctx T={T} NH={NH} KV={KV} D={D} W={window} p0={p0}")


def test_small_full_separate_v():
    _prefill_case(200, 4, 2, 64, 0, 0.0, False, 1e4, 1.0, 41)


def test_small_sliding_k_eq_v_softcap_after_cached_prefix():
    _prefill_case(150, 8, 2, 128, 48, 50.0, True, 1e4, 1.0, 42, p0=70)


def test_26b_sliding_shape():
    _prefill_case(300, 16, 8, 256, 100, 0.0, False, 1e4, 1.0, 43)


def test_26b_full_shape():
    _prefill_case(300, 16, 2, 512, 0, 0.0, True, 1e6, 0.25, 44)


def test_long_cached_prefix_beyond_the_staged_page_entries():
    """A block stages the page-table entries of its first 256 key pages in LDS
    and reads later entries directly: 70 query rows after a 16,448-position
    cached prefix (258 pages of 64 over a shuffled table) attend keys on both
    sides of that limit."""
    _prefill_case(70, 4, 2, 64, 0, 0.0, False, 1e4, 1.0, 45, p0=16448)
