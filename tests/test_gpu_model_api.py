"""GPU: the reference's model API (gemma4_tpu/model.py) on the HIP path.

  * the standalone primitives rms_norm, gelu, rope_tables and apply_rope
    (model.py:42-78) against the oracle's restatements;
  * sample / fold_in (model.py:414-424, engine.py:66 and 80): greedy and
    top_k = 1 are the first maximal index, and fold_in(seed, p) draws what the
    engine's decode step at position p draws;
  * the reference's parity procedure (tests/test_parity.py:86-143) call by
    call: make_mesh, params_from_arrays on checkpoint-named arrays,
    init_cache, a padded bucket prefill through forward with prefill_masks
    and the dense-MoE path, then a second cache prefilled to seq - 1 and one
    decode step through forward with decode_masks and the sparse path; the
    logits against the committed HF fixture (tests/golden/hf_tiny_c1.npz)
    and the oracle;
  * forward with B > 1 rows (shared positions, each row its own cache row)
    equals the B = 1 calls; Engine(batch=2) prefills both rows;
  * reset_cache leaves a zero cache after a request.
"""

import numpy as np
import pytest
import torch

from gemma4_mi import model as M
from gemma4_mi import ops
from gemma4_mi.config import tiny_parity_config
from gemma4_mi.engine import Engine
from gemma4_mi.weights import checkpoint_key_map, init_random_params, params_from_arrays
from oracle import twin

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
LOGIT_TOL = 5e-4  # measured max |d| 1.2e-4 against the HF fixture and the oracle
TIE = 2.5e-4


def _bits(t):
    return t.contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32).cpu()


# ---------------------------------------------------------------- primitives
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape,with_w", [((3, 5, 2816), True), ((7, 4, 64), True), ((2, 512), False)])
def test_rms_norm_matches_oracle(dtype, shape, with_w):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * 3.0).to(dtype)
    w = (torch.randn(shape[-1], generator=g) * 0.5).to(torch.bfloat16) if with_w else None
    got = M.rms_norm(x.to(DEV), None if w is None else w.to(DEV), 1e-6).cpu()
    exp = twin.rms_norm(x, w, 1e-6)
    assert got.dtype == dtype and torch.equal(_bits(got), _bits(exp))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gelu_matches_oracle(dtype):
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(100000, generator=g) * 3.0).to(dtype)
    got = M.gelu(x.to(DEV)).cpu()
    exp = twin.gelu(x)
    # device tanhf and torch's CPU tanh may differ in the last f32 ulp; for
    # large negative x, 1 + tanh cancels, so that ulp is bounded in absolute
    # terms (|x| * 2^-24 per ulp of tanh) rather than relative to the output
    d = (got.double() - exp.double()).abs()
    xa = x.double().abs()
    if dtype == torch.bfloat16:
        assert (got == exp).float().mean().item() >= 0.999
        assert bool((d <= exp.double().abs() * 2.0 ** -7 + xa * 2.0 ** -22).all())
    else:
        assert bool((d <= exp.double().abs() * 2.0 ** -21 + xa * 2.0 ** -22).all())


@pytest.mark.parametrize("d,theta,partial", [(256, 1e4, 1.0), (512, 1e6, 0.25), (64, 1e4, 1.0)])
def test_rope_tables_and_apply_rope_match_oracle(d, theta, partial):
    inv = M.rope_inv_freq(d, theta, partial)
    assert np.array_equal(inv, twin.rope_inv_freq(d, theta, partial))
    positions = [0, 1, 7, 1000, 32767]
    cos, sin = M.rope_tables(positions, inv)
    ec, es = twin.rope_tables(positions, inv)
    assert cos.shape == (5, d) and cos.dtype == torch.float32
    for got, exp in ((cos.cpu(), ec), (sin.cpu(), es)):
        ulp = np.spacing(np.abs(exp.numpy()).astype(np.float32))
        assert np.all(np.abs(got.numpy() - exp.numpy()) <= ulp)
        assert (got == exp).float().mean().item() >= 0.999
    g = torch.Generator().manual_seed(d)
    x = torch.randn((2, 5, 3, d), generator=g).to(torch.bfloat16)  # [B, T, heads, D]
    got = M.apply_rope(x.to(DEV), cos, sin).cpu()
    exp = twin.apply_rope(x, cos.cpu(), sin.cpu())
    assert torch.equal(_bits(got), _bits(exp))


def test_sample_greedy_and_fold_in():
    g = torch.Generator().manual_seed(3)
    lg = torch.randn(50000, generator=g) * 4.0
    lg[123] = lg[40000] = 30.0  # a tie: the first index wins
    d = lg.to(DEV)
    assert int(M.sample(d, 5, 0.0, 64, 0.9).item()) == 123
    assert int(M.sample(d, 5, 1.0, 1, 0.9).item()) == 123
    t = M.sample(d, 5, torch.tensor(0.0), 64, torch.tensor(1.0))
    assert t.dtype == torch.int32 and t.ndim == 0 and int(t.item()) == 123
    # fold_in(seed, p) draws what the decode step at position p draws
    lg2 = torch.randn(50000, generator=g).to(DEV)
    for p in (0, 5, 812):
        params = ops.sample_params(0.8, 0.95, 11, DEV)
        tok = torch.zeros(1, dtype=torch.int32, device=DEV)
        pos = torch.tensor([p], dtype=torch.int32, device=DEV)
        ops.sample(lg2, 64, params, tok, 1, pos)
        assert int(M.sample(lg2, M.fold_in(11, p), 0.8, 64, 0.95).item()) == int(tok.item())
    # fold_in(seed, 0) is the draw after a prefill (counter 0)
    params = ops.sample_params(0.8, 0.95, 11, DEV)
    tok = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.sample(lg2, 64, params, tok, 0)
    assert int(M.sample(lg2, M.fold_in(11, 0), 0.8, 64, 0.95).item()) == int(tok.item())
    assert int(M.sample(lg2, 11, 0.8, 64, 0.95).item()) == int(tok.item())


# ---------------------------------------------------------------- the reference's parity procedure
def _hf_named_arrays(cfg, params_cpu):
    """The tiny model's weights under the checkpoint names of a
    Gemma4ForCausalLM state dict (prefix "model."), in HF's 2-D shapes."""
    inv = {v: k for k, v in checkpoint_key_map(cfg, "model.").items()}
    out = {}
    for flat, t in params_cpu.items():
        a = t
        if flat.endswith(("q_proj", "k_proj", "v_proj")):
            a = t.reshape(-1, t.shape[-1])
        elif flat.endswith("o_proj"):
            a = t.reshape(t.shape[0], -1)
        out[inv[flat]] = a.contiguous().view(torch.int16).numpy().view(np.uint16)
    return out


@pytest.fixture(scope="module")
def parity():
    fx = np.load("tests/golden/hf_tiny_c1.npz")
    cfg = tiny_parity_config()
    params_cpu = twin.random_params(cfg, int(fx["seed"]))
    arrays = _hf_named_arrays(cfg, params_cpu)
    mesh = M.make_mesh()
    with mesh:
        params = params_from_arrays(cfg, arrays.__getitem__, list(arrays), mesh, prefix="model.")
    missing = set(M.param_shapes(cfg)) - set(params)
    assert not missing
    return cfg, fx, params, params_cpu, mesh


def test_parity_procedure_prefill(parity):
    cfg, fx, params, params_cpu, mesh = parity
    seq, bucket = int(fx["prompt_len"]), 256
    ids = fx["ids"][:seq][None].astype(np.int32)
    padded = np.zeros((1, bucket), np.int32)
    padded[0, :seq] = ids[0]
    cache = M.init_cache(cfg, mesh, 1, bucket)
    masks = M.prefill_masks(cfg, bucket, seq)
    logits, cache = M.forward(cfg, mesh, params, padded, np.arange(bucket), cache, 0, masks, kv_len=bucket,
                              dense_moe=True, last_index=None)
    assert logits.shape == (1, bucket, cfg.vocab_size)
    got = logits[0, :seq].cpu().numpy()
    rows = [r for r in fx["rows"] if r < seq]
    exp = fx["logits_rows"][: len(rows)]
    err = np.abs(got[rows] - exp)
    corr = np.corrcoef(got[rows].ravel(), exp.ravel())[0, 1]
    print(f"prefill vs HF fixture: max|d|={err.max():.3e} corr={corr:.7f}")
    assert corr >= 0.9999 and err.max() <= LOGIT_TOL
    mism = np.nonzero(got.argmax(-1) != fx["argmax"][:seq])[0]
    assert all(fx["top2_gap"][i] <= TIE for i in mism), mism
    assert bool((logits[0, seq:] == 0).all())  # padded rows are not computed


def test_parity_procedure_decode_step(parity):
    cfg, fx, params, params_cpu, mesh = parity
    seq, bucket = int(fx["prompt_len"]), 256
    ids = fx["ids"][:seq][None].astype(np.int32)
    dec_cache = M.init_cache(cfg, mesh, 1, bucket)
    pref_len = seq - 1
    pad2 = np.zeros((1, bucket), np.int32)
    pad2[0, :pref_len] = ids[0, :pref_len]
    M.forward(cfg, mesh, params, pad2, np.arange(bucket), dec_cache, 0, M.prefill_masks(cfg, bucket, pref_len),
              kv_len=bucket, dense_moe=True)
    pos = torch.tensor(pref_len, dtype=torch.int32)
    dlogits, _ = M.forward(cfg, mesh, params, ids[:, pref_len:pref_len + 1], pos.reshape(1), dec_cache, pos,
                           M.decode_masks(cfg, bucket, pos), kv_len=bucket, dense_moe=False)
    dgot = dlogits[0, 0].cpu().numpy()
    row = list(fx["rows"]).index(seq - 1)
    dexp = fx["logits_rows"][row]
    corr = np.corrcoef(dgot, dexp)[0, 1]
    print(f"decode vs HF fixture: max|d|={np.abs(dgot - dexp).max():.3e} corr={corr:.7f}")
    # the reference's bar for its sparse decode row against the dense prefill row
    assert corr > 0.999 and (dgot.argmax() == dexp.argmax() or fx["top2_gap"][seq - 1] <= TIE)
    # and the oracle's sparse decode step on the same cache contents
    oc = twin.init_cache(cfg, 1, bucket)
    _, oc = twin.forward(cfg, params_cpu, ids[:, :pref_len], np.arange(pref_len), oc, 0,
                         twin.prefill_masks(cfg, pref_len, pref_len), pref_len, True)
    olg, _ = twin.forward(cfg, params_cpu, ids[:, pref_len:pref_len + 1], np.array([pref_len]), oc, pref_len,
                          twin.decode_masks(cfg, bucket, pref_len), bucket, False)
    oexp = olg[0, 0].numpy()
    assert np.abs(dgot - oexp).max() <= LOGIT_TOL and np.corrcoef(dgot, oexp)[0, 1] >= 0.9999


def test_forward_rows_are_sequences(parity):
    """forward with tokens [2, T]: each row runs on its own cache row and
    equals the single-row call, for the prefill and for a decode step at a
    shared position."""
    cfg, fx, params, _, mesh = parity
    T = 40
    rng = np.random.default_rng(9)
    toks = rng.integers(0, cfg.vocab_size, size=(2, T)).astype(np.int32)
    cache2 = M.init_cache(cfg, mesh, 2, 128)
    lg2, cache2 = M.forward(cfg, mesh, params, toks, np.arange(T), cache2, 0, M.prefill_masks(cfg, T, T), T, True)
    nxt = np.array([[5], [77]], np.int32)
    dl2, cache2 = M.forward(cfg, mesh, params, nxt, np.array([T]), cache2, T, M.decode_masks(cfg, 128, T), 128,
                            False)
    for b in range(2):
        c1 = M.init_cache(cfg, mesh, 1, 128)
        lg1, c1 = M.forward(cfg, mesh, params, toks[b:b + 1], np.arange(T), c1, 0, M.prefill_masks(cfg, T, T), T,
                            True)
        dl1, c1 = M.forward(cfg, mesh, params, nxt[b:b + 1], np.array([T]), c1, T, M.decode_masks(cfg, 128, T), 128,
                            False)
        assert torch.equal(lg2[b], lg1[0]) and torch.equal(dl2[b], dl1[0]), b
        for layer in range(cfg.num_hidden_layers):
            for j in range(2):
                a = M.cache_positions(cache2, layer, batch=b, upto=T + 1)[j]
                e = M.cache_positions(c1, layer, batch=0, upto=T + 1)[j]
                assert torch.equal(_bits(a), _bits(e)), (b, layer, j)
    # last_index picks one row
    c1 = M.init_cache(cfg, mesh, 1, 128)
    li, _ = M.forward(cfg, mesh, params, toks[:1], np.arange(T), c1, 0, M.prefill_masks(cfg, T, T), T, True,
                      last_index=T - 1)
    assert li.shape == (1, 1, cfg.vocab_size) and torch.equal(li[0, 0], lg2[0, T - 1])
    with pytest.raises(ValueError):
        M.forward(cfg, mesh, params, toks, np.arange(T), M.init_cache(cfg, mesh, 1, 128), 0,
                  M.prefill_masks(cfg, T, T), T, True)


def test_engine_batch_rows_and_reset_cache():
    cfg = tiny_parity_config()
    params = init_random_params(cfg, 0, device=DEV)
    eng = Engine(None, 256, 2, cfg=cfg, params=params, device=DEV)
    assert eng.batch == 2 and eng.cache["page_table"].shape[0] == 2
    assert eng.cache_bytes == M.cache_bytes(cfg, 2, 256) and eng.n_devices == 1
    rng = np.random.default_rng(12)
    t = 48
    toks = rng.integers(0, cfg.vocab_size, size=(2, t)).astype(np.int32)
    tok, cache, n = eng.prefill_fn(256)(eng.params, torch.tensor(toks), eng.cache, t, 0, 0.0, 1.0)
    # row 0's token equals a batch-1 engine's; row 1's cache equals a prefill of row 1 alone
    one = Engine(None, 256, 1, cfg=cfg, params=params, device=DEV)
    tok1, *_ = one.prefill_fn(256)(one.params, torch.tensor(toks[:1]), one.cache, t, 0, 0.0, 1.0)
    assert int(tok.item()) == int(tok1.item())
    ref = M.init_cache(cfg, None, 1, 256)
    pr = M.PrefillRunner(cfg, params, ref, 64)
    pr.run(torch.tensor(toks[1], dtype=torch.int32, device=DEV), t)
    torch.cuda.synchronize()
    for layer in range(cfg.num_hidden_layers):
        for j in range(2):
            a = M.cache_positions(eng.cache, layer, batch=1, upto=t)[j]
            e = M.cache_positions(ref, layer, batch=0, upto=t)[j]
            assert torch.equal(_bits(a), _bits(e)), (layer, j)
    # a request through generate, then reset_cache: the cache is zero again
    ev = list(eng.generate(toks[0].tolist(), max_new_tokens=20, temperature=0.0, stop_ids=()))
    assert len(ev) == 20
    eng.reset_cache()
    torch.cuda.synchronize()
    for pool in eng.cache["k"] + eng.cache["v"]:
        assert int(torch.count_nonzero(pool).item()) == 0


def test_forward_keeps_no_reference_to_params_or_cache():
    """forward() builds its runners per call: once the caller drops its params
    and cache, nothing in the library keeps them (or their HBM) alive."""
    import gc
    import weakref

    cfg = tiny_parity_config()
    params = init_random_params(cfg, 0, device=DEV)
    cache = M.init_cache(cfg, None, 1, 256, device=DEV)
    ids = np.arange(8, dtype=np.int32)[None]
    logits, cache = M.forward(cfg, None, params, ids, np.arange(8), cache, 0, M.prefill_masks(cfg, 8, 8), kv_len=8,
                              dense_moe=True)
    logits2, cache = M.forward(cfg, None, params, ids[:, :1], np.array([8]), cache, 8, M.decode_masks(cfg, 256, 8),
                               kv_len=256, dense_moe=False)
    torch.cuda.synchronize()
    refs = [weakref.ref(params["embed"]), weakref.ref(params["layers.0.q_proj"]), weakref.ref(cache["k"][0]),
            weakref.ref(cache["page_table"])]
    del params, cache, logits, logits2
    gc.collect()
    assert all(r() is None for r in refs), [r() is None for r in refs]
