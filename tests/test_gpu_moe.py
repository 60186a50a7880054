"""GPU parity of the MoE decode block (router/top-k, expert GEMVs, combine,
and the batched decode's grouped experts) against the CPU oracle, on the isolated-block workload (hidden 2816, 128
experts top-8, width 704, seed 1, batches 1/4/8) and on the tiny model's
shapes.  Also checks the device weight generator bit for bit against its
numpy restatement.

Tolerances: top-k indices bit-exact; top-k weights within 2 f32 ulps (the
recipes are identical, so they are expected bit-exact); expert outputs (bf16)
corr >= 0.9999 with every element within 2^-7 of the output's max magnitude
and >= 98% of elements bit-identical (the GPU accumulates the GEMVs in f32,
the oracle in f64: rare one-ulp flips of bf16 roundings are expected).
"""

import numpy as np
import pytest
import torch

from gemma4_mi import ops
from gemma4_mi.config import tiny_parity_config
from oracle import philox, twin

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


class _C2Cfg:
    hidden_size = 2816
    num_experts = 128
    top_k_experts = 8
    moe_intermediate_size = 704
    rms_norm_eps = 1e-6


def _gen(shape, seed, name, std, device=DEV):
    t = torch.empty(shape, dtype=torch.bfloat16, device=device)
    ops.fill_normal_(t, philox.tensor_key(seed, name), std)
    return t


@pytest.fixture(scope="module")
def c2():
    cfg = _C2Cfg()
    h, e, f = cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size
    g = {
        "router.proj": _gen((e, h), 1, "router.proj", 0.02),
        "router.scale": torch.ones(h, dtype=torch.bfloat16, device=DEV),
        "router.per_expert_scale": torch.ones(e, dtype=torch.bfloat16, device=DEV),
        "experts.gate_up_proj": _gen((e, 2, f, h), 1, "experts.gate_up_proj", 0.02),
        "experts.down_proj": _gen((e, h, f), 1, "experts.down_proj", 0.02),
    }
    torch.cuda.synchronize()
    cpu = {k: v.cpu() for k, v in g.items()}
    return cfg, g, cpu


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def test_fill_normal_matches_numpy_generator():
    n = 3_000_001
    key = philox.tensor_key(7, "probe.tensor")
    t = torch.empty(n + 1, dtype=torch.bfloat16, device=DEV)
    ops.fill_normal_(t[:n], key, 0.02)
    got = _bits(t[:n]).view(np.uint16)
    exp = philox.normal_bf16_bits(n, key, 0.02)
    assert np.array_equal(got, exp), f"{np.sum(got != exp)} of {n} elements differ"


def test_philox_known_answers():
    # Random123 kat_vectors, philox4x32 with 10 rounds
    cases = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in cases:
        c = torch.tensor(np.array(ctr, np.uint32).view(np.int32), device=DEV)
        out = ops.philox4x32_10(c, key[0] | (key[1] << 32)).cpu().numpy().view(np.uint32)
        assert tuple(int(v) for v in out) == want


def _check_out(got, exp, what):
    g = got.float().cpu().numpy().ravel()
    e = exp.float().numpy().ravel()
    scale = float(np.abs(e).max())
    err = np.abs(g - e)
    corr = np.corrcoef(g, e)[0, 1]
    same = np.mean(_bits(got).ravel() == exp.contiguous().view(torch.int16).numpy().ravel())
    print(f"{what}: max|d|={err.max():.3e} (scale {scale:.3e}) corr={corr:.7f} bit-identical={same:.4f}")
    assert corr >= 0.9999, what
    assert err.max() <= scale * 2.0**-7, what
    assert same >= 0.98, what


@pytest.mark.parametrize("n", [1, 4, 8])
def test_router_topk_bit_exact_c2(c2, n):
    cfg, g, cpu = c2
    x = _gen((n, cfg.hidden_size), 1, f"x.n{n}", 1.0)
    tw, ti = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                 cfg.top_k_experts, cfg.rms_norm_eps)
    torch.cuda.synchronize()
    ew, ei = twin.router(cfg, cpu, x.cpu())
    assert np.array_equal(ti.cpu().numpy(), ei.numpy().astype(np.int32))
    np.testing.assert_allclose(tw.cpu().numpy(), ew.numpy(), rtol=2.5e-7, atol=0)


@pytest.mark.parametrize("n", [1, 4, 8])
def test_experts_decode_c2(c2, n):
    cfg, g, cpu = c2
    x = _gen((n, cfg.hidden_size), 1, f"x.n{n}", 1.0)
    tw, ti = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                 cfg.top_k_experts, cfg.rms_norm_eps)
    out = ops.moe_experts(x, g["experts.gate_up_proj"], g["experts.down_proj"], tw, ti)
    torch.cuda.synchronize()
    exp = twin.moe(cfg, cpu, x.cpu(), dense=False)
    _check_out(out, exp, f"experts decode n={n}")


@pytest.mark.parametrize("n", [2, 8, 16])
def test_grouped_decode_experts_equal_pair_path_c2(c2, n):
    """The batched decode's grouped experts (each selected expert's rows read
    once for all the tokens that chose it) compute the same act and partial
    dot products as the per-(token, slot) kernels, so the output is
    bit-identical to moe_experts for both combines; rows 1 and 3 repeat row 0
    so that some experts serve several tokens."""
    cfg, g, cpu = c2
    x = _gen((n, cfg.hidden_size), 1, f"xg.n{n}", 1.0)
    x[1] = x[0]
    if n > 3:
        x[3] = x[0]
    tw, ti = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                 cfg.top_k_experts, cfg.rms_norm_eps)
    gu, dn = g["experts.gate_up_proj"], g["experts.down_proj"]
    for combine in ("bf16_running", "f32"):
        ref = ops.moe_experts(x, gu, dn, tw, ti, combine=combine)
        got = ops.moe_decode_grouped(x, tw, ti, gu, dn, combine=combine)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (n, combine)
    _check_out(got, _dense_selected(cfg, cpu, x.cpu()), f"grouped experts f32 combine n={n}")


@pytest.mark.parametrize("n,pool", [(2, 8), (4, 12), (8, 8), (8, 20), (8, 128)])
def test_gateup_shared_experts_read_once_bit_identical(c2, n, pool):
    """With the routing given and several tokens, an expert chosen by more than
    one (token, slot) pair has its gate/up rows read once (the first pair's
    waves compute every pair's act); act must equal the token-at-a-time calls
    (one token: no sharing) bit for bit.  The experts are drawn from `pool` of
    them (pool 8: every token chose the same 8 experts, in different slots)."""
    cfg, g, _ = c2
    k = cfg.top_k_experts
    x = _gen((n, cfg.hidden_size), 3, f"xs.n{n}.{pool}", 1.0)
    rng = np.random.default_rng(1000 + 10 * n + pool)
    ti = torch.tensor(np.stack([rng.permutation(pool)[:k] for _ in range(n)]), dtype=torch.int32, device=DEV)
    tw = torch.tensor(rng.uniform(0.01, 0.3, size=(n, k)), dtype=torch.float32, device=DEV)
    gu = g["experts.gate_up_proj"]
    got = ops.moe_gateup(x, gu, tw, ti)
    ref = torch.cat([ops.moe_gateup(x[i:i + 1], gu, tw[i:i + 1], ti[i:i + 1]) for i in range(n)])
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (n, pool)


@pytest.mark.parametrize("n,pool", [(2, 8), (3, 128), (4, 12), (8, 8), (8, 20), (8, 128)])
def test_down_shared_rows_bit_identical(c2, n, pool, monkeypatch):
    """From 2 to 8 tokens the down kernel reads an expert's row h once for all
    the tokens that chose it (one wave per row h for every token); its output
    must equal the one-token-row-per-block kernel (G4MI_MOE_DOWN_SHARED=0) bit
    for bit, for both combines, also with expert indices outside the table."""
    cfg, g, _ = c2
    k = cfg.top_k_experts
    x = _gen((n, cfg.hidden_size), 5, f"xd.n{n}.{pool}", 1.0)
    rng = np.random.default_rng(2000 + 10 * n + pool)
    ti = torch.tensor(np.stack([rng.permutation(pool)[:k] for _ in range(n)]), dtype=torch.int32, device=DEV)
    tw = torch.tensor(rng.uniform(0.01, 0.3, size=(n, k)), dtype=torch.float32, device=DEV)
    act = ops.moe_gateup(x, g["experts.gate_up_proj"], tw, ti)
    dn = g["experts.down_proj"]
    ti_bad = ti.clone()
    ti_bad[0, 2] = -1
    ti_bad[n - 1, 6] = cfg.num_experts + 3
    for routing in (ti, ti_bad):
        for combine in ("bf16_running", "f32"):
            monkeypatch.setenv("G4MI_MOE_DOWN_SHARED", "0")
            ref = ops.moe_down(act, dn, routing, combine)
            monkeypatch.setenv("G4MI_MOE_DOWN_SHARED", "1")
            got = ops.moe_down(act, dn, routing, combine)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (n, pool, combine)


@pytest.mark.parametrize("n", [1, 4])
def test_expert_indices_outside_the_table_contribute_nothing(c2, n):
    """A routed expert index outside [0, E) (-1, E + 7) is skipped: the
    output is bit-identical to the same routing with that slot pointing at a
    valid expert with routing weight 0 (whose activation is exactly zero),
    at one token and at four (the gate/up that reads a shared expert once)."""
    cfg, g, _ = c2
    x = _gen((n, cfg.hidden_size), 1, f"x.badexp{n}", 1.0)
    tw, ti = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                 cfg.top_k_experts, cfg.rms_norm_eps)
    ti_bad, tw_zero = ti.clone(), tw.clone()
    ti_bad[0, 3] = -1
    tw_zero[0, 3] = 0.0
    if n > 1:
        ti_bad[n - 1, 5] = cfg.num_experts + 7
        tw_zero[n - 1, 5] = 0.0
    out_bad = ops.moe_experts(x, g["experts.gate_up_proj"], g["experts.down_proj"], tw, ti_bad)
    out_zero = ops.moe_experts(x, g["experts.gate_up_proj"], g["experts.down_proj"], tw_zero, ti)
    torch.cuda.synchronize()
    assert torch.equal(out_bad.view(torch.int16), out_zero.view(torch.int16))


def test_grouped_decode_experts_tiny_shapes():
    """Tiny-model expert shapes (hidden 256, 16 experts top-4, width 128) at
    16 tokens: 64 pairs over at most 16 experts."""
    cfg = tiny_parity_config()
    h, e, f = cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size
    gu = _gen((e, 2, f, h), 7, "tiny.gate_up", 0.02)
    dn = _gen((e, h, f), 7, "tiny.down", 0.02)
    x = _gen((16, h), 7, "tiny.x", 1.0)
    rng = np.random.default_rng(7)
    ti = torch.tensor(np.stack([rng.permutation(e)[: cfg.top_k_experts] for _ in range(16)]), dtype=torch.int32,
                      device=DEV)
    tw = torch.tensor(rng.random((16, cfg.top_k_experts)), dtype=torch.float32, device=DEV)
    ref = ops.moe_experts(x, gu, dn, tw, ti)
    got = ops.moe_decode_grouped(x, tw, ti, gu, dn)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def _dense_selected(cfg, lp, x):
    """Dense-MoE semantics (model.py:241-250) restricted to the selected experts
    (the others carry an exact zero weight)."""
    tw, ti = twin.router(cfg, lp, x)
    outs = []
    for n in range(x.shape[0]):
        acc = torch.zeros(cfg.hidden_size, dtype=torch.float64)
        for kk in range(cfg.top_k_experts):
            e = int(ti[n, kk])
            gu = twin.ein("h,cfh->cf", x[n], lp["experts.gate_up_proj"][e])
            a = twin.rb(twin.f32(twin.gelu(gu[0])) * twin.f32(gu[1]))
            a = twin.rb(twin.f32(a) * twin.f32(twin.rb(tw[n, kk])))
            acc += torch.einsum("f,hf->h", a.double(), lp["experts.down_proj"][e].double())
        outs.append(twin.rb(acc))
    return torch.stack(outs, 0)


def test_experts_f32_combine_c2(c2):
    cfg, g, cpu = c2
    x = _gen((4, cfg.hidden_size), 1, "x.dense", 1.0)
    tw, ti = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                 cfg.top_k_experts, cfg.rms_norm_eps)
    out = ops.moe_experts(x, g["experts.gate_up_proj"], g["experts.down_proj"], tw, ti, combine="f32")
    torch.cuda.synchronize()
    _check_out(out, _dense_selected(cfg, cpu, x.cpu()), "experts f32 combine")


def test_moe_tiny_model_layers():
    """Tiny-model shapes (hidden 256, 16 experts top-4, width 128) with random
    router scales, routed from the residual with the fused pre-norm."""
    cfg = tiny_parity_config()
    params = twin.random_params(cfg, 0)
    for i in range(cfg.num_hidden_layers):
        lp = twin.layer_params(params, i)
        gl = {k: v.to(DEV) for k, v in lp.items()}
        resid = _gen((16, cfg.hidden_size), 5, f"resid.{i}", 1.0)
        tw, ti = ops.moe_router_topk(resid, gl["router.scale"], gl["router.proj"], gl["router.per_expert_scale"],
                                     cfg.top_k_experts, cfg.rms_norm_eps,
                                     pre_norm_w=gl["pre_feedforward_layernorm_2"])
        flat = twin.rms_norm(resid.cpu(), lp["pre_feedforward_layernorm_2"], cfg.rms_norm_eps)
        ew, ei = twin.router(cfg, lp, flat)
        assert np.array_equal(ti.cpu().numpy(), ei.numpy().astype(np.int32)), f"layer {i}"
        np.testing.assert_allclose(tw.cpu().numpy(), ew.numpy(), rtol=2.5e-7, atol=0)
        out = ops.moe_experts(flat.to(DEV), gl["experts.gate_up_proj"], gl["experts.down_proj"], tw, ti)
        _check_out(out, twin.moe(cfg, lp, flat, dense=False), f"tiny layer {i}")


def test_router_rejects_bad_arguments(c2):
    cfg, g, _ = c2
    x = torch.zeros((1, cfg.hidden_size), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(Exception):
        ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"], 0, 1e-6)
    with pytest.raises(Exception):
        ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"], 200, 1e-6)


def test_router_workspace_reuse_across_batch_sizes(c2):
    """A workspace grown for a large batch stays valid for a smaller one (the
    completion counter sits at a fixed offset, not after the score array)."""
    cfg, g, cpu = c2
    for n in (8, 1, 4, 1):
        x = _gen((n, cfg.hidden_size), 1, f"x.reuse{n}", 1.0)
        tw, ti = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                     cfg.top_k_experts, cfg.rms_norm_eps)
        torch.cuda.synchronize()
        _, ei = twin.router(cfg, cpu, x.cpu())
        assert np.array_equal(ti.cpu().numpy(), ei.numpy().astype(np.int32)), n


@pytest.mark.parametrize("n", [1, 4, 8, 16, 17])
def test_router_scores_bit_exact(c2, n):
    cfg, g, cpu = c2
    x = _gen((n, cfg.hidden_size), 1, f"x.n{n}", 1.0)
    s = ops.moe_router_scores(x, g["router.scale"], g["router.proj"], cfg.rms_norm_eps)
    torch.cuda.synchronize()
    xc = twin.rms_norm(x.cpu(), None, cfg.rms_norm_eps)
    c = float(twin.rb(torch.tensor(cfg.hidden_size ** -0.5, dtype=torch.float32)))
    x2 = twin.rb(twin.f32(twin.rb(twin.f32(xc) * twin.f32(cpu["router.scale"]))) * np.float32(c))
    exp = twin.f32(twin.rb(torch.einsum("nh,eh->ne", x2.double(), cpu["router.proj"].double())))
    assert np.array_equal(s.cpu().numpy(), exp.numpy())


@pytest.mark.parametrize("n", [1, 4, 8])
def test_moe_block_decode_c2(c2, n):
    """Router scores -> gate/up with fused selection -> down, against the oracle."""
    cfg, g, cpu = c2
    x = _gen((n, cfg.hidden_size), 1, f"x.block{n}", 1.0)
    out, tw, ti = ops.moe_block(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                g["experts.gate_up_proj"], g["experts.down_proj"], cfg.top_k_experts, cfg.rms_norm_eps)
    torch.cuda.synchronize()
    ew, ei = twin.router(cfg, cpu, x.cpu())
    assert np.array_equal(ti.cpu().numpy(), ei.numpy().astype(np.int32))
    np.testing.assert_allclose(tw.cpu().numpy(), ew.numpy(), rtol=2.5e-7, atol=0)
    _check_out(out, twin.moe(cfg, cpu, x.cpu(), dense=False), f"moe block n={n}")


def test_moe_block_tiny_and_f32_combine():
    """Tiny-model shapes (16 experts top-4) through the fused block, both combines."""
    cfg = tiny_parity_config()
    lp = twin.layer_params(twin.random_params(cfg, 0), 2)
    gl = {k: v.to(DEV) for k, v in lp.items()}
    flat = twin.rms_norm(_gen((32, cfg.hidden_size), 9, "flat", 1.0).cpu(), lp["pre_feedforward_layernorm_2"],
                         cfg.rms_norm_eps)
    out, tw, ti = ops.moe_block(flat.to(DEV), gl["router.scale"], gl["router.proj"], gl["router.per_expert_scale"],
                                gl["experts.gate_up_proj"], gl["experts.down_proj"], cfg.top_k_experts,
                                cfg.rms_norm_eps)
    out32, _, _ = ops.moe_block(flat.to(DEV), gl["router.scale"], gl["router.proj"], gl["router.per_expert_scale"],
                                gl["experts.gate_up_proj"], gl["experts.down_proj"], cfg.top_k_experts,
                                cfg.rms_norm_eps, combine="f32")
    torch.cuda.synchronize()
    _, ei = twin.router(cfg, lp, flat)
    assert np.array_equal(ti.cpu().numpy(), ei.numpy().astype(np.int32))
    _check_out(out, twin.moe(cfg, lp, flat, dense=False), "tiny block")
    _check_out(out32, twin.moe(cfg, lp, flat, dense=True), "tiny block dense")


def test_router_scores_many_rows_match_row_path(c2):
    """N >= 128 rows take the f64-MFMA router kernel (16 rows x 64 experts per
    block); its scores equal the per-row kernel's (64-row calls) bit for bit
    (both sum exact bf16 products in f64 and round once), with and without
    the pre_feedforward_layernorm_2 pre-norm; 1,031 rows leave a ragged last
    tile."""
    cfg, g, _ = c2
    h, e = cfg.hidden_size, cfg.num_experts
    n = 1031
    x = _gen((n, h), 9, "router.rows", 1.0)
    pre = _gen((h,), 9, "router.pre", 0.5)
    for pw in (None, pre):
        many = ops.moe_router_scores(x, g["router.scale"], g["router.proj"], cfg.rms_norm_eps, pre_norm_w=pw)
        rows = torch.cat([ops.moe_router_scores(x[i:i + 64].contiguous(), g["router.scale"], g["router.proj"],
                                                cfg.rms_norm_eps, pre_norm_w=pw) for i in range(0, n, 64)])
        torch.cuda.synchronize()
        assert torch.equal(many, rows), (pw is None, (many != rows).sum().item())


def test_router_scores_wave_kernel_matches_block_kernel(c2):
    """Up to 16 rows the router runs one-wave blocks of two experts, from 17
    rows 4-wave blocks of eight.  Both take exact f64 dots of the same
    rounded router input, so 17 rows in one call equal the same rows in calls
    of 16 and 1, bit for bit, with and without the pre_feedforward_layernorm_2
    pre-norm."""
    cfg, g, _ = c2
    x = _gen((17, cfg.hidden_size), 9, "router.wave", 1.0)
    pre = _gen((cfg.hidden_size,), 9, "router.wave.pre", 0.5)
    for pw in (None, pre):
        block = ops.moe_router_scores(x, g["router.scale"], g["router.proj"], cfg.rms_norm_eps, pre_norm_w=pw)
        wave = torch.cat([ops.moe_router_scores(x[i:j].contiguous(), g["router.scale"], g["router.proj"],
                                                cfg.rms_norm_eps, pre_norm_w=pw) for i, j in ((0, 16), (16, 17))])
        torch.cuda.synchronize()
        assert torch.equal(block, wave), (pw is None, (block != wave).sum().item())


def test_router_scores_mfma_path_bit_exact(c2):
    """300 rows (the f64-MFMA kernel, a ragged last tile) against the oracle's
    f64 product of the same normalised rows, rounded once."""
    cfg, g, cpu = c2
    n = 300
    x = _gen((n, cfg.hidden_size), 1, "x.mfma300", 1.0)
    s = ops.moe_router_scores(x, g["router.scale"], g["router.proj"], cfg.rms_norm_eps)
    torch.cuda.synchronize()
    xc = twin.rms_norm(x.cpu(), None, cfg.rms_norm_eps)
    c = float(twin.rb(torch.tensor(cfg.hidden_size ** -0.5, dtype=torch.float32)))
    x2 = twin.rb(twin.f32(twin.rb(twin.f32(xc) * twin.f32(cpu["router.scale"]))) * np.float32(c))
    exp = twin.f32(twin.rb(torch.einsum("nh,eh->ne", x2.double(), cpu["router.proj"].double())))
    assert np.array_equal(s.cpu().numpy(), exp.numpy())


@pytest.mark.parametrize("e,k,n", [(128, 8, 64), (16, 4, 64), (256, 32, 16), (200, 8, 16)])
def test_wave_selection_equals_block_selection(e, k, n):
    """The selection every gate/up block makes from the router scores
    (moe_block) against the standalone selection kernel (moe_router_topk) on
    the same scores: expert indices and weights bit-identical.  The
    per-expert scale is not all ones (the weight picks up the selected
    expert's scale), E runs from 16 to 256 (one to four waves of experts, the
    last one ragged at 200), and bf16 scores tie within most rows."""
    h, f = 256, 64
    proj = _gen((e, h), 7, f"sel.proj{e}", 0.05)
    scale = _gen((h,), 7, f"sel.scale{e}", 1.0)
    pes = (1.0 + _gen((e,), 7, f"sel.pes{e}", 1.0).float().abs()).to(torch.bfloat16)
    gate_up = _gen((e, 2, f, h), 7, f"sel.gu{e}", 0.02)
    down = _gen((e, h, f), 7, f"sel.dn{e}", 0.02)
    x = _gen((n, h), 8, f"sel.x{e}", 1.0)
    tw_b, ti_b = ops.moe_router_topk(x, scale, proj, pes, k, 1e-6)
    _, tw_w, ti_w = ops.moe_block(x, scale, proj, pes, gate_up, down, k, 1e-6)
    s = ops.moe_router_scores(x, scale, proj, 1e-6)
    torch.cuda.synchronize()
    tied = sum(len(r) != len(set(r)) for r in s.cpu().numpy().tolist())
    print(f"E={e} k={k}: {tied} of {n} rows hold tied scores")
    assert torch.equal(ti_b, ti_w)
    assert torch.equal(tw_b.view(torch.int32), tw_w.view(torch.int32))
