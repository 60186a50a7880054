"""GPU: the MFMA GEMM of the batched prefill and the dense-MoE prefill
(model.py:241-250).

GEMM (g4mi_gemm_bf16) against float64 products of the same bf16 operands:
  * f32 outputs: |got - ref| <= 2^-16 * sum_k |a_k b_k| + 1e-30 per element
    (f32 accumulation of K products, far inside the (K-1) u bound);
  * bf16 outputs: every element within one bf16 ulp of the f64 value, i.e.
    |got - ref| <= 2^-8 |ref| + the f32 bound above, and >= 99% of elements
    equal to the f64 value rounded once;
  * the gated epilogue against the same rounding points built from f64 gate
    and up values (model.py:220, 246-247): >= 97% bit-identical, corr >= 0.9999
    (a one-ulp flip of a rounded gate or up moves the product by one ulp).
Cases: the tile kernel at the 2,048-token prefill's product shapes (q/k/v/o
and the dense MLP of both layer kinds; 2-stage two-blocks-per-CU and
3-stage one-block-per-CU variants) and through prefill_gemm with the gated
epilogue on separate gate and up tensors; 128x128 tiles with ragged edges,
small M (64-row tiles) with split-K (the slices are summed in order, so
split-K equals the one-slice result within f32 reassociation), the skinny
kernel (M <= 16) alone and with column segments (several weight matrices
sharing A in one launch), row gather, grouped per-expert tiles.

MoE prefill (g4mi_moe_prefill) against the oracle's dense path
(oracle.twin.moe(dense=True): every expert, masked by the routing weights),
with routing from the device router (top-k indices bit-exact to the oracle's):
output corr >= 0.9999, every element within 2^-7 of the output's max
magnitude and >= 97% bit-identical (the oracle sums the 128 x 704 masked
products in f64, the GPU sums eight f32 expert partials).  At the 512-token
prefill size the check is row independence: each token's output equals the
output computed for that token alone, bit for bit (per-row MFMA results do
not depend on the other rows of a tile, and the combine runs in slot order).
"""

import numpy as np
import pytest
import torch

from gemma4_mi import ops
from gemma4_mi.config import tiny_parity_config
from oracle import twin

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _rand(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


def _ref(a, b):
    """float64 A . B^T of bf16 operands and the abs-sum bound."""
    a64, b64 = a.double(), b.double()
    return a64 @ b64.T, a64.abs() @ b64.abs().T


def _check_f32(got, ref, absum):
    err = (got.double().cpu() - ref).abs()
    bound = absum * 2.0**-16 + 1e-30
    assert bool((err <= bound).all()), f"max err/bound {(err / bound).max().item():.3g}"


def _check_bf16(got, ref, absum):
    g = got.cpu().double()
    err = (g - ref).abs()
    bound = ref.abs() * 2.0**-8 + absum * 2.0**-16 + 1e-30
    assert bool((err <= bound).all()), f"max err/bound {(err / bound).max().item():.3g}"
    same = (got.cpu() == twin.rb(ref)).float().mean().item()
    assert same >= 0.99, same


@pytest.mark.parametrize("m,n,k", [(512, 4096, 2816), (300, 1000, 2112), (130, 2816, 4096)])
def test_gemm_plain_bf16_and_f32(m, n, k):
    a, b = _rand((m, k), 1), _rand((n, k), 2, 0.02)
    ref, absum = _ref(a, b)
    ad, bd = a.to(DEV), b.to(DEV)
    _check_bf16(ops.gemm(ad, bd), ref, absum)
    _check_f32(ops.gemm(ad, bd, epilogue=ops.EP_F32), ref, absum)


@pytest.mark.parametrize("m,slices", [(1, 4), (17, 8), (64, 3)])
def test_gemm_small_m_split_k(m, slices):
    n, k = 2816, 4096
    a, b = _rand((m, k), 3), _rand((n, k), 4, 0.02)
    ref, absum = _ref(a, b)
    ad, bd = a.to(DEV), b.to(DEV)
    _check_f32(ops.gemm(ad, bd, epilogue=ops.EP_F32, k_slices=slices), ref, absum)
    _check_bf16(ops.gemm(ad, bd, k_slices=slices), ref, absum)


@pytest.mark.parametrize("m,n,k", [(1, 4096, 2816), (8, 1000, 2112), (16, 2816, 4096), (5, 300, 320),
                                   (8, 20000, 512)])
def test_gemm_skinny_rows(m, n, k):
    """M <= 16 without split-K: the skinny kernel (K split over the block's
    waves, partials summed in wave order; 64 columns per block from N =
    16384)."""
    a, b = _rand((m, k), 12), _rand((n, k), 13, 0.02)
    ref, absum = _ref(a, b)
    ad, bd = a.to(DEV), b.to(DEV)
    _check_bf16(ops.gemm(ad, bd), ref, absum)
    _check_f32(ops.gemm(ad, bd, epilogue=ops.EP_F32), ref, absum)
    rows = torch.tensor([3, 0, 2, 1, 0][: min(m, 5)] * 3, dtype=torch.int32)[:m] % m
    ref2, absum2 = _ref(a[rows.long()], b)
    _check_bf16(ops.gemm(ad, bd, a_rows=rows.to(DEV)), ref2, absum2)


@pytest.mark.parametrize("m", [1, 8, 16])
def test_gemm_segments_share_a(m):
    """q/k/v-style segments in one launch (2816 inputs; 4096 + 2048 + 2048
    columns, and a full layer's 8192 + 1024 at K = 4096): each segment equals
    its own product."""
    for k, widths in ((2816, (4096, 2048, 2048)), (4096, (8192, 1024))):
        a = _rand((m, k), 14)
        bs = [_rand((w, k), 15 + i, 0.02) for i, w in enumerate(widths)]
        outs = [torch.zeros((m, w), dtype=torch.bfloat16, device=DEV) for w in widths]
        ops.gemm_segments(a.to(DEV), [b.to(DEV) for b in bs], outs)
        for b, o in zip(bs, outs):
            ref, absum = _ref(a, b)
            _check_bf16(o, ref, absum)


def test_gemm_row_gather_and_strides():
    a, b = _rand((200, 1024), 5), _rand((384, 1024), 6, 0.02)
    rows = torch.tensor(np.random.default_rng(0).integers(0, 200, size=333), dtype=torch.int32)
    ref, absum = _ref(a[rows.long()], b)
    out = torch.zeros((333, 512), dtype=torch.bfloat16, device=DEV)
    ops.gemm(a.to(DEV), b.to(DEV), out=out, a_rows=rows.to(DEV))
    _check_bf16(out[:, :384], ref, absum)
    assert bool((out[:, 384:] == 0).all())  # ldc 512: columns past N untouched


def _gated_ref(a, gate, up, w):
    g = twin.rb(a.double() @ gate.double().T)
    u = twin.rb(a.double() @ up.double().T)
    act = twin.rb(twin.f32(twin.gelu(g)) * twin.f32(u))
    if w is not None:
        act = twin.rb(twin.f32(act) * twin.f32(twin.rb(w))[:, None])
    return act


def _close_bf16(got, ref, same_min=0.97):
    g, r = got.cpu().float(), ref.float()
    same = (g == r).float().mean().item()
    corr = np.corrcoef(g.flatten().numpy(), r.flatten().numpy())[0, 1]
    assert same >= same_min and corr >= 0.9999, (same, corr)


@pytest.mark.parametrize("m,n,k", [(2048, 4096, 2816), (2048, 2048, 2816), (2048, 8192, 2816), (2048, 2816, 4096),
                                   (2048, 2816, 2112), (2048, 1024, 2816), (54, 4096, 2816)])
def test_gemm_prefill_shapes(m, n, k):
    """The products of a 2,048-token (and the 54-token) prefill through
    prefill_gemm: 512+ tiles run two blocks per CU with 2 LDS stages, fewer
    one block with 3 stages, 54 rows 64-row tiles split over K; repeated
    calls are bit-identical."""
    a, b = _rand((m, k), 16), _rand((n, k), 17, 0.02)
    ref, absum = _ref(a, b)
    ad, bd = a.to(DEV), b.to(DEV)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    ops.prefill_gemm(ad, bd, out)
    _check_bf16(out, ref, absum)
    again = torch.empty_like(out)
    ops.prefill_gemm(ad, bd, again)
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))
    out32 = torch.empty((m, n), dtype=torch.float32, device=DEV)
    ops.prefill_gemm(ad, bd, out32, epilogue=ops.EP_F32)
    _check_f32(out32, ref, absum)


@pytest.mark.parametrize("m", [17, 300, 2048])
def test_prefill_gemm_gated_separate_tensors(m):
    """The dense MLP's gate/up product as the prefill issues it: gate and up
    are separate allocations, reached as b and b + pair_offset (a signed
    element distance) by the fused gated epilogue."""
    h, f = 2816, 2112
    a = _rand((m, h), 18)
    gate, up = _rand((f, h), 19, 0.02), _rand((f, h), 20, 0.02)
    gd, ud = gate.to(DEV), up.to(DEV)
    out = torch.empty((m, f), dtype=torch.bfloat16, device=DEV)
    ops.prefill_gemm(a.to(DEV), gd, out, epilogue=ops.EP_GATED, pair_offset=(ud.data_ptr() - gd.data_ptr()) // 2,
                     n=f)
    _close_bf16(out, _gated_ref(a, gate, up, None))


@pytest.mark.parametrize("m", [5, 64, 300])
def test_gemm_gated_pair(m):
    h, f = 2816, 2112
    a = _rand((m, h), 7)
    gu = _rand((2, f, h), 8, 0.02)  # (gate, up) rows as one tensor
    w = torch.rand(m, generator=torch.Generator().manual_seed(9))
    got = ops.gemm(a.to(DEV), gu.to(DEV), epilogue=ops.EP_GATED, pair_offset=f * h, n=f,
                   row_scale=w.to(DEV))
    _close_bf16(got, _gated_ref(a, gu[0], gu[1], w))
    got1 = ops.gemm(a.to(DEV), gu.to(DEV), epilogue=ops.EP_GATED, pair_offset=f * h, n=f)
    _close_bf16(got1, _gated_ref(a, gu[0], gu[1], None))


def test_gemm_grouped_tiles():
    E, n, k, rows = 6, 320, 512, 400
    a = _rand((150, k), 10)
    b = _rand((E, n, k), 11, 0.05)
    rng = np.random.default_rng(1)
    grp = np.sort(rng.integers(0, E, size=rows))
    grp[grp == 2] = 3  # an empty group
    src = rng.integers(0, 150, size=rows).astype(np.int32)
    tiles = []
    for e in range(E):
        idx = np.nonzero(grp == e)[0]
        for s in range(0, len(idx), 64):
            tiles.append((e, idx[s], idx[min(s + 64, len(idx)) - 1] + 1))
    cap = len(tiles) + 3  # blocks past the live count exit
    t = np.zeros((cap, 3), np.int32)
    t[: len(tiles)] = tiles
    out = ops.gemm(a.to(DEV), b.to(DEV), a_rows=torch.tensor(src, device=DEV), tiles=torch.tensor(t, device=DEV),
                   ntiles=torch.tensor([len(tiles)], dtype=torch.int32, device=DEV), m=rows,
                   epilogue=ops.EP_F32)
    for e in range(E):
        idx = np.nonzero(grp == e)[0]
        if len(idx):
            ref, absum = _ref(a[src[idx]], b[e])
            _check_f32(out[idx], ref, absum)


# ------------------------------------------------------------------ MoE prefill
class _C2Cfg:
    hidden_size = 2816
    num_experts = 128
    top_k_experts = 8
    moe_intermediate_size = 704
    rms_norm_eps = 1e-6


def _moe_params(cfg, seed):
    h, e, f = cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size
    return {
        "router.proj": _rand((e, h), seed, 0.02),
        "router.scale": (1.0 + 0.1 * _rand((h,), seed + 1).float()).to(torch.bfloat16),
        "router.per_expert_scale": (1.0 + 0.1 * _rand((e,), seed + 2).float()).to(torch.bfloat16),
        "experts.gate_up_proj": _rand((e, 2, f, h), seed + 3, 0.02),
        "experts.down_proj": _rand((e, h, f), seed + 4, 0.02),
    }


def _device_moe(cfg, g, x):
    top_w, top_i = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                       cfg.top_k_experts, cfg.rms_norm_eps)
    out = ops.moe_prefill(x, top_w, top_i, g["experts.gate_up_proj"], g["experts.down_proj"])
    return out, top_w, top_i


@pytest.mark.parametrize("which,n", [("tiny", 1), ("tiny", 37), ("tiny", 256), ("tiny", 512), ("26b", 32)])
def test_moe_prefill_matches_dense_oracle(which, n):
    cfg = tiny_parity_config() if which == "tiny" else _C2Cfg()
    lp = _moe_params(cfg, 20)
    g = {k: v.to(DEV) for k, v in lp.items()}
    x = _rand((n, cfg.hidden_size), 30)
    out, top_w, top_i = _device_moe(cfg, g, x.to(DEV))
    ref, rw, ri = twin.moe(cfg, lp, x, dense=True, return_route=True)
    assert torch.equal(top_i.cpu().long(), ri)
    o, r = out.cpu().float(), ref.float()
    corr = np.corrcoef(o.flatten().numpy(), r.flatten().numpy())[0, 1]
    same = (o == r).float().mean().item()
    dmax = (o - r).abs().max().item()
    print(f"{which} n={n}: corr {corr:.7f} identical {same:.4f} max diff {dmax:.3g} of {r.abs().max().item():.3g}")
    assert corr >= 0.9999 and same >= 0.97
    assert dmax <= r.abs().max().item() * 2.0**-7


def test_moe_prefill_rows_independent_at_512_tokens():
    cfg = _C2Cfg()
    g = {k: v.to(DEV) for k, v in _moe_params(cfg, 40).items()}
    x = _rand((512, cfg.hidden_size), 41).to(DEV)
    out, top_w, top_i = _device_moe(cfg, g, x)
    counts = torch.bincount(top_i.flatten().long(), minlength=cfg.num_experts)
    assert int(counts.sum()) == 512 * cfg.top_k_experts
    for t in (0, 1, 255, 511):
        alone = ops.moe_prefill(x[t : t + 1].contiguous(), top_w[t : t + 1].contiguous(),
                                top_i[t : t + 1].contiguous(), g["experts.gate_up_proj"], g["experts.down_proj"])
        assert torch.equal(alone[0], out[t]), t
    assert bool(torch.isfinite(out.float()).all())


@pytest.mark.parametrize("which,n", [("tiny", 512), ("26b", 2048)])
def test_moe_prefill_192_row_tiles_equal_128(monkeypatch, which, n):
    """From 96 (token, slot) pairs per expert on, the expert tiles are 192
    rows (one tile per expert at the 2,048-token prefill, so each expert's
    weights stream once); every output row accumulates over K in the same
    order either way, so the two tilings agree bit for bit, and a row alone
    equals the row in the batch."""
    cfg = tiny_parity_config() if which == "tiny" else _C2Cfg()
    g = {k: v.to(DEV) for k, v in _moe_params(cfg, 50).items()}
    x = _rand((n, cfg.hidden_size), 51).to(DEV)
    top_w, top_i = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                       cfg.top_k_experts, cfg.rms_norm_eps)
    counts = torch.bincount(top_i.flatten().long(), minlength=cfg.num_experts)
    print(f"{which} n={n}: rows per expert {int(counts.min())}..{int(counts.max())}")
    outs = {}
    for rows in ("128", "192"):
        monkeypatch.setenv("G4MI_MOE_TILE_ROWS", rows)
        outs[rows] = ops.moe_prefill(x, top_w, top_i, g["experts.gate_up_proj"], g["experts.down_proj"]).clone()
    torch.cuda.synchronize()
    assert torch.equal(outs["128"].view(torch.int16), outs["192"].view(torch.int16))
    monkeypatch.delenv("G4MI_MOE_TILE_ROWS")
    for t in (0, n // 2, n - 1):
        alone = ops.moe_prefill(x[t : t + 1].contiguous(), top_w[t : t + 1].contiguous(),
                                top_i[t : t + 1].contiguous(), g["experts.gate_up_proj"], g["experts.down_proj"])
        assert torch.equal(alone[0], outs["192"][t]), t
    assert bool(torch.isfinite(outs["192"].float()).all())


@pytest.mark.parametrize("n", [513, 2048, 20000])
def test_moe_sort_blocks_equal_one_block(monkeypatch, n):
    """The expert grouping over several blocks (more than 4,096 (token, slot)
    entries; 20,000 tokens of the tiny model's 4 slots take 2 entries per
    thread) gives what the one-block sort gives, bit for bit, also with expert
    indices outside the table (they contribute nothing)."""
    cfg = tiny_parity_config()
    g = {k: v.to(DEV) for k, v in _moe_params(cfg, 60).items()}
    x = _rand((n, cfg.hidden_size), 61).to(DEV)
    top_w, top_i = ops.moe_router_topk(x, g["router.scale"], g["router.proj"], g["router.per_expert_scale"],
                                       cfg.top_k_experts, cfg.rms_norm_eps)
    top_i[::7, 1] = -1
    top_i[::11, 2] = cfg.num_experts + 3
    outs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("G4MI_MOE_SORT_ONE_BLOCK", flag)
        outs[flag] = ops.moe_prefill(x, top_w, top_i, g["experts.gate_up_proj"], g["experts.down_proj"]).clone()
    torch.cuda.synchronize()
    assert torch.equal(outs["0"].view(torch.int16), outs["1"].view(torch.int16))
    assert bool(torch.isfinite(outs["0"].float()).all())


@pytest.mark.parametrize("which,n", [("tiny", 37), ("tiny", 512), ("26b", 300)])
def test_rows_tail_experts_equals_combine_then_tail(which, n):
    """The layer tail with the MoE combine inside it (moe_prefill without its
    combine, then rows_tail_experts) equals moe_prefill's combined output
    followed by rows_tail, bit for bit (x and the next layer's normed x)."""
    cfg = tiny_parity_config() if which == "tiny" else _C2Cfg()
    H, K, E = cfg.hidden_size, cfg.top_k_experts, cfg.num_experts
    g = {k: v.to(DEV) for k, v in _moe_params(cfg, 60).items()}
    xe = _rand((n, H), 61).to(DEV)
    x1, mlp = _rand((n, H), 62).to(DEV), _rand((n, H), 63, 0.5).to(DEV)
    w1, w2, w3, wn = (_rand((H,), 64 + j).to(DEV) for j in range(4))
    ls = _rand((1,), 70).to(DEV)
    top_w, top_i = ops.moe_router_topk(xe, g["router.scale"], g["router.proj"], g["router.per_expert_scale"], K,
                                       cfg.rms_norm_eps)
    F = g["experts.down_proj"].shape[2]
    moe = ops.moe_prefill(xe, top_w, top_i, g["experts.gate_up_proj"], g["experts.down_proj"])
    xa, xna = torch.empty_like(x1), torch.empty_like(x1)
    ops.rows_tail(x1, mlp, moe, w1, w2, w3, ls, wn, cfg.rms_norm_eps, xa, xna)
    ws = ops.moe_prefill(xe, top_w, top_i, g["experts.gate_up_proj"], g["experts.down_proj"], combine=False)
    xb, xnb = torch.empty_like(x1), torch.empty_like(x1)
    ops.rows_tail_experts(x1, mlp, ws, K, E, F, w1, w2, w3, ls, wn, cfg.rms_norm_eps, xb, xnb)
    torch.cuda.synchronize()
    assert torch.equal(xa.view(torch.int16), xb.view(torch.int16))
    assert torch.equal(xna.view(torch.int16), xnb.view(torch.int16))
