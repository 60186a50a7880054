"""GPU parity of split-K decode attention over the paged cache against the
CPU oracle (model.py:197-213 restated in oracle/twin.py).

Cases: small shapes with shuffled page tables, full and sliding masks, two
sequences at different positions; k==v with softcap; the 26B layer shapes at
decode positions on both sides of the 512-position limit between the
per-slice PV path and the split partials; and the two isolated
attention workloads at 32K positions (sliding window 1024 with 16 q / 8 KV
heads at head_dim 256; full k==v with 16 q / 2 KV heads at head_dim 512;
RoPE applied, softcap 50, seed 2); positions outside the cache (past it,
negative) and page-table entries outside the pool on each P.V path.

Tolerances: the appended K/V rows are bit-exact (same deterministic norm and
RoPE recipe); ctx (bf16) has corr >= 0.9999, every element within 2^-7 of
the output's max magnitude and >= 95% of elements bit-identical (the GPU
accumulates dots in f32 in another order than the oracle's f64, which moves
some bf16-rounded probabilities by one ulp).
"""

import math

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


def _pages_from_contig(contig, page, perm, num_pages):
    """contig [lmax, KV, D] -> pages [num_pages, KV, page, D] through perm."""
    lmax, kv, d = contig.shape
    pages = torch.zeros((num_pages, kv, page, d), dtype=torch.bfloat16, device=contig.device)
    for i in range((lmax + page - 1) // page):
        blk = contig[i * page: (i + 1) * page]
        pages[perm[i], :, : blk.shape[0]] = blk.permute(1, 0, 2)
    return pages


def _contig_from_pages(pages, page, perm, lmax):
    num, kv, _, d = pages.shape
    out = torch.empty((lmax, kv, d), dtype=pages.dtype, device=pages.device)
    for i in range((lmax + page - 1) // page):
        n = min(page, lmax - i * page)
        out[i * page: i * page + n] = pages[perm[i], :, :n].permute(1, 0, 2)
    return out


def _check(got, exp, what, min_same=0.95):
    g = got.float().cpu().numpy().ravel()
    e = exp.float().cpu().numpy().ravel()
    scale = float(np.abs(e).max())
    err = np.abs(g - e)
    corr = float(np.corrcoef(g, e)[0, 1])
    same = float(np.mean(got.cpu().view(torch.int16).numpy().ravel() == exp.cpu().view(torch.int16).numpy().ravel()))
    print(f"{what}: max|d|={err.max():.3e} scale={scale:.3e} corr={corr:.7f} bit-identical={same:.4f}")
    assert corr >= 0.9999, what
    assert err.max() <= scale * 2.0 ** -7, what
    assert same >= min_same, what


def _run_case(B, NH, KV, D, lmax, page, positions, window, softcap, k_eq_v, theta, partial, seed, compact=False):
    G = NH // KV
    eps = 1e-6
    q_raw = _gen((B, NH, D), seed, "q")
    k_raw = _gen((B, KV, D), seed, "k")
    v_raw = None if k_eq_v else _gen((B, KV, D), seed, "v")
    q_norm = _gen((D,), seed, "q_norm", 0.5)
    k_norm = _gen((D,), seed, "k_norm", 0.5)
    cos, sin = gm.rope_table(D, theta, partial, lmax, DEV)
    max_pages = (lmax + page - 1) // page
    num_pages = B * max_pages + 3
    g = torch.Generator().manual_seed(seed)
    perm_all = torch.randperm(num_pages, generator=g)
    pt = torch.stack([perm_all[b * max_pages:(b + 1) * max_pages] for b in range(B)]).to(torch.int32)
    ck = [_gen((lmax, KV, D), seed, f"cache_k{b}") for b in range(B)]
    cv = [_gen((lmax, KV, D), seed, f"cache_v{b}") for b in range(B)]
    kp = torch.zeros((num_pages, KV, page, D), dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros_like(kp)
    for b in range(B):
        for i in range(max_pages):
            n = min(page, lmax - i * page)
            kp[pt[b, i], :, :n] = ck[b][i * page: i * page + n].permute(1, 0, 2)
            vp[pt[b, i], :, :n] = cv[b][i * page: i * page + n].permute(1, 0, 2)
    pos = torch.tensor(positions, dtype=torch.int32, device=DEV)
    ctx = ops.decode_attention(q_raw, k_raw, v_raw, q_norm, k_norm, cos, sin, kp, vp, pt.to(DEV), pos, window,
                               softcap, eps, lmax)
    torch.cuda.synchronize()

    inv = twin.rope_inv_freq(D, theta, partial)
    for b, p in enumerate(positions):
        c, s = twin.rope_tables([p], inv)
        qb = q_raw[b].cpu().reshape(1, 1, KV, G, D)
        kb = k_raw[b].cpu().reshape(1, 1, KV, D)
        vb = kb if k_eq_v else v_raw[b].cpu().reshape(1, 1, KV, D)
        lo = max(0, p + 1 - window) if window else 0
        if compact:  # only the attended rows: masked rows contribute exact zeros
            ckc = ck[b][lo: p + 1].cpu()[None]
            cvc = cv[b][lo: p + 1].cpu()[None]
            n = p + 1 - lo
            mask = torch.ones((1, 1, 1, 1, n), dtype=torch.bool)
            ectx, ek, ev = twin.attention_core(qb, kb, vb, q_norm.cpu(), k_norm.cpu(), c, s, ckc, cvc, n - 1, mask, n,
                                               eps, softcap)
            k_row, v_row = ek[0, n - 1], ev[0, n - 1]
        else:
            class C:
                sliding_window = window
            mk = twin.decode_masks(C, lmax, p)
            mask = mk[twin.SLIDING] if window else mk[twin.FULL]
            ectx, ek, ev = twin.attention_core(qb, kb, vb, q_norm.cpu(), k_norm.cpu(), c, s, ck[b].cpu()[None],
                                               cv[b].cpu()[None], p, mask, lmax, eps, softcap)
            k_row, v_row = ek[0, p], ev[0, p]
        got_k = _contig_from_pages(kp, page, pt[b].tolist(), lmax)[p].cpu()
        got_v = _contig_from_pages(vp, page, pt[b].tolist(), lmax)[p].cpu()
        assert torch.equal(got_k.view(torch.int16), k_row.view(torch.int16)), f"appended K row, seq {b}"
        assert torch.equal(got_v.view(torch.int16), v_row.view(torch.int16)), f"appended V row, seq {b}"
        _check(ctx[b].reshape(-1), ectx.reshape(-1), f"ctx seq {b} pos {p}")


def test_small_full_two_sequences():
    _run_case(2, 4, 2, 64, 300, 16, [37, 250], 0, 0.0, False, 1e4, 1.0, 21)


def test_small_sliding_two_sequences():
    _run_case(2, 4, 2, 64, 300, 16, [20, 299], 64, 0.0, False, 1e4, 1.0, 22)


def test_small_position_zero_and_page_boundary():
    _run_case(2, 4, 2, 64, 96, 16, [0, 16], 64, 0.0, False, 1e4, 1.0, 23)


def test_k_eq_v_softcap_eight_heads_per_kv():
    _run_case(1, 8, 1, 128, 520, 64, [519], 0, 50.0, True, 1e6, 0.25, 24)


def test_full_layer_shape_both_sides_of_the_short_range_limit():
    """26B full-layer shape (16 q / 2 KV heads, head_dim 512, k==v): attended
    lengths 301, 511 and 512 take the per-slice path, 513 and 1501 the split
    partials."""
    _run_case(5, 16, 2, 512, 2048, 64, [300, 510, 511, 512, 1500], 0, 0.0, True, 1e6, 0.25, 31)


def test_one_query_head_per_kv_head_long_splits():
    """G = 1 (as many query heads as KV heads) on the 8-wave path for ranges
    of more than 64 positions per split: more threads than score slots."""
    _run_case(2, 2, 2, 64, 2048, 64, [1800, 700], 0, 0.0, False, 1e4, 1.0, 33)


def test_sliding_layer_shape_decode_positions():
    """26B sliding-layer shape (16 q / 8 KV heads, head_dim 256, window
    1024) at decode positions from the first token to a full window."""
    _run_case(4, 16, 8, 256, 4096, 64, [5, 600, 1023, 3000], 1024, 0.0, False, 1e4, 1.0, 32)


def test_isolated_sliding_attention_32k():
    """16 q / 8 KV heads, head_dim 256, window 1024, 32K positions, softcap 50."""
    _run_case(1, 16, 8, 256, 32768, 64, [32767], 1024, 50.0, False, 1e4, 1.0, 2, compact=True)


def test_isolated_full_kv_shared_attention_32k():
    """16 q / 2 KV heads, head_dim 512, k==v, 32,768 cached positions, softcap 50."""
    _run_case(1, 16, 2, 512, 32768, 64, [32767], 0, 50.0, True, 1e6, 0.25, 2, compact=True)


def test_out_of_range_position_attends_to_nothing():
    """A device position beyond the cache leaves it untouched and yields ctx = 0."""
    B, NH, KV, D, lmax, page = 1, 4, 2, 64, 64, 16
    q = _gen((B, NH, D), 5, "q")
    k = _gen((B, KV, D), 5, "k")
    qn = _gen((D,), 5, "qn")
    cos, sin = gm.rope_table(D, 1e4, 1.0, lmax, DEV)
    kp = _gen((4, KV, page, D), 5, "kp")
    vp = _gen((4, KV, page, D), 5, "vp")
    kp0, vp0 = kp.clone(), vp.clone()
    pt = torch.arange(4, dtype=torch.int32, device=DEV)[None]
    ctx = ops.decode_attention(q, k, k, qn, qn, cos, sin, kp, vp, pt, torch.tensor([lmax + 5], dtype=torch.int32,
                               device=DEV), 0, 0.0, 1e-6, lmax)
    torch.cuda.synchronize()
    assert torch.count_nonzero(ctx).item() == 0
    assert torch.equal(kp, kp0) and torch.equal(vp, vp0)


def test_negative_position_attends_to_nothing():
    """A device position below zero leaves the cache untouched and yields ctx = 0."""
    B, NH, KV, D, lmax, page = 1, 4, 2, 64, 64, 16
    q = _gen((B, NH, D), 6, "q")
    k = _gen((B, KV, D), 6, "k")
    qn = _gen((D,), 6, "qn")
    cos, sin = gm.rope_table(D, 1e4, 1.0, lmax, DEV)
    kp = _gen((4, KV, page, D), 6, "kp")
    vp = _gen((4, KV, page, D), 6, "vp")
    kp0, vp0 = kp.clone(), vp.clone()
    pt = torch.arange(4, dtype=torch.int32, device=DEV)[None]
    ctx = ops.decode_attention(q, k, k, qn, qn, cos, sin, kp, vp, pt, torch.tensor([-1], dtype=torch.int32,
                               device=DEV), 0, 0.0, 1e-6, lmax)
    torch.cuda.synchronize()
    assert torch.count_nonzero(ctx).item() == 0
    assert torch.equal(kp, kp0) and torch.equal(vp, vp0)


@pytest.mark.parametrize("lmax,pos,ns", [
    (1024, 300, 16),    # one range of at most 512 positions (per-slice P.V)
    (2048, 900, 32),    # 4-wave splits with the in-kernel reduction
    (4096, 3000, 16),   # 8-wave splits and the reduction launch
])
def test_page_entries_outside_the_pool_are_skipped(lmax, pos, ns):
    """Two page-table entries inside the attended range point outside the
    pool (-1 and num_pages + 5): their positions take no part, as if masked
    (the oracle with those positions masked out), the appended K/V rows are
    bit-exact, and no other page of the pool changes."""
    B, NH, KV, D, page, seed, eps = 1, 8, 2, 64, 16, 61, 1e-6
    G = NH // KV
    max_pages = lmax // page
    q_raw = _gen((B, NH, D), seed, "q")
    k_raw = _gen((B, KV, D), seed, "k")
    v_raw = _gen((B, KV, D), seed, "v")
    q_norm, k_norm = _gen((D,), seed, "q_norm", 0.5), _gen((D,), seed, "k_norm", 0.5)
    cos, sin = gm.rope_table(D, 1e4, 1.0, lmax, DEV)
    ck, cv = _gen((lmax, KV, D), seed, "ck"), _gen((lmax, KV, D), seed, "cv")
    ident = list(range(max_pages))
    kp = _pages_from_contig(ck, page, ident, max_pages)
    vp = _pages_from_contig(cv, page, ident, max_pages)
    bad = [3, (pos // page) // 2]
    pt = torch.arange(max_pages, dtype=torch.int32)
    pt[bad[0]] = -1
    pt[bad[1]] = max_pages + 5
    kp0, vp0 = kp.clone(), vp.clone()
    ctx = ops.decode_attention(q_raw, k_raw, v_raw, q_norm, k_norm, cos, sin, kp, vp, pt[None].to(DEV),
                               torch.tensor([pos], dtype=torch.int32, device=DEV), 0, 0.0, eps, lmax,
                               n_split_max=ns)
    torch.cuda.synchronize()

    class C:
        sliding_window = 0
    mask = twin.decode_masks(C, lmax, pos)[twin.FULL].clone()
    for i in bad:
        mask[..., i * page:(i + 1) * page] = False
    c, s = twin.rope_tables([pos], twin.rope_inv_freq(D, 1e4, 1.0))
    ectx, ek, ev = twin.attention_core(q_raw[0].cpu().reshape(1, 1, KV, G, D), k_raw[0].cpu().reshape(1, 1, KV, D),
                                       v_raw[0].cpu().reshape(1, 1, KV, D), q_norm.cpu(), k_norm.cpu(), c, s,
                                       ck.cpu()[None], cv.cpu()[None], pos, mask, lmax, eps, 0.0)
    _check(ctx[0].reshape(-1), ectx.reshape(-1), f"ctx pos {pos} with pages {bad} outside the pool")
    wp = pos // page
    assert torch.equal(kp[wp, :, pos % page].cpu().view(torch.int16), ek[0, pos].view(torch.int16))
    assert torch.equal(vp[wp, :, pos % page].cpu().view(torch.int16), ev[0, pos].view(torch.int16))
    others = [i for i in range(max_pages) if i != wp]
    assert torch.equal(kp[others], kp0[others]) and torch.equal(vp[others], vp0[others])


def test_sliding_and_full_layers_share_one_workspace():
    """The decode step hands its sliding layers (head_dim 256, 16 splits) and
    full layers (head_dim 512, 128 splits) one workspace.  Its arrival
    counters sit at the start for any head_dim, lmax and split count, so
    alternating the two layouts at positions where both use split partials
    (1,500 and 20,000: the full layer writes partials of 79 splits) gives the
    same results as a fresh workspace per call."""
    lmax, page, seed, eps, NH = 32768, 64, 6, 1e-6, 16
    layers = []
    for D, KV, window, theta, partial, ns in ((256, 8, 1024, 1e4, 1.0, 16), (512, 2, 0, 1e6, 0.25, 128)):
        q_raw, k_raw = _gen((1, NH, D), seed, f"q{D}"), _gen((1, KV, D), seed, f"k{D}")
        v_raw = _gen((1, KV, D), seed, f"v{D}") if window else None
        qn, kn = _gen((D,), seed, f"qn{D}", 0.5), _gen((D,), seed, f"kn{D}", 0.5)
        cos, sin = gm.rope_table(D, theta, partial, lmax, DEV)
        kp = _gen((lmax // page, KV, page, D), seed, f"pk{D}")
        vp = _gen((lmax // page, KV, page, D), seed, f"pv{D}")
        layers.append((D, window, ns, q_raw, k_raw, v_raw, qn, kn, cos, sin, kp, vp))
    nbytes = max(ops._lib.lib().g4mi_decode_attention_workspace_bytes(1, NH, L[0], lmax, L[2]) for L in layers)
    shared = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    pt = torch.arange(lmax // page, dtype=torch.int32, device=DEV).view(1, -1)
    for p in (1500, 20000, 1500):
        pos = torch.tensor([p], dtype=torch.int32, device=DEV)
        for (D, window, ns, q_raw, k_raw, v_raw, qn, kn, cos, sin, kp, vp) in layers + layers:
            got = ops.decode_attention(q_raw, k_raw, v_raw, qn, kn, cos, sin, kp, vp, pt, pos, window, 50.0, eps,
                                       lmax, n_split_max=ns, ws=shared)
            fresh = torch.zeros_like(shared)
            exp = ops.decode_attention(q_raw, k_raw, v_raw, qn, kn, cos, sin, kp, vp, pt, pos, window, 50.0, eps,
                                       lmax, n_split_max=ns, ws=fresh)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), exp.view(torch.int16)), (p, D)


@pytest.mark.parametrize("NH,KV,D,lmax,window,positions", [
    (16, 8, 256, 2048, 1024, [0, 53, 511, 512, 700, 1500]),     # 4-wave kernels
    (16, 2, 512, 32768, 0, [53, 700, 5000, 32767]),            # 8-wave kernels + split reduction
])
def test_dense_page_table_matches_identity_table(NH, KV, D, lmax, window, positions):
    """page_table = NULL (sequence b owns pages [b*max_pages, (b+1)*max_pages)
    in order) computes page indices instead of loading them: ctx and the
    appended K/V rows must be bit-identical to the same call with the
    identity table, for two sequences at different positions."""
    B, page, seed, eps = 2, 16, 51, 1e-6
    max_pages = lmax // page
    q_raw = _gen((B, NH, D), seed, "q")
    k_raw = _gen((B, KV, D), seed, "k")
    v_raw = None if window == 0 else _gen((B, KV, D), seed, "v")
    q_norm, k_norm = _gen((D,), seed, "q_norm", 0.5), _gen((D,), seed, "k_norm", 0.5)
    cos, sin = gm.rope_table(D, 1e4, 1.0, lmax, DEV)
    kp0 = _gen((B * max_pages, KV, page, D), seed, "kp")
    vp0 = _gen((B * max_pages, KV, page, D), seed, "vp")
    ident = torch.arange(B * max_pages, dtype=torch.int32, device=DEV).view(B, max_pages)
    ns = gm.decode_splits(KV, window if window else lmax)
    for i, p in enumerate(positions):
        print(f"case D={D} KV={KV} pos={p}", flush=True)
        pos = torch.tensor([p, positions[(i + 1) % len(positions)]], dtype=torch.int32, device=DEV)
        out = []
        for table in (ident, None):
            kp, vp = kp0.clone(), vp0.clone()
            ctx = ops.decode_attention(q_raw, k_raw, v_raw, q_norm, k_norm, cos, sin, kp, vp, table, pos, window,
                                       50.0, eps, lmax, n_split_max=ns)
            torch.cuda.synchronize()
            out.append((ctx, kp, vp))
        assert torch.equal(out[0][0].view(torch.int16), out[1][0].view(torch.int16)), f"ctx differs at {p}"
        assert torch.equal(out[0][1].view(torch.int16), out[1][1].view(torch.int16)), f"K pages differ at {p}"
        assert torch.equal(out[0][2].view(torch.int16), out[1][2].view(torch.int16)), f"V pages differ at {p}"


def test_dense_page_table_needs_enough_pages():
    q = torch.zeros((2, 4, 64), dtype=torch.bfloat16, device=DEV)
    kp = torch.zeros((3, 2, 16, 64), dtype=torch.bfloat16, device=DEV)  # 2 sequences x 4 pages need 8
    cos = torch.zeros((64, 32), dtype=torch.bfloat16, device=DEV)
    nrm = torch.zeros(64, dtype=torch.bfloat16, device=DEV)
    pos = torch.zeros(2, dtype=torch.int32, device=DEV)
    ops_max_pages = 4
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=DEV)
    ctx = torch.zeros_like(q)
    with pytest.raises(RuntimeError, match="without a page table"):
        ops._lib.call("g4mi_decode_attention", ops._ptr(q), ops._ptr(q[:, :2]), None, ops._ptr(nrm), ops._ptr(nrm),
                      ops._ptr(cos), ops._ptr(cos), ops._ptr(kp), ops._ptr(kp), 3, None, ops_max_pages,
                      ops._ptr(pos), 2, 4, 2, 64, 16, 0, 0.0, 1e-6, 1, 64, 1, ops._ptr(ctx), ops._ptr(ws), ws.numel(),
                      ops.stream_handle(q.device))
