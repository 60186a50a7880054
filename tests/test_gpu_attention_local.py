"""GPU: the one-launch decode attention (attn_local_kernel) that batch-1
calls on layers with one KV head per XCD take (8 KV heads, every split within
one K tile per wave, at most 1,024 attended positions: the sliding layers of
the 26B shapes, model.py:207-213 with the window of model.py:402-408).

It computes the scores exactly as the two-launch path's first kernel does and
the P.V in the order of its per-slice path (at most 512 attended positions),
so against the two-launch path (selected with G4MI_ATTN_LOCAL=0):
  * ctx bit-identical up to 512 attended positions; beyond (513-1,024, where
    the two-launch path sums split partials instead) against the oracle with
    the attention tests' bounds;
  * the appended K/V rows and every other cache page bit-identical;
  * the page table (explicit identity) and no page table give the same bits;
  * one workspace reused across calls and positions equals a fresh one (the
    head counters are left at zero by every call);
  * a HIP graph of the call, replayed at changing positions with eager work
    in between, equals the eager call at every replay.
"""

import numpy as np
import pytest
import torch

from gemma4_mi import model as gm
from gemma4_mi import ops
from oracle import twin
from test_gpu_attention import _check, _gen, _run_case

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NH, KV, D, W, PAGE = 16, 8, 256, 1024, 64


def _layer(lmax, seed):
    q_raw, k_raw, v_raw = _gen((1, NH, D), seed, "q"), _gen((1, KV, D), seed, "k"), _gen((1, KV, D), seed, "v")
    qn, kn = _gen((D,), seed, "qn", 0.5), _gen((D,), seed, "kn", 0.5)
    cos, sin = gm.rope_table(D, 1e4, 1.0, lmax, DEV)
    kp = _gen((lmax // PAGE, KV, PAGE, D), seed, "kp")
    vp = _gen((lmax // PAGE, KV, PAGE, D), seed, "vp")
    return q_raw, k_raw, v_raw, qn, kn, cos, sin, kp, vp


def _call(layer, pos, lmax, table, ws=None, kp=None, vp=None):
    q_raw, k_raw, v_raw, qn, kn, cos, sin, kp0, vp0 = layer
    kp = kp0.clone() if kp is None else kp
    vp = vp0.clone() if vp is None else vp
    ctx = ops.decode_attention(q_raw, k_raw, v_raw, qn, kn, cos, sin, kp, vp, table,
                               torch.tensor([pos], dtype=torch.int32, device=DEV), W, 0.0, 1e-6, lmax,
                               n_split_max=gm.decode_splits(KV, W), ws=ws)
    return ctx, kp, vp


def _bits(t):
    return t.contiguous().view(torch.int16).cpu()


@pytest.mark.parametrize("pos", [0, 1, 15, 63, 64, 65, 127, 300, 510, 511, 512, 700, 1023, 1024, 1500, 4095])
def test_one_launch_matches_two_launches(monkeypatch, pos):
    lmax = 4096
    layer = _layer(lmax, 71)
    ident = torch.arange(lmax // PAGE, dtype=torch.int32, device=DEV)[None]
    monkeypatch.setenv("G4MI_ATTN_LOCAL", "0")
    ref_ctx, ref_kp, ref_vp = _call(layer, pos, lmax, ident)
    monkeypatch.setenv("G4MI_ATTN_LOCAL", "1")
    outs = [_call(layer, pos, lmax, t) for t in (ident, None)]
    torch.cuda.synchronize()
    for (ctx, kp, vp), what in zip(outs, ("identity table", "no table")):
        print(f"pos {pos} ({what}): ctx bit-identical to the two launches "
              f"{float((_bits(ctx) == _bits(ref_ctx)).float().mean()):.4f}", flush=True)
        assert torch.equal(_bits(kp), _bits(ref_kp)), f"K pages at {pos} ({what})"
        assert torch.equal(_bits(vp), _bits(ref_vp)), f"V pages at {pos} ({what})"
        if pos + 1 <= 512:
            assert torch.equal(_bits(ctx), _bits(ref_ctx)), f"ctx at {pos} ({what})"
    assert torch.equal(_bits(outs[0][0]), _bits(outs[1][0]))
    if pos + 1 > 512:  # the two-launch path sums split partials here: the oracle decides
        q_raw, k_raw, v_raw, qn, kn, cos, sin, kp0, vp0 = layer
        ck = kp0.permute(0, 2, 1, 3).reshape(lmax, KV, D).cpu()
        cv = vp0.permute(0, 2, 1, 3).reshape(lmax, KV, D).cpu()
        lo = max(0, pos + 1 - W)
        n = pos + 1 - lo
        c, s = twin.rope_tables([pos], twin.rope_inv_freq(D, 1e4, 1.0))
        ectx, ek, ev = twin.attention_core(q_raw[0].cpu().reshape(1, 1, KV, NH // KV, D),
                                           k_raw[0].cpu().reshape(1, 1, KV, D), v_raw[0].cpu().reshape(1, 1, KV, D),
                                           qn.cpu(), kn.cpu(), c, s, ck[lo:pos + 1][None], cv[lo:pos + 1][None],
                                           n - 1, torch.ones((1, 1, 1, 1, n), dtype=torch.bool), n, 1e-6, None)
        _check(outs[0][0].reshape(-1), ectx.reshape(-1), f"one launch, pos {pos} vs oracle")
        _check(ref_ctx.reshape(-1), ectx.reshape(-1), f"two launches, pos {pos} vs oracle")


def test_one_launch_against_oracle_with_softcap():
    """The shared attention test harness (shuffled page table, oracle over the
    whole masked cache) at 8 KV heads, B = 1, softcap 50."""
    _run_case(1, NH, KV, D, 2048, PAGE, [900], W, 50.0, False, 1e4, 1.0, 72)
    _run_case(1, NH, KV, D, 2048, PAGE, [200], W, 50.0, False, 1e4, 1.0, 73)


def test_one_workspace_across_calls():
    """A workspace reused by calls at changing positions (each call resets
    its head counters) gives what fresh workspaces give."""
    lmax = 4096
    layer = _layer(lmax, 74)
    nbytes = ops._lib.lib().g4mi_decode_attention_workspace_bytes(1, NH, D, lmax, gm.decode_splits(KV, W))
    shared = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    for pos in (700, 5, 1023, 64, 3000, 700):
        got = _call(layer, pos, lmax, None, ws=shared)[0]
        exp = _call(layer, pos, lmax, None, ws=torch.zeros_like(shared))[0]
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(exp)), pos
    # the counters are back at zero
    assert int(shared[: 16 * 17 * 4].view(torch.int32).abs().sum()) == 0


def test_graph_replays_at_changing_positions():
    """The call captured once in a HIP graph (the decode step's form): replays
    at positions 40, 600, 1023, 2000 and 40 again, with eager work between
    them, each equal to the eager call at that position."""
    lmax = 4096
    layer = _layer(lmax, 75)
    q_raw, k_raw, v_raw, qn, kn, cos, sin, kp0, vp0 = layer
    ns = gm.decode_splits(KV, W)
    nbytes = ops._lib.lib().g4mi_decode_attention_workspace_bytes(1, NH, D, lmax, ns)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    pos_d = torch.zeros(1, dtype=torch.int32, device=DEV)
    kp, vp = kp0.clone(), vp0.clone()
    ctx = torch.empty((1, NH, D), dtype=torch.bfloat16, device=DEV)

    def step():
        ops.decode_attention(q_raw, k_raw, v_raw, qn, kn, cos, sin, kp, vp, None, pos_d, W, 0.0, 1e-6, lmax,
                             n_split_max=ns, ctx=ctx, ws=ws)

    pos_d.fill_(3)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    for p in (40, 600, 1023, 2000, 40):
        kp.copy_(kp0)
        vp.copy_(vp0)
        pos_d.fill_(p)
        g.replay()
        torch.cuda.synchronize()
        got = (_bits(ctx), _bits(kp), _bits(vp))
        exp = _call(layer, p, lmax, None)
        torch.cuda.synchronize()
        assert torch.equal(got[0], _bits(exp[0])), f"ctx at {p}"
        assert torch.equal(got[1], _bits(exp[1])) and torch.equal(got[2], _bits(exp[2])), f"cache at {p}"
        _ = torch.randn(1024, device=DEV).sum().item()  # eager work between replays


@pytest.mark.parametrize("pos", [0, 1, 63, 64, 300, 511, 512, 700, 1023])
def test_one_launch_full_kv_shared_layer(monkeypatch, pos):
    """The full k==v layer shape (16 q / 2 KV heads of 512, partial RoPE, two
    XCDs busy) while its span is at most 1,024 positions: bit-identical to
    the two launches up to 512 attended positions, the oracle beyond."""
    lmax, nh, kv, d, seed, eps = 1024, 16, 2, 512, 76, 1e-6
    q_raw, k_raw = _gen((1, nh, d), seed, "q"), _gen((1, kv, d), seed, "k")
    qn, kn = _gen((d,), seed, "qn", 0.5), _gen((d,), seed, "kn", 0.5)
    cos, sin = gm.rope_table(d, 1e6, 0.25, lmax, DEV)
    kp0 = _gen((lmax // PAGE, kv, PAGE, d), seed, "kp")
    vp0 = _gen((lmax // PAGE, kv, PAGE, d), seed, "vp")
    ns = gm.decode_splits(kv, lmax)
    posd = torch.tensor([pos], dtype=torch.int32, device=DEV)
    out = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("G4MI_ATTN_LOCAL", flag)
        kp, vp = kp0.clone(), vp0.clone()
        ctx = ops.decode_attention(q_raw, k_raw, None, qn, kn, cos, sin, kp, vp, None, posd, 0, 0.0, eps, lmax,
                                   n_split_max=ns)
        torch.cuda.synchronize()
        out[flag] = (ctx, kp, vp)
    same = float((_bits(out["1"][0]) == _bits(out["0"][0])).float().mean())
    print(f"full layer pos {pos}: ctx bit-identical to the two launches {same:.4f}", flush=True)
    assert torch.equal(_bits(out["1"][1]), _bits(out["0"][1])) and torch.equal(_bits(out["1"][2]), _bits(out["0"][2]))
    if pos + 1 <= 512:
        assert same == 1.0
    else:
        ck = kp0.permute(0, 2, 1, 3).reshape(lmax, kv, d).cpu()
        cv = vp0.permute(0, 2, 1, 3).reshape(lmax, kv, d).cpu()
        n = pos + 1
        c, s = twin.rope_tables([pos], twin.rope_inv_freq(d, 1e6, 0.25))
        ectx, _, _ = twin.attention_core(q_raw[0].cpu().reshape(1, 1, kv, nh // kv, d),
                                         k_raw[0].cpu().reshape(1, 1, kv, d), k_raw[0].cpu().reshape(1, 1, kv, d),
                                         qn.cpu(), kn.cpu(), c, s, ck[:n][None], cv[:n][None], n - 1,
                                         torch.ones((1, 1, 1, 1, n), dtype=torch.bool), n, eps, None)
        _check(out["1"][0].reshape(-1), ectx.reshape(-1), f"one launch, full layer, pos {pos} vs oracle")
