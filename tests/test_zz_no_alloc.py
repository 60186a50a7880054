"""GPU: g4mi_decode_attention_noalloc (the decode attention entry point that
allocates nothing: its split-K scratch is the library's per-device array)
against g4mi_decode_attention with a caller-owned workspace, through the C
ABI, on two calls in a row -- the 26B-A4B full k==v layer at position
20,000 (128 splits, the two-level partial reduction), then the smaller
sliding layer at position 700 -- and on a two-sequence call after them
(another counter layout in the same scratch).  ctx and the appended cache
rows must be identical bit for bit.  A call needing more scratch than the
array holds is rejected before anything is launched."""

import pytest
import torch

from gemma4_mi import _lib, ops
from gemma4_mi import model as M

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
LMAX = 32768


def _gen(shape, key, std=1.0):
    t = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
    ops.fill_normal_(t, key, std)
    return t


def _case(B, NH, KV, D, window, pos_list, key, theta, partial):
    page = 64
    max_pages = LMAX // page
    kp = _gen((B * max_pages, KV, page, D), key + 1)
    vp = _gen((B * max_pages, KV, page, D), key + 2)
    pt = torch.arange(B * max_pages, dtype=torch.int32, device=DEV).reshape(B, max_pages)
    q = _gen((B, NH, D), key + 3)
    k = _gen((B, KV, D), key + 4)
    qn, kn = _gen((D,), key + 5, 0.5), _gen((D,), key + 6, 0.5)
    cos, sin = M.rope_table(D, theta, partial, LMAX, DEV)
    pos = torch.tensor(pos_list, dtype=torch.int32, device=DEV)
    span = window if 0 < window < LMAX else LMAX
    ns = M.decode_splits(KV, span)
    return dict(q=q, k=k, qn=qn, kn=kn, cos=cos, sin=sin, kp=kp, vp=vp, pt=pt, pos=pos, window=window, ns=ns)


def _run_both(c):
    kp_a, vp_a = c["kp"].clone(), c["vp"].clone()
    kp_b, vp_b = c["kp"].clone(), c["vp"].clone()
    B, NH, D = c["q"].shape
    ctx_a = torch.empty((B, NH, D), dtype=torch.bfloat16, device=DEV)
    ctx_b = torch.full((B, NH, D), 7.0, dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(_lib.lib().g4mi_decode_attention_workspace_bytes(B, NH, D, LMAX, c["ns"]), dtype=torch.uint8,
                     device=DEV)
    ops.decode_attention(c["q"], c["k"], None, c["qn"], c["kn"], c["cos"], c["sin"], kp_a, vp_a, c["pt"], c["pos"],
                         c["window"], 50.0, 1e-6, LMAX, c["ns"], append=True, ctx=ctx_a, ws=ws)
    ops.decode_attention_noalloc(c["q"], c["k"], None, c["qn"], c["kn"], c["cos"], c["sin"], kp_b, vp_b, c["pt"],
                                 c["pos"], c["window"], 50.0, 1e-6, LMAX, c["ns"], ctx_b)
    torch.cuda.synchronize()
    assert torch.equal(ctx_a.view(torch.int16), ctx_b.view(torch.int16))
    assert torch.equal(kp_a.view(torch.int16), kp_b.view(torch.int16))
    assert torch.equal(vp_a.view(torch.int16), vp_b.view(torch.int16))
    assert bool(ctx_b.float().abs().sum() > 0)


def test_noalloc_attention_equals_workspace_entry_point():
    full = _case(1, 16, 2, 512, 0, [20000], 100, 1e6, 0.25)
    assert _lib.lib().g4mi_decode_attention_workspace_bytes(1, 16, 512, LMAX, full["ns"]) > (4 << 20)
    _run_both(full)
    sliding = _case(1, 16, 8, 256, 1024, [700], 200, 1e4, 1.0)
    _run_both(sliding)
    two = _case(2, 16, 8, 256, 1024, [5000, 90], 300, 1e4, 1.0)
    _run_both(two)


def test_noalloc_attention_rejects_oversized_calls():
    c = _case(1, 16, 2, 512, 0, [100], 400, 1e6, 0.25)
    big_b = 8
    need = _lib.lib().g4mi_decode_attention_workspace_bytes(big_b, 16, 512, LMAX, 128)
    assert need > (16 << 20)
    q = c["q"].expand(big_b, -1, -1).contiguous()
    pt = torch.zeros((big_b, LMAX // 64), dtype=torch.int32, device=DEV)
    pos = torch.full((big_b,), 100, dtype=torch.int32, device=DEV)
    ctx = torch.full((big_b, 16, 512), 3.0, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.G4miError) as e:
        ops.decode_attention_noalloc(q, None, None, c["qn"], c["kn"], c["cos"], c["sin"], c["kp"], c["vp"], pt, pos,
                                     0, 50.0, 1e-6, LMAX, 128, ctx, append=False)
    assert e.value.code == -3
    torch.cuda.synchronize()
    assert bool((ctx == 3.0).all())
