"""The decode step's first kernel in tail mode (layer_in mode 1: the previous
layer's tail, the input norm, then the q/k/v projections) against the oracle,
at the 26B-A4B shapes (hidden 2816, up to 8192 + 1024 weight rows).

The tail and the norm are bf16 elementwise steps around f64 sums of squares,
so the residual the kernel stores must equal the oracle's bit for bit, and the
projections must equal those of the same kernel fed the oracle's normalised
vector (mode 3), bit for bit.  Cases: the 26B-A4B hidden size (2816) with and
without the MoE branch, the tiny model's (256), and more weight rows than one
block's prefetch window.
"""

import pytest
import torch

from gemma4_mi import ops
from oracle import twin

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6


def _r(shape, g, std=1.0):
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


@pytest.mark.parametrize("h,moe,rows", [(2816, True, (4096, 2048, 2048)), (2816, False, (512, 256, 256)),
                                        (256, True, (256, 128, 128)), (2816, True, (8192, 1024, 0))])
def test_layer_in_tail_matches_oracle(h, moe, rows):
    g = torch.Generator().manual_seed(h + rows[0] + int(moe))
    x1, mlp, mo = _r((h,), g), _r((h,), g, 4.0), _r((h,), g, 0.25)
    w1, w2, w3, win = _r((h,), g), _r((h,), g), _r((h,), g), _r((h,), g)
    ls = _r((1,), g)
    q, k, v = rows
    wq, wk = _r((q, h), g, 0.02), _r((k, h), g, 0.02)
    wv = _r((v, h), g, 0.02) if v else None

    # oracle: model.py:312-322 (tail) and model.py:298 (input norm)
    if moe:
        hs = twin.rb(twin.f32(twin.rms_norm(mlp, w1, EPS)) + twin.f32(twin.rms_norm(mo, w2, EPS)))
    else:
        hs = mlp
    hh = twin.rms_norm(hs, w3, EPS)
    x = twin.rb(twin.f32(x1) + twin.f32(hh))
    x = twin.rb(twin.f32(x) * twin.f32(ls))
    xn = twin.rms_norm(x, win, EPS)

    d = {n: t.to(DEV) for n, t in dict(x1=x1, mlp=mlp, mo=mo, w1=w1, w2=w2, w3=w3, win=win, ls=ls, wq=wq,
                                         wk=wk, xn=xn).items()}
    wv_d = wv.to(DEV) if wv is not None else None
    x_out = torch.empty(h, dtype=torch.bfloat16, device=DEV)
    out1 = torch.empty(q + k + v, dtype=torch.bfloat16, device=DEV)
    out3 = torch.empty_like(out1)
    ops.layer_in(1, h, EPS, d["win"], x_out, d["wq"], d["wk"], wv_d, q, k, v, out1, x1=d["x1"], mlp_out=d["mlp"],
                 moe_out=d["mo"] if moe else None, post_ff1=d["w1"] if moe else None,
                 post_ff2=d["w2"] if moe else None, post_ff=d["w3"], layer_scalar=d["ls"])
    ops.layer_in(3, h, EPS, d["win"], None, d["wq"], d["wk"], wv_d, q, k, v, out3, x_in=d["xn"])
    torch.cuda.synchronize()
    assert torch.equal(x_out.cpu().view(torch.int16), x.view(torch.int16)), "residual x"
    assert torch.equal(out1.view(torch.int16), out3.view(torch.int16)), "q/k/v from the kernel's own norm"
    ref = (xn.double() @ torch.cat([wq, wk] + ([wv] if wv is not None else [])).double().T)
    err = (out1.cpu().double() - ref).abs().max().item()
    assert err <= ref.abs().max().item() * 2.0 ** -7


@pytest.mark.parametrize("rows,k", [(2816, 4096), (2816, 8192), (256, 256), (1001, 512), (37, 1024)])
def test_oproj_matches_f64_products(rows, k):
    """The decode o_proj GEMV (out = ctx . W^T, one bf16 rounding of an f32
    dot) against the f64 product: every element within one bf16 rounding plus
    the f32 accumulation bound, >= 99% equal to the rounded f64 value.  The
    26B sliding (4096) and full (8192) widths, the tiny model's, and row
    counts that leave partial row groups."""
    g = torch.Generator().manual_seed(rows + k)
    ctx, w = _r((k,), g), _r((rows, k), g, 0.02)
    out = torch.empty(rows, dtype=torch.bfloat16, device=DEV)
    ops.oproj(ctx.to(DEV), w.to(DEV), rows, k, out)
    torch.cuda.synchronize()
    ref = w.double() @ ctx.double()
    absum = w.double().abs() @ ctx.double().abs()
    got = out.cpu().double()
    assert bool(((got - ref).abs() <= ref.abs() * 2.0 ** -8 + absum * 2.0 ** -16).all())
    assert (out.cpu() == twin.rb(ref)).float().mean().item() >= 0.99
