"""Lane layout of the cross-lane reductions (DPP row moves + bpermute) that
every kernel uses: each lane must hold the sum of its aligned group."""

import numpy as np
import pytest
import torch

from gemma4_mi import _lib, ops

pytestmark = pytest.mark.gpu


def test_group_sums_match_host():
    waves = 4
    rng = np.random.default_rng(3)
    x = rng.standard_normal(64 * waves).astype(np.float32)
    # distinct magnitudes so a wrong partner lane changes the sum
    x += np.arange(64 * waves, dtype=np.float32) * 1000.0
    inp = torch.tensor(x, device="cuda:0")
    out = torch.empty(waves * 6 * 64, dtype=torch.float32, device="cuda:0")
    out_d = torch.empty(waves * 6 * 64, dtype=torch.float64, device="cuda:0")
    _lib.call("g4mi_selftest_lane_reductions", ops._ptr(inp), ops._ptr(out), ops._ptr(out_d), waves,
              ops.stream_handle())
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(waves, 6, 64)
    got_d = out_d.cpu().numpy().reshape(waves, 6, 64)
    for w in range(waves):
        xs = x[64 * w: 64 * (w + 1)].astype(np.float64)
        for j in range(6):
            width = 2 ** (j + 1)
            exp = np.repeat(xs.reshape(-1, width).sum(1), width)
            np.testing.assert_allclose(got[w, j], exp, rtol=1e-6, err_msg=f"f32 width {width}")
            np.testing.assert_allclose(got_d[w, j], exp, rtol=1e-12, err_msg=f"f64 width {width}")
            # every lane of a group holds the bitwise-same total
            g = got[w, j].reshape(-1, width)
            assert np.all(g == g[:, :1]), f"f32 width {width} not uniform across the group"


def test_softmax_exp_matches_expf_on_every_nonpositive_float():
    """The prefill attention's exp for x <= 0 (exp_nonpos) rounds as expf does
    for every float in [-104, 0]: all 1,120,927,745 of them."""
    mism = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    count = 0x42D00000 + 1  # bits of -0.0 .. -104.0
    _lib.call("g4mi_selftest_exp_nonpositive", 0, count, ops._ptr(mism), ops.stream_handle())
    torch.cuda.synchronize()
    assert int(mism.item()) == 0
