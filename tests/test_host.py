"""CPU: host-side logic of gemma4_mi (config, accounting, layout, masks, RoPE
tables, limits, checkpoint loading) against known answers, the oracle and the
reference's own tests.

Known answers: the reference's limits tests (tests/test_limits.py:9-21); the
26B-A4B parameter, active-parameter and cache sizes (weights.py:138-159,
session.py:49-50, model.py:188-189 evaluated on the published config).
"""

import json

import numpy as np
import pytest
import torch

from gemma4_mi import model as gm
from gemma4_mi import weights as gw
from gemma4_mi.config import (FULL, SLIDING, gemma4_26b_a4b_config, load_text_config, tiny_parity_config,
                              write_text_config)
from gemma4_mi.limits import allowed_output_tokens
from oracle import philox, twin


# ----------------------------------------------------------------- limits (tests/test_limits.py:9-21)
def test_limits_known_answers():
    assert allowed_output_tokens(5000, 54, 32768) == 5000
    assert allowed_output_tokens(32768, 54, 32768) == 32714
    assert allowed_output_tokens(128000, 54, 32768) == 32714
    assert allowed_output_tokens(5000, 32768, 32768) == 0
    assert allowed_output_tokens(0, 10, 100) == 1


# ----------------------------------------------------------------- config and accounting
def test_26b_a4b_sizes():
    cfg = gemma4_26b_a4b_config()
    assert cfg.layer_types.count(FULL) == 5 and cfg.layer_types.count(SLIDING) == 25
    assert [i for i, t in enumerate(cfg.layer_types) if t == FULL] == [5, 11, 17, 23, 29]
    assert cfg.head_dim_for(SLIDING) == 256 and cfg.kv_heads_for(SLIDING) == 8
    assert cfg.head_dim_for(FULL) == 512 and cfg.kv_heads_for(FULL) == 2 and cfg.k_eq_v_for(FULL)
    n_params = sum(int(np.prod(s)) for s in gm.param_shapes(cfg).values())
    assert n_params == 25_233_141_790
    assert gw.param_bytes(cfg) == 2 * n_params
    assert gw.active_params_per_token(cfg) == 3_821_830_144
    assert gw.kv_bytes_per_token(cfg) == 225_280
    assert gm.cache_bytes(cfg, 1, 32768) == 7_381_975_040
    assert gw.decode_bytes(cfg, 54) == 7_656_050_688
    # window-clamped sliding KV: past position 1023 only the full layers grow
    assert gw.decode_bytes(cfg, 2000) - gw.decode_bytes(cfg, 1999) == 5 * 2 * 2 * 2 * 512
    # sqrt(H) in f32, which the reference rounds to bf16 before the multiply (README.md:220)
    assert float(torch.tensor(np.float32(cfg.embed_scale)).to(torch.bfloat16)) == 53.0


def test_tiny_config_sizes():
    cfg = tiny_parity_config()
    assert sum(int(np.prod(s)) for s in gm.param_shapes(cfg).values()) == 9_691_972
    assert tuple(cfg.layer_types) == (SLIDING,) * 3 + (FULL,)


def test_param_shapes_match_oracle():
    for cfg in (tiny_parity_config(), gemma4_26b_a4b_config()):
        a, b = gm.param_shapes(cfg), twin.param_shapes(cfg)
        assert list(a.keys()) == list(b.keys())
        assert all(tuple(a[k]) == tuple(b[k]) for k in a)


def test_config_round_trip(tmp_path):
    cfg = gemma4_26b_a4b_config()
    write_text_config(cfg, str(tmp_path))
    back = load_text_config(str(tmp_path))
    for f in ("hidden_size", "num_hidden_layers", "num_experts", "top_k_experts", "moe_intermediate_size",
              "intermediate_size", "vocab_size", "sliding_window", "head_dim", "global_head_dim",
              "num_key_value_heads", "num_global_key_value_heads", "final_logit_softcapping"):
        assert getattr(back, f) == getattr(cfg, f), f
    assert list(back.layer_types) == list(cfg.layer_types)


def test_config_reads_nested_text_config(tmp_path):
    cfg = tiny_parity_config()
    write_text_config(cfg, str(tmp_path))
    raw = json.load(open(tmp_path / "config.json"))
    nested = {"model_type": "gemma4", "text_config": raw if "text_config" not in raw else raw["text_config"]}
    d2 = tmp_path / "nested"
    d2.mkdir()
    json.dump(nested, open(d2 / "config.json", "w"))
    back = load_text_config(str(d2))
    assert back.hidden_size == cfg.hidden_size and list(back.layer_types) == list(cfg.layer_types)


# ----------------------------------------------------------------- cache layout
def test_cache_pages_cover_the_logical_cache():
    cfg = tiny_parity_config()
    cache = gm.init_cache(cfg, None, 2, 200, device="cpu")
    assert cache["page_size"] == 64
    mp = (200 + 63) // 64
    assert tuple(cache["page_table"].shape) == (2, mp)
    assert sorted(cache["page_table"].reshape(-1).tolist()) == list(range(2 * mp))  # each page owned once
    for i, lt in enumerate(cfg.layer_types):
        assert tuple(cache["k"][i].shape) == (2 * mp, cfg.kv_heads_for(lt), 64, cfg.head_dim_for(lt))
    # a write through the page table lands at the logical position
    kp = cache["k"][0]
    pt = cache["page_table"]
    p, kvh = 130, 1
    kp[pt[1, p // 64], kvh, p % 64] = 7.0
    k, _ = gm.cache_positions(cache, 0, batch=1)
    assert torch.all(k[p, kvh] == 7.0) and int((k != 0).sum()) == cfg.head_dim_for(SLIDING)
    with pytest.raises(ValueError):
        gm.init_cache(cfg, None, 1, 64, dtype=torch.float32, device="cpu")


def test_cache_shapes_match_reference_layout():
    cfg = gemma4_26b_a4b_config()
    assert gm.cache_shapes(cfg, 1, 32768) == twin.cache_shapes(cfg, 1, 32768)


# ----------------------------------------------------------------- masks and RoPE
def test_masks_match_oracle():
    cfg = tiny_parity_config()
    for t, p in ((16, 16), (32, 20), (100, 70)):
        a, b = gm.prefill_masks(cfg, t, p), twin.prefill_masks(cfg, t, p)
        assert torch.equal(a[FULL], b[FULL]) and torch.equal(a[SLIDING], b[SLIDING]) and a["prompt_len"] == p
    for pos in (0, 63, 64, 200):
        a, b = gm.decode_masks(cfg, 256, pos), twin.decode_masks(cfg, 256, pos)
        assert torch.equal(a[FULL], b[FULL]) and torch.equal(a[SLIDING], b[SLIDING]) and a["pos"] == pos


@pytest.mark.parametrize("d,theta,partial", [(256, 1e4, 1.0), (512, 1e6, 0.25), (64, 1e4, 1.0)])
def test_rope_table_matches_oracle(d, theta, partial):
    assert np.array_equal(gm.rope_inv_freq(d, theta, partial), twin.rope_inv_freq(d, theta, partial))
    cos, sin = gm.rope_table(d, theta, partial, 4096, device="cpu")
    pos = [0, 1, 77, 1023, 4095]
    oc, os_ = twin.rope_tables(pos, twin.rope_inv_freq(d, theta, partial))
    assert torch.equal(cos[pos], oc[:, : d // 2].to(torch.bfloat16))
    assert torch.equal(sin[pos], os_[:, : d // 2].to(torch.bfloat16))


# ----------------------------------------------------------------- weights
def test_tensor_key_matches_oracle():
    for seed in (0, 3, 12345):
        for name in ("embed", "layers.29.experts.down_proj"):
            assert gw.tensor_key(seed, name) == philox.tensor_key(seed, name)


def test_checkpoint_loading_from_arrays(tmp_path):
    """params_from_arrays (weights.py:70-83) maps HF checkpoint names and
    reshapes flat projections; load_params streams safetensors and reports
    what is missing (weights.py:86-135)."""
    from safetensors.torch import save_file

    cfg = tiny_parity_config()
    params = twin.random_params(cfg, 0)
    inv = {v: k for k, v in gw.checkpoint_key_map(cfg).items()}
    shapes = gm.param_shapes(cfg)
    ckpt = {}
    for flat, t in params.items():
        if flat.endswith(("q_proj", "k_proj", "v_proj")):
            t = t.reshape(-1, cfg.hidden_size)  # HF stores [heads*D, H]
        elif flat.endswith("o_proj"):
            t = t.reshape(cfg.hidden_size, -1)
        ckpt[inv[flat]] = t.contiguous()
    got = gw.params_from_arrays(cfg, ckpt.__getitem__, list(ckpt), device="cpu")
    assert set(got) == set(shapes)
    assert all(torch.equal(got[k], params[k]) for k in params)
    save_file(ckpt, str(tmp_path / "model.safetensors"))
    loaded = gw.load_params(cfg, str(tmp_path), device="cpu")
    assert all(torch.equal(loaded[k], params[k]) for k in params)
    with pytest.raises(FileNotFoundError):
        gw.load_params(cfg, str(tmp_path / "empty"), device="cpu")
    del ckpt[inv["norm"]]
    (tmp_path / "partial").mkdir()
    save_file(ckpt, str(tmp_path / "partial" / "model.safetensors"))
    with pytest.raises(KeyError):
        gw.load_params(cfg, str(tmp_path / "partial"), device="cpu")


def test_page_pool_allocates_and_releases_pages():
    """batch.PagePool on a CPU cache: rows start unmapped, ensure() maps
    whole pages in order from the shared pool, release() returns them, and an
    exhausted pool or an over-long sequence is refused."""
    from gemma4_mi import model as gm
    from gemma4_mi.batch import PagePool
    from gemma4_mi.config import tiny_parity_config

    cfg = tiny_parity_config()
    cache = gm.init_cache(cfg, None, 2, 256, device="cpu", num_pages=5)
    pool = PagePool(cache)
    pt = cache["page_table"]
    assert pt.shape == (2, 4) and bool((pt == -1).all())
    pool.ensure(0, 1)
    pool.ensure(0, 64)  # still one page
    pool.ensure(1, 130)  # three pages
    assert pool.owned[0] == [0] and pool.owned[1] == [1, 2, 3]
    assert pt[0].tolist() == [0, -1, -1, -1] and pt[1].tolist() == [1, 2, 3, -1]
    with pytest.raises(MemoryError):
        pool.ensure(0, 200)  # needs 3 more, 1 free
    pool.release(1)
    assert pool.free_pages() == 4 and pt[1].tolist() == [-1, -1, -1, -1]
    pool.ensure(0, 256)
    assert len(pool.owned[0]) == 4 and len(set(pt[0].tolist())) == 4
    with pytest.raises(ValueError):
        pool.ensure(1, 257)


def test_make_mesh_is_a_one_device_stand_in():
    """model.py:159-161 callers read mesh.devices.size (engine.py:39) and use
    the mesh as a context manager (tests/test_parity.py:88-90)."""
    from gemma4_mi import model as M

    mesh = M.make_mesh()
    assert int(mesh.devices.size) == 1 and mesh.axis_names == ("tp",) and mesh.size == 1
    with mesh as m:
        assert m is mesh


def test_fold_in_keys():
    from gemma4_mi import model as M

    assert M.fold_in(7, 3) == (7, 3)
    assert M.fold_in((7, 99), 5) == (7, 5)


def _run_bench(*argv):
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    return subprocess.run([sys.executable, os.path.join(root, "bench.py"), *argv], capture_output=True, text=True,
                          timeout=300, cwd=root)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits 2 with a message that
    says so, before touching torch or a device."""
    r = _run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one MI355X" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout == ""


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU exit")
def test_bench_without_a_gpu_exits_without_a_result_line():
    r = _run_bench("--workload", "moe_block", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "needs a GPU" in r.stderr
    assert r.stdout == ""
