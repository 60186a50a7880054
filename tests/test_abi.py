"""CPU: the C-ABI library (include/g4mi.h) loads, exports every declared
symbol, and its Python binding matches the header.  No compute calls: the
entry points are only driven down their argument-validation paths, which
return before any HIP call, and the host-only size helpers are checked
against known answers."""

import ctypes
import os
import re

import pytest

from gemma4_mi import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "g4mi.h")
EINVAL, EALIGN, EWORKSPACE, EUNSUPPORTED = -1, -2, -3, -4


def _declarations():
    """name -> number of parameters, from the header's prototypes."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    out = {}
    for m in re.finditer(r"\b(g4mi_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        import importlib.util

        spec = importlib.util.spec_from_file_location("g4mi_build", os.path.join(ROOT, "kaggle-tpu-inference_amd",
                                                                                 "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return _lib.lib()


def test_header_declares_the_entry_points():
    decl = _declarations()
    assert len(decl) >= 25
    for name in ("g4mi_moe_router_topk", "g4mi_moe_experts_decode", "g4mi_decode_attention", "g4mi_lm_head",
                 "g4mi_argmax_finalize", "g4mi_last_error_string"):
        assert name in decl


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declarations() if not hasattr(raw, n)]
    assert not missing, missing


def test_binding_matches_header(lib):
    decl = _declarations()
    assert set(_lib.SIGNATURES) == set(decl)
    for name, nparams in decl.items():
        assert len(_lib.SIGNATURES[name][1]) == nparams, name


def test_abi_version(lib):
    ver = int(re.search(r"#define G4MI_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.g4mi_version() == ver == _lib.ABI_VERSION


def test_host_size_helpers(lib):
    assert lib.g4mi_attention_min_splits(32768) == 128
    assert lib.g4mi_attention_min_splits(1024) == 4
    assert lib.g4mi_attention_min_splits(1) == 1
    # the vocabulary over ~3 blocks per CU (768), rows per block a multiple of 8
    assert lib.g4mi_lm_head_blocks(262144) == 763  # 344 rows per block
    assert lib.g4mi_lm_head_blocks(4097) == 513  # 8 rows per block
    assert lib.g4mi_lm_head_blocks(1) == 1
    assert lib.g4mi_moe_router_workspace_bytes(1, 128) == 512
    assert lib.g4mi_moe_router_workspace_bytes(3, 16) == 256
    assert lib.g4mi_moe_experts_workspace_bytes(8, 704, 8) == 8 * 8 * 704 * 2
    assert lib.g4mi_moe_block_workspace_bytes(1, 128, 704, 8) == 512 + 11264
    # scores [B,NH,lmax] f32 + stats [2,B,NH,splits] f32 + partials [B,splits,NH,D] f32 + group sums
    # [B,16,NH,D] f32 + arrival counters [B,NH,17] u32, each 256-aligned
    assert lib.g4mi_decode_attention_workspace_bytes(1, 16, 512, 32768, 128) == (
        16 * 32768 * 4 + 2 * 16 * 128 * 4 + 128 * 16 * 512 * 4 + 16 * 16 * 512 * 4 + 1280)


def _expect(rc, code, fragment):
    assert rc == code, rc
    msg = _lib.lib().g4mi_last_error_string().decode()
    assert fragment in msg, msg


def test_null_arguments_are_rejected_before_any_device_call(lib):
    n = None
    _expect(lib.g4mi_moe_router_topk(n, n, n, n, n, 1, 2816, 128, 8, 1e-6, n, n, n, 0, n), EINVAL, "moe_router_topk")
    _expect(lib.g4mi_moe_gateup(n, n, n, n, 1, 2816, 704, 128, 8, n, n), EINVAL, "moe_gateup")
    _expect(lib.g4mi_moe_down(n, n, n, 1, 2816, 704, 128, 8, 0, n, n), EINVAL, "moe_down")
    _expect(lib.g4mi_moe_experts_decode(n, n, n, n, n, 1, 2816, 704, 128, 8, 0, n, n, 0, n), EINVAL,
            "moe_experts_decode")
    _expect(lib.g4mi_decode_attention(*([n] * 9), 1, n, 1, n, 1, 16, 8, 256, 64, 1024, 0.0, 1e-6, 1, 32768, 128,
                                      n, n, 0, n), EINVAL, "decode_attention")
    _expect(lib.g4mi_kv_append(*([n] * 7), 1, n, 1, n, 1, 8, 256, 64, 32768, 1e-6, n), EINVAL, "kv_append")
    _expect(lib.g4mi_oproj(n, n, 2816, 4096, n, n), EINVAL, "oproj")
    _expect(lib.g4mi_argmax_finalize(n, n, 1024, n, n, n, 0, n), EINVAL, "argmax_finalize")
    _expect(lib.g4mi_philox4x32_10(n, 0, n, 4, n), EINVAL, "philox4x32_10")
    assert lib.g4mi_fill_normal_bf16(n, 0, 0, 1.0, n) == 0  # empty fill is a no-op


def test_unsupported_shapes_are_reported(lib):
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    _expect(lib.g4mi_oproj(fake, fake, 2816, 4100, fake, None), EUNSUPPORTED, "oproj")
    _expect(lib.g4mi_decode_attention(*([fake] * 9), 4, fake, 1, fake, 1, 16, 8, 96, 64, 0, 0.0, 1e-6, 0, 128, 1,
                                      fake, fake, 1 << 30, None), EUNSUPPORTED, "head_dim")
    _expect(lib.g4mi_decode_attention(*([fake] * 9), 4, fake, 1, fake, 1, 16, 8, 256, 64, 0, 0.0, 1e-6, 0, 32768, 8,
                                      fake, fake, 1 << 30, None), EINVAL, "n_split_max")
    _expect(lib.g4mi_decode_attention(*([fake] * 9), 4, fake, 1, fake, 1, 16, 8, 256, 64, 0, 0.0, 1e-6, 0, 32768, 257,
                                      fake, fake, 1 << 30, None), EINVAL, "n_split_max")


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises((ImportError, OSError)):
        _lib.lib()


@pytest.mark.parametrize("grouped", [0, 1])
@pytest.mark.parametrize("max_tiles,ncol", [(256, 22), (256, 1), (17, 5), (9, 3), (1, 1), (64, 11)])
def test_gemm_tile_order_covers_each_live_tile_once(lib, grouped, max_tiles, ncol):
    """The MFMA GEMM's block -> tile map (the library's own code, run on the
    host): with any live tile count up to the grid's maximum, every (row tile,
    column tile) is computed by exactly one block and no block computes a tile
    past the live count.  Plain tiling always runs at mtiles == max_tiles."""
    grid = (max_tiles * ncol + 7) // 8 * 8
    out = (ctypes.c_int32 * (2 * grid))()
    lives = range(max_tiles + 1) if grouped else [max_tiles]
    for mt in lives:
        assert lib.g4mi_selftest_tile_order(mt, max_tiles, ncol, grouped, out, 2 * grid) == 0
        seen = {}
        for b in range(grid):
            tx, ty = out[2 * b], out[2 * b + 1]
            if tx < 0:
                assert ty < 0
                continue
            assert 0 <= tx < mt and 0 <= ty < ncol, (mt, b, tx, ty)
            assert (tx, ty) not in seen, f"tile {(tx, ty)} computed by blocks {seen[(tx, ty)]} and {b} (live {mt})"
            seen[(tx, ty)] = b
        assert len(seen) == mt * ncol, (mt, len(seen))


def test_gemm_tile_order_groups_row_tiles_per_xcd(lib):
    """Plain tiling: consecutive blocks go to the 8 XCDs in turn, and each XCD's
    run holds consecutive tile ids (groups of 8 row tiles, column tiles inner)."""
    mt, ncol = 32, 4
    grid = mt * ncol
    out = (ctypes.c_int32 * (2 * grid))()
    assert lib.g4mi_selftest_tile_order(mt, mt, ncol, 0, out, 2 * grid) == 0
    per = grid // 8
    for x in range(8):
        tiles = [(out[2 * (y * 8 + x)], out[2 * (y * 8 + x) + 1]) for y in range(per)]
        # XCD x runs ids [x*per, (x+1)*per): one group of 8 row tiles x 2 column tiles
        assert {t[0] for t in tiles} == set(range((x // 2) * 8, (x // 2) * 8 + 8)), (x, tiles)
    _expect(lib.g4mi_selftest_tile_order(5, 4, 1, 1, out, 2 * grid), EINVAL, "selftest_tile_order")
