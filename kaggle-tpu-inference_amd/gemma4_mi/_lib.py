"""ctypes binding of libg4mi.so (the gfx950 kernels behind the C ABI in include/g4mi.h).

The library is built in-tree by ``kaggle-tpu-inference_amd/build.py``.  There
is no fallback: if the shared object is missing, :func:`lib` raises, and every
op that needs it fails loudly.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libg4mi.so")

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_u64 = ctypes.c_uint64
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_int = ctypes.c_int

# name -> (restype, argtypes); must cover every function declared in include/g4mi.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "g4mi_version": (_int, []),
    "g4mi_last_error_string": (ctypes.c_char_p, []),
    "g4mi_selftest_lane_reductions": (_int, [_p, _p, _p, _i32, _p]),
    "g4mi_selftest_tile_order": (_int, [_i32, _i32, _i32, _i32, _p, _i64]),
    "g4mi_selftest_exp_nonpositive": (_int, [_i64, _i64, _p, _p]),
    "g4mi_fill_normal_bf16": (_int, [_p, _i64, _u64, _f64, _p]),
    "g4mi_philox4x32_10": (_int, [_p, _u64, _p, _i64, _p]),
    "g4mi_moe_router_scores": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _f32, _p, _p]),
    "g4mi_moe_router_workspace_bytes": (_i64, [_i64, _i64]),
    "g4mi_moe_router_topk": (
        _int,
        [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p, _p, _p, _i64, _p],
    ),
    "g4mi_moe_experts_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "g4mi_moe_gateup": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p]),
    "g4mi_moe_gateup_routed": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "g4mi_moe_down": (_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p]),
    "g4mi_moe_experts_decode": (
        _int,
        [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _i64, _p],
    ),
    "g4mi_moe_block_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "g4mi_attention_min_splits": (_i64, [_i64]),
    "g4mi_decode_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "g4mi_decode_attention": (
        _int,
        [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _f32,
         _i32, _i64, _i64, _p, _p, _i64, _p],
    ),
    "g4mi_gemm_bf16_segments": (_int, [_p, _i64, _i64, _i64, _i32, _p, _p, _p, _p]),
    "g4mi_moe_decode_grouped": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _i64, _p]),
    "g4mi_layer_in": (
        _int,
        [_i32, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _f32,
         _p],
    ),
    "g4mi_oproj": (_int, [_p, _p, _i64, _i64, _p, _p]),
    "g4mi_ffn_in_workspace_bytes": (_i64, []),
    "g4mi_ffn_in": (
        _int,
        [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _i64, _p, _p, _i64, _p, _p, _p, _i64, _i64, _f32, _p],
    ),
    "g4mi_ffn_out_workspace_bytes": (_i64, []),
    "g4mi_ffn_out": (
        _int,
        [_p, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _f32, _p, _i64,
         _i64, _p],
    ),
    "g4mi_lm_head_normed": (_int, [_p, _p, _i64, _i64, _f32, _p, _p, _p, _p]),
    "g4mi_lm_head_blocks": (_i64, [_i64]),
    "g4mi_lm_head": (
        _int,
        [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _f32, _f32, _p, _p, _p, _p],
    ),
    "g4mi_argmax_finalize": (_int, [_p, _p, _i64, _p, _p, _p, _i64, _p]),
    "g4mi_advance_feed": (_int, [_p, _i64, _p, _p, _p, _i64, _p]),
    "g4mi_sample_workspace_bytes": (_i64, [_i64]),
    "g4mi_gemm_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "g4mi_gemm_bf16": (
        _int,
        [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _i32, _p, _i64, _p, _i64, _p, _i64, _p],
    ),
    "g4mi_moe_prefill_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "g4mi_moe_prefill": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p]),
    "g4mi_rows_embed": (_int, [_p, _i64, _p, _i64, _p, _i64, _f32, _p, _p, _p]),
    "g4mi_q_norm_rope": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _p]),
    "g4mi_argmax_rows_workspace_bytes": (_i64, [_i64]),
    "g4mi_argmax_rows": (_int, [_p, _i64, _i64, _f32, _p, _p, _p, _p, _i64, _p, _i64, _p]),
    "g4mi_prefill_attention": (
        _int, [_p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _p, _p],
    ),
    "g4mi_rows_post_attn": (_int, [_p, _p, _i64, _p, _p, _p, _i64, _f32, _p, _p, _p, _p]),
    "g4mi_rows_tail": (_int, [_p, _p, _p, _i64, _p, _p, _p, _p, _p, _i64, _f32, _p, _p, _p]),
    "g4mi_rows_tail_experts": (
        _int,
        [_p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _f32, _p, _p, _p, _i64, _p],
    ),
    "g4mi_sample": (_int, [_p, _i64, _i64, _p, _i32, _p, _p, _p, _i64, _p, _i64, _p]),
    "g4mi_kv_append": (
        _int,
        [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32, _p],
    ),
    "g4mi_moe_block_decode": (
        _int,
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p, _p, _p, _p, _i64, _p],
    ),
    "g4mi_decode_attention_noalloc": (
        _int,
        [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _f32,
         _i32, _i64, _i64, _p, _p],
    ),
    "g4mi_rms_norm": (_int, [_p, _i32, _p, _i32, _i64, _i64, _f32, _p, _p]),
    "g4mi_gelu_tanh": (_int, [_p, _i32, _i64, _p, _p]),
    "g4mi_rope_tables": (_int, [_p, _i64, _p, _i64, _p, _p, _p]),
    "g4mi_apply_rope": (_int, [_p, _i32, _p, _p, _i64, _i64, _i64, _i64, _p, _p]),
}

ABI_VERSION = 1
COMBINE_BF16_RUNNING = 0
COMBINE_F32 = 1

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class G4miError(RuntimeError):
    """A libg4mi entry point rejected its arguments or a launch failed."""

    def __init__(self, what: str, code: int, message: str):
        super().__init__(f"{what} failed (code {code}): {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Loads libg4mi.so once and declares every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python kaggle-tpu-inference_amd/build.py` "
                "(the gfx950 kernels have no CPU fallback)"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        got = handle.g4mi_version()
        if got != ABI_VERSION:
            raise ImportError(f"libg4mi ABI version {got}, expected {ABI_VERSION}; rebuild it")
        _lib = handle
        return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().g4mi_last_error_string()
        raise G4miError(what, rc, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    """Calls an int-returning entry point and raises G4miError on failure."""
    check(getattr(lib(), name)(*args), name)
