"""Gemma-4 MoE decode on one MI355X: hand-written gfx950 kernels behind the
engine/model API of gemma4_tpu (YLiu95/kaggle-tpu-inference).

Heavy modules load lazily, as the reference's package does
(gemma4_tpu/__init__.py), so config-only callers stay light.
"""

__all__ = ["Engine", "TextConfig", "load_text_config"]


def __getattr__(name):
    if name == "Engine":
        from .engine import Engine

        return Engine
    if name in ("TextConfig", "load_text_config"):
        from . import config

        return getattr(config, name)
    raise AttributeError(name)
