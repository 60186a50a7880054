"""Greedy-token parity for free-running streams: every token a GPU stream
produced must be the oracle's greedy choice given the same history, or a
declared near tie (the oracle's top-two logits within `tie`).  The oracle is
run teacher-forced on the GPU's own tokens, so one early near tie does not
hide what follows it."""

import numpy as np

from oracle import twin


def check_stream(cfg, params_cpu, prompt, gen, max_len, tie=2e-3, what="stream"):
    """gen = the GPU's first token after the prompt, then its decode tokens.
    Returns the teacher-forced agreement count; asserts the near-tie rule."""
    logits, _ = twin.prefill_then_decode(cfg, params_cpu, prompt, len(gen) - 1, max_len, all_logits=False,
                                         forced=gen)
    rows = logits.numpy()
    agree = 0
    for s, t in enumerate(gen):
        best = int(np.argmax(rows[s]))
        if t == best:
            agree += 1
            continue
        gap = float(rows[s][best] - rows[s][t])
        print(f"{what}: step {s} token {t} vs oracle {best}, oracle gap {gap:.3e}")
        assert gap <= tie, f"{what}: step {s} is not a near tie ({gap:.3e})"
    print(f"{what}: teacher-forced agreement {agree}/{len(gen)}")
    return agree
