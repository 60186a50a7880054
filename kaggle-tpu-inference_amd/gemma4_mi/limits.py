"""Context limits of the resident 32K-token configuration (gemma4_tpu/limits.py)."""

MAX_OUTPUT_TOKENS = 32768
DEFAULT_CONTEXT_TOKENS = 32768


def allowed_output_tokens(requested: int, prompt_tokens: int, context_tokens: int) -> int:
    """Clamp a request to what fits (limits.py:7-9): at least 1 asked, at most
    MAX_OUTPUT_TOKENS, never past the context; 0 when the prompt fills it."""
    room = context_tokens - prompt_tokens
    if room <= 0:
        return 0
    return min(max(requested, 1), MAX_OUTPUT_TOKENS, room)
