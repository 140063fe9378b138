"""Error type raised by the verify-step operators (mirrors snowllm/errors.py)."""


class SnowLLMError(RuntimeError):
    pass
