"""Global grad mode (reference: src/nanotorch/autograd/grad_mode.py:1-21)."""

_grad_enabled = True


def is_grad_enabled() -> bool:
    """If False, operations do not record the graph."""
    return _grad_enabled


class no_grad:
    """Context manager disabling graph recording."""

    def __init__(self) -> None:
        self._init_state = _grad_enabled

    def __enter__(self):
        global _grad_enabled
        self._init_state = _grad_enabled
        _grad_enabled = False

    def __exit__(self, exc_type, exc, tb):
        global _grad_enabled
        _grad_enabled = self._init_state
