"""Exceptions, mirroring comfy_kitchen.exceptions (roblennon/mac-kernels-public
tests/test_lora_sidepath.py:274-296: ``NoCapableBackendError(func_name, {backend: reason})``)."""


class QlinError(RuntimeError):
    """The HIP library is missing or a HIP runtime call failed."""


class NoCapableBackendError(RuntimeError):
    """No backend accepts the call; callers fall back to their stock path."""

    def __init__(self, func_name, reasons=None):
        self.func_name = func_name
        self.reasons = dict(reasons or {})
        detail = "; ".join(f"{k}: {v}" for k, v in self.reasons.items())
        super().__init__(f"no capable backend for {func_name}" + (f" ({detail})" if detail else ""))
