"""Dispatch errors with the reference's names and meanings
(CK/exceptions.py:1-40, CK = backends/turbo/vendor/comfy_kitchen)."""


class BackendError(RuntimeError):
    """Base class of dispatch errors."""


class BackendNotFoundError(BackendError):
    def __init__(self, backend_name: str, reason: str | None = None):
        self.backend_name = backend_name
        super().__init__(f"Backend '{backend_name}' is not available" + (f": {reason}" if reason else ""))


class BackendNotImplementedError(BackendError):
    def __init__(self, backend_name: str, func_name: str):
        self.backend_name = backend_name
        self.func_name = func_name
        super().__init__(f"Backend '{backend_name}' does not implement '{func_name}'")


class NoCapableBackendError(BackendError):
    """No registered backend accepts the call (device, dtype or shape)."""

    def __init__(self, func_name: str, failures: dict[str, str]):
        self.func_name = func_name
        self.failures = failures
        if failures:
            detail = "; ".join(f"{k}: {v}" for k, v in failures.items())
            msg = f"No backend can handle '{func_name}': {detail}"
        else:
            msg = f"No backend available for '{func_name}'"
        super().__init__(msg)
