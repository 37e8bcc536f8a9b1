"""Capability-checked backend dispatch with the reference's plugin surface.

Mirrors the interface of CK/registry.py:20-307 and CK/constraints.py:94-255
(CK = backends/turbo/vendor/comfy_kitchen): a backend registers a module and a
``{function name: FunctionConstraints}`` map; a call picks the first backend in
priority order whose constraints accept the arguments (device type, dtype,
shape rules, call rules), with a thread-local ``use_backend`` override. The
MI355X backend registers as ``"mi355x"``; with no capable backend the call
raises ``NoCapableBackendError`` (there is no silent CPU path).
"""

from __future__ import annotations

import threading
from abc import ABC, abstractmethod
from collections.abc import Callable, Mapping
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any

import torch

from .exceptions import BackendNotFoundError, BackendNotImplementedError, NoCapableBackendError


# --------------------------------------------------------------------------- constraints
# The classes carry every attribute and method the reference's own
# validation reads (CK/constraints.py:90-255: ``dtypes``, ``devices``,
# ``shape_rules``, ``check_dtype``, ``check_device``, ``check_shape``,
# ``default_devices``, ``min_compute_capability``, ``call_rules``), so a
# capability table built here registers unchanged in the reference registry.

@dataclass(frozen=True)
class ValidationResult:
    success: bool
    failed_param: str | None = None
    failure_reason: str | None = None

    @staticmethod
    def ok() -> "ValidationResult":
        return ValidationResult(True)

    @staticmethod
    def fail(param: str, reason: str) -> "ValidationResult":
        return ValidationResult(False, param, reason)


class ShapeRule(ABC):
    """A predicate on a tensor's shape with a readable description."""

    @abstractmethod
    def check(self, t: torch.Tensor) -> bool: ...

    @abstractmethod
    def describe(self) -> str: ...


@dataclass(frozen=True)
class DivisibleBy(ShapeRule):
    dim: int
    factor: int

    def check(self, t: torch.Tensor) -> bool:
        return t.dim() > self.dim and t.shape[self.dim] % self.factor == 0

    def describe(self) -> str:
        return f"dim[{self.dim}] divisible by {self.factor}"


@dataclass(frozen=True)
class ExactDims(ShapeRule):
    ndim: int

    def check(self, t: torch.Tensor) -> bool:
        return t.dim() == self.ndim

    def describe(self) -> str:
        return f"exactly {self.ndim}D"


@dataclass(frozen=True)
class MinDims(ShapeRule):
    ndim: int

    def check(self, t: torch.Tensor) -> bool:
        return t.dim() >= self.ndim

    def describe(self) -> str:
        return f"at least {self.ndim}D"


@dataclass(frozen=True)
class ParamConstraint:
    """dtypes (None = any; a set of torch dtypes, or Python types for
    non-tensor arguments), device types (None = the function's default) and
    shape rules of one argument."""

    dtypes: frozenset | None = None
    devices: frozenset[str] | None = None
    shape_rules: tuple = ()

    def check_dtype(self, value: Any) -> bool:
        if self.dtypes is None:
            return True
        dt = value.dtype if isinstance(value, torch.Tensor) else value
        return dt in self.dtypes or type(value) in self.dtypes

    def check_device(self, tensor: torch.Tensor, default_devices: frozenset[str]) -> bool:
        allowed = self.devices if self.devices is not None else default_devices
        return "*" in allowed or tensor.device.type in allowed

    def check_shape(self, tensor: torch.Tensor) -> bool:
        return all(rule.check(tensor) for rule in self.shape_rules)


@dataclass(frozen=True)
class FunctionConstraints:
    params: dict[str, ParamConstraint] = field(default_factory=dict)
    default_devices: frozenset[str] = frozenset({"cuda"})
    min_compute_capability: tuple[int, int] | None = None
    call_rules: tuple[Callable[[Mapping[str, Any]], ValidationResult], ...] = ()

    def __hash__(self) -> int:
        return hash((tuple(sorted(self.params)), self.default_devices, self.min_compute_capability,
                     self.call_rules))


def validate_param(name: str, value: Any, c: ParamConstraint, default_devices: frozenset[str]) -> ValidationResult:
    if value is None:
        return ValidationResult.ok()
    if not c.check_dtype(value):
        dt = value.dtype if isinstance(value, torch.Tensor) else value
        return ValidationResult.fail(name, f"dtype {dt} not in {set(c.dtypes)}")
    if not isinstance(value, torch.Tensor):
        return ValidationResult.ok()
    if not c.check_device(value, default_devices):
        allowed = c.devices if c.devices is not None else default_devices
        return ValidationResult.fail(name, f"device {value.device.type} not in {set(allowed)}")
    for rule in c.shape_rules:
        if not rule.check(value):
            return ValidationResult.fail(name, f"shape {list(value.shape)} fails: {rule.describe()}")
    return ValidationResult.ok()


def validate_function_call(c: FunctionConstraints, kwargs: Mapping[str, Any],
                           compute_capability: tuple[int, int] | None = None) -> ValidationResult:
    if c.min_compute_capability is not None:
        if compute_capability is None:
            return ValidationResult.fail("__hardware__", "compute capability required but not available")
        if tuple(compute_capability) < tuple(c.min_compute_capability):
            return ValidationResult.fail(
                "__hardware__", f"compute capability {compute_capability} < required {c.min_compute_capability}")
    for name, pc in c.params.items():
        r = validate_param(name, kwargs.get(name), pc, c.default_devices)
        if not r.success:
            return r
    for rule in c.call_rules:
        r = rule(kwargs)
        if not r.success:
            return r
    return ValidationResult.ok()


# --------------------------------------------------------------------------- registry

class BackendRegistry:
    def __init__(self) -> None:
        self._backends: dict[str, Any] = {}
        self._caps: dict[str, set[str]] = {}
        self._constraints: dict[tuple[str, str], FunctionConstraints] = {}
        self._priority: list[str] = ["mi355x"]
        self._disabled: set[str] = set()
        self._unavailable: dict[str, str] = {}
        self._lock = threading.Lock()
        self._tls = threading.local()
        self._cc_known = False
        self._cc: tuple[int, int] | None = None

    # registration ---------------------------------------------------------
    def register(self, name: str, module: Any, capabilities: dict[str, FunctionConstraints]) -> None:
        with self._lock:
            self._backends[name] = module
            self._caps[name] = set(capabilities)
            for fn, c in capabilities.items():
                self._constraints[(name, fn)] = c
            self._unavailable.pop(name, None)
            if name not in self._priority:
                self._priority.append(name)

    def mark_unavailable(self, name: str, reason: str) -> None:
        with self._lock:
            self._unavailable[name] = reason

    def get_constraints(self, backend: str, func: str) -> FunctionConstraints | None:
        return self._constraints.get((backend, func))

    # configuration --------------------------------------------------------
    def disable(self, name: str) -> None:
        with self._lock:
            self._disabled.add(name)

    def enable(self, name: str) -> None:
        with self._lock:
            self._disabled.discard(name)

    def set_priority(self, names: list[str]) -> None:
        with self._lock:
            self._priority = list(names)

    def is_available(self, name: str) -> bool:
        return name in self._backends and name not in self._disabled

    def list_backends(self) -> dict:
        names = set(self._priority) | set(self._backends) | set(self._unavailable)
        return {n: {"available": n in self._backends, "disabled": n in self._disabled,
                    "unavailable_reason": self._unavailable.get(n),
                    "capabilities": sorted(self._caps.get(n, ()))} for n in names}

    # selection ------------------------------------------------------------
    def validate_backend_for_call(self, backend: str, func: str, kwargs: Mapping[str, Any]) -> ValidationResult:
        if not self.is_available(backend):
            return ValidationResult.fail("__backend__", self._unavailable.get(backend, "not available"))
        if func not in self._caps.get(backend, ()):
            return ValidationResult.fail("__function__", "not implemented")
        c = self._constraints.get((backend, func))
        return ValidationResult.ok() if c is None else validate_function_call(c, kwargs, self.compute_capability())

    def compute_capability(self) -> tuple[int, int] | None:
        """(major, minor) of the current GPU as torch reports it, or None."""
        if not self._cc_known:
            self._cc_known = True
            if torch.cuda.is_available():
                try:
                    props = torch.cuda.get_device_properties(torch.cuda.current_device())
                    self._cc = (props.major, props.minor)
                except Exception:  # noqa: BLE001 - no device properties: no capability
                    self._cc = None
        return self._cc

    def get_capable_backend(self, func: str, kwargs: Mapping[str, Any] | None = None) -> str:
        failures: dict[str, str] = {}
        override = getattr(self._tls, "override", None)
        candidates = [override] if override else []
        candidates += [b for b in self._priority if b != override]
        for b in candidates:
            if not self.is_available(b):
                if b == override:
                    failures[b] = "not available"
                continue
            if func not in self._caps.get(b, ()):
                if b == override:
                    failures[b] = "not implemented"
                continue
            if kwargs:
                r = self.validate_backend_for_call(b, func, kwargs)
                if not r.success:
                    failures[b] = f"{r.failed_param}: {r.failure_reason}"
                    continue
            return b
        raise NoCapableBackendError(func, failures)

    def get_implementation(self, func: str, backend: str | None = None,
                           kwargs: Mapping[str, Any] | None = None) -> Callable:
        if backend:
            if backend not in self._backends:
                raise BackendNotFoundError(backend, self._unavailable.get(backend, "not registered"))
            if backend in self._disabled:
                raise BackendNotFoundError(backend, "disabled")
            if func not in self._caps.get(backend, ()):
                raise BackendNotImplementedError(backend, func)
            if kwargs:
                r = self.validate_backend_for_call(backend, func, kwargs)
                if not r.success:
                    raise NoCapableBackendError(func, {backend: f"{r.failed_param}: {r.failure_reason}"})
            return getattr(self._backends[backend], func)
        return getattr(self._backends[self.get_capable_backend(func, kwargs)], func)

    @contextmanager
    def use_backend(self, name: str):
        if not self.is_available(name):
            reason = self._unavailable.get(name) or ("disabled" if name in self._disabled else "not registered")
            raise BackendNotFoundError(name, reason)
        prev = getattr(self._tls, "override", None)
        self._tls.override = name
        try:
            yield
        finally:
            self._tls.override = prev


registry = BackendRegistry()
