"""``torch.library`` registration of the ``ayaka::*`` operators.

Same operator names, schemas and ``out=`` convention as the reference's
``custom_op`` (``python/ayaka/kernel/ops.py:278-442``): an operator with an
optional ``out`` argument is registered twice,

* ``ayaka::<name>`` -- functional, rejects a non-None ``out``;
* ``ayaka::<name>_out`` -- returns nothing and mutates ``out``,

and the :class:`OpHandle` routes a call to one or the other, so ``torch.compile``
sees a correct alias/mutation contract. Every operator gets a meta (fake) kernel.

Differences from the reference, on purpose:

* There is no reference mode. The reference can route any op to its plain-torch
  oracle (``AYAKA_FORCE_REFERENCE_OPS`` / ``force_reference``); this package has a
  single implementation per op, the HIP kernel, so setting the variable or entering
  ``force_reference`` raises :class:`CapabilityError` instead of silently running
  something else. Parity checking lives in the test-suite (:func:`verify_against`
  takes the checker explicitly).
* Dispatcher failures (no kernel for the tensor's backend, e.g. a CPU tensor) are
  rewritten to :class:`CapabilityError`, as the reference does (``ops.py:132-148``).
"""

from __future__ import annotations

import contextlib
import functools
import inspect
import os
from collections.abc import Callable, Generator
from typing import Any

import torch
import torch.library

from ayaka.utils.import_utils import CapabilityError

__all__ = ["OpHandle", "custom_op", "force_reference", "registered_ops", "verify_against"]

_LIBRARIES: dict[str, torch.library.Library] = {}
_REGISTRY: dict[str, OpHandle] = {}


def _library(namespace: str) -> torch.library.Library:
    lib = _LIBRARIES.get(namespace)
    if lib is None:
        # Kept alive for the process lifetime: dropping it unregisters the ops.
        lib = torch.library.Library(namespace, "FRAGMENT")
        _LIBRARIES[namespace] = lib
    return lib


def _reference_requested() -> bool:
    return os.environ.get("AYAKA_FORCE_REFERENCE_OPS", "0").lower() in ("1", "true", "yes")


class OpHandle:
    """A registered operator: callable like the Python function it wraps."""

    def __init__(self, *, name: str, namespace: str, kernel: Callable[..., Any], mutates_args: list[str]) -> None:
        self.name = name
        self.namespace = namespace
        self.kernel = kernel
        self.mutates_args = mutates_args
        self.qualified = f"{namespace}::{name}"
        self._dispatch: Callable[..., Any] | None = None
        functools.update_wrapper(self, kernel)

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        if _reference_requested():
            raise CapabilityError(
                f"reference::{self.name}",
                detail="this package has no plain-torch reference mode; every op runs its HIP kernel",
                remedy="unset AYAKA_FORCE_REFERENCE_OPS",
            )
        assert self._dispatch is not None
        try:
            return self._dispatch(*args, **kwargs)
        except NotImplementedError as exc:
            raise CapabilityError(
                self.qualified,
                detail=f"kernel is unavailable for these inputs: {exc}",
                remedy="pass CUDA (HIP) tensors on an MI355X (gfx950) device",
            ) from exc
        except RuntimeError as exc:
            msg = str(exc)
            if "Could not run" in msg or "no kernel image" in msg.lower():
                raise CapabilityError(
                    self.qualified,
                    detail=f"kernel is unavailable for these inputs: {msg.splitlines()[0]}",
                    remedy="pass CUDA (HIP) tensors on an MI355X (gfx950) device",
                ) from exc
            raise

    def __repr__(self) -> str:
        return f"<OpHandle {self.qualified}>"


def _define(lib: torch.library.Library, name: str, fn: Callable[..., Any], mutates: list[str],
            fake: Callable[..., Any], dispatch_key: str) -> None:
    ns_ops = getattr(torch.ops, lib.ns)
    if hasattr(ns_ops, name):  # already registered in this process
        return
    schema = torch.library.infer_schema(fn, mutates_args=mutates)
    lib.define(name + schema)
    lib.impl(name, fn, dispatch_key)
    lib._register_fake(name, fake)


def custom_op(
    *,
    name: str,
    fake_impl: Callable[..., Any],
    mutates_args: list[str] | None = None,
    namespace: str = "ayaka",
    dispatch_key: str = "CUDA",
) -> Callable[[Callable[..., Any]], OpHandle]:
    """Register the decorated function as ``<namespace>::<name>``.

    ``fake_impl`` is the meta kernel. ``mutates_args=["out"]`` with an optional
    ``out`` parameter produces the functional / ``_out`` pair described above.
    """
    mutations = list(mutates_args or [])

    def decorator(fn: Callable[..., Any]) -> OpHandle:
        lib = _library(namespace)
        handle = OpHandle(name=name, namespace=namespace, kernel=fn, mutates_args=mutations)
        sig = inspect.signature(fn)
        optional_out = mutations == ["out"] and "out" in sig.parameters and sig.parameters["out"].default is None
        if optional_out:
            out_index = list(sig.parameters).index("out")

            def void_impl(*args: Any, **kwargs: Any) -> None:
                fn(*args, **kwargs)

            void_impl.__signature__ = sig.replace(return_annotation=None)  # type: ignore[attr-defined]

            def functional_impl(*args: Any, **kwargs: Any) -> Any:
                if (args[out_index] if len(args) > out_index else kwargs.get("out")) is not None:
                    raise ValueError("use the public OpHandle for out= dispatch")
                return fn(*args, **kwargs)

            functional_impl.__signature__ = sig  # type: ignore[attr-defined]
            _define(lib, name + "_out", void_impl, mutations, lambda *a, **k: None, dispatch_key)
            _define(lib, name, functional_impl, [], fake_impl, dispatch_key)
            void_op = getattr(getattr(torch.ops, namespace), name + "_out")
            functional_op = getattr(getattr(torch.ops, namespace), name)

            def dispatch(*args: Any, **kwargs: Any) -> Any:
                out = args[out_index] if len(args) > out_index else kwargs.get("out")
                if out is None:
                    return functional_op(*args, **kwargs)
                void_op(*args, **kwargs)
                return out

            handle._dispatch = dispatch
        else:
            _define(lib, name, fn, mutations, fake_impl, dispatch_key)
            handle._dispatch = getattr(getattr(torch.ops, namespace), name)
        _REGISTRY[name] = handle
        return handle

    return decorator


def registered_ops() -> dict[str, OpHandle]:
    """Every operator registered so far."""
    return dict(_REGISTRY)


@contextlib.contextmanager
def force_reference(*names: str) -> Generator[None, None, None]:
    """Not supported: there is no reference implementation to route to."""
    raise CapabilityError(
        "reference mode",
        detail="this package has no plain-torch reference mode; every op runs its HIP kernel",
        remedy="compare against an explicit checker with verify_against(op, reference, ...)",
    )
    yield  # pragma: no cover


def verify_against(
    op: str | OpHandle,
    reference: Callable[..., Any],
    *args: Any,
    rtol: float = 1e-3,
    atol: float = 1e-3,
    **kwargs: Any,
) -> None:
    """Run ``op`` and an explicit ``reference`` on cloned inputs and compare.

    Same tolerance rule as the reference's ``verify_against_reference``
    (``ops.py:507-631``): ``|kernel - reference| <= atol + rtol * |reference|``,
    NaN positions must agree. Raises ``AssertionError`` naming the worst element.
    """
    handle = _REGISTRY[op] if isinstance(op, str) else op

    def clone(v: Any) -> Any:
        return v.clone() if isinstance(v, torch.Tensor) else v

    expected = reference(*[clone(a) for a in args], **{k: clone(v) for k, v in kwargs.items()})
    actual = handle(*[clone(a) for a in args], **{k: clone(v) for k, v in kwargs.items()})
    _compare_nested(expected, actual, rtol, atol, handle.name)


def _compare_nested(expected: Any, actual: Any, rtol: float, atol: float, label: str) -> None:
    if isinstance(expected, (tuple, list)):
        if not isinstance(actual, (tuple, list)) or len(actual) != len(expected):
            raise AssertionError(f"{label}: output structure differs")
        for i, (e, a) in enumerate(zip(expected, actual)):
            _compare_nested(e, a, rtol, atol, f"{label}[{i}]")
        return
    e = expected.detach().float().cpu()
    a = actual.detach().float().cpu()
    if e.shape != a.shape:
        raise AssertionError(f"{label}: shape {tuple(a.shape)} != reference {tuple(e.shape)}")
    nan_mismatch = torch.isnan(e) ^ torch.isnan(a)
    if nan_mismatch.any():
        raise AssertionError(f"{label}: NaN in one output but not the other at {int(nan_mismatch.sum())} positions")
    finite = torch.isfinite(e) & torch.isfinite(a)
    diff = torch.where(finite, (e - a).abs(), torch.zeros_like(e))
    bad = diff > atol + rtol * e.abs()
    if bad.any():
        worst = int(diff.argmax())
        raise AssertionError(
            f"{label}: {int(bad.sum())}/{diff.numel()} elements exceed tolerance "
            f"(rtol={rtol}, atol={atol}); worst at {worst}: reference "
            f"{e.flatten()[worst].item():.6g} vs kernel {a.flatten()[worst].item():.6g}"
        )
