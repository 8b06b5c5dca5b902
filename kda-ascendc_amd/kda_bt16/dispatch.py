"""Per-function backend dispatch for the KDA ops, after flash-linear-attention's
registry as the reference describes it (``docs/KDA_ANALYSIS.md:10, 26-36``:
``fla/ops/backends/__init__.py``'s ``dispatch`` decorator and the backends
of ``fla/ops/kda/backends/__init__.py``, each with a priority, an
availability test and, per dispatched function, a verifier; FlashKDA, for
example, takes over only the top-level ``chunk_kda`` and only for the calls
its verifier accepts).

Here:

* :class:`Backend` -- ``name``, ``priority``, ``is_available()``; an
  implementation is an attribute named after the dispatched function, its
  verifier ``verify_<name>`` returns ``None`` (serve) or a reason (decline);
* :func:`dispatch` -- decorator: a call goes to the available backend of
  highest priority whose verifier accepts it, else to the decorated
  function itself;
* :class:`MI355XKDABackend` -- ``chunk_kda`` / ``fused_recurrent_kda`` of
  :mod:`kda_bt16.fla` on gfx950, registered for op ``"kda"`` on import;
* :func:`install_into_fla` -- when FLA is importable, wrap its public
  ``fla.ops.kda.chunk_kda`` / ``fused_recurrent_kda`` with this dispatch, FLA's
  own function being the fallback.  FLA is not installed in this build's
  environment, so that hook is exercised here only against a stand-in
  module (tests/test_dispatch.py).
"""

from __future__ import annotations

import functools
import inspect
import threading
from typing import Callable

import torch

_registry: dict[str, list] = {}
_lock = threading.Lock()


class Backend:
    """A provider of some dispatched functions."""

    name = "backend"
    priority = 0

    def is_available(self) -> bool:
        return True


def register_backend(op: str, backend: Backend) -> None:
    """Add ``backend`` for ``op`` (replacing one of the same name)."""
    with _lock:
        lst = [b for b in _registry.get(op, []) if b.name != backend.name]
        lst.append(backend)
        lst.sort(key=lambda b: -b.priority)
        _registry[op] = lst


def unregister_backend(op: str, name: str) -> None:
    with _lock:
        _registry[op] = [b for b in _registry.get(op, []) if b.name != name]


def backends(op: str) -> list:
    """The backends of ``op``, highest priority first."""
    with _lock:
        return list(_registry.get(op, []))


def select(op: str, fn_name: str, signature: inspect.Signature, args, kwargs):
    """``(backend, implementation)`` that would serve this call, or
    ``(None, None)``.  Verifiers see every argument by name, positional
    ones bound through ``signature`` (the dispatched function's)."""
    try:
        bound = signature.bind(*args, **kwargs)
    except TypeError:
        return None, None
    named = dict(bound.arguments)
    extra = named.pop(next((p.name for p in signature.parameters.values()
                            if p.kind is inspect.Parameter.VAR_KEYWORD), ""), {}) or {}
    named.update(extra)
    for be in backends(op):
        impl = getattr(be, fn_name, None)
        if impl is None:
            continue
        try:
            if not be.is_available():
                continue
        except Exception:  # an availability probe that fails means unavailable
            continue
        verify = getattr(be, "verify_" + fn_name, None)
        if verify is not None and verify(**named) is not None:
            continue
        return be, impl
    return None, None


def dispatch(op: str, name: str | None = None) -> Callable:
    """Route calls of the decorated function through the backends of ``op``;
    the decorated function is the fallback.  Backends provide it under
    ``name`` (default: the function's ``__name__``)."""

    def deco(fn):
        sig = inspect.signature(fn)
        fn_name = name or fn.__name__

        @functools.wraps(fn)
        def wrapper(*args, **kwargs):
            _, impl = select(op, fn_name, sig, args, kwargs)
            if impl is not None:
                return impl(*args, **kwargs)
            return fn(*args, **kwargs)

        wrapper.__kda_dispatch__ = (op, fn)
        return wrapper

    return deco


class MI355XKDABackend(Backend):
    """The HIP kernels of this package, on AMD gfx950 (MI355X)."""

    name = "mi355x_hip"
    priority = 10  # above FLA's own KDA backends (0-5 in the reference's survey)

    def __init__(self):
        self._available = None

    def is_available(self) -> bool:
        if self._available is None:
            ok = False
            try:
                if torch.cuda.is_available():
                    arch = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")
                    if arch.split(":")[0] == "gfx950":
                        from . import _hip
                        _hip.lib()
                        ok = True
            except Exception:
                ok = False
            self._available = ok
        return self._available

    @staticmethod
    def chunk_kda(*args, **kwargs):
        from .fla import chunk_kda
        return chunk_kda(*args, **kwargs)

    @staticmethod
    def verify_chunk_kda(**named):
        from .fla import verify_chunk_kda
        return verify_chunk_kda(**named)

    @staticmethod
    def fused_recurrent_kda(*args, **kwargs):
        from .fla import fused_recurrent_kda
        return fused_recurrent_kda(*args, **kwargs)

    @staticmethod
    def verify_fused_recurrent_kda(**named):
        from .fla import verify_fused_recurrent_kda
        return verify_fused_recurrent_kda(**named)


MI355X_BACKEND = MI355XKDABackend()
register_backend("kda", MI355X_BACKEND)


def install_into_fla(module=None) -> list[str]:
    """Wrap ``chunk_kda`` and ``fused_recurrent_kda`` of FLA's ``fla.ops.kda``
    (or of ``module``) with :func:`dispatch` over op ``"kda"``, keeping FLA's
    functions as the fallback.  Code that imports them afterwards gets the
    dispatching versions.  Returns the names wrapped; ``[]`` if FLA is not
    importable.  Idempotent."""
    if module is None:
        try:
            import fla.ops.kda as module  # noqa: PLC0415
        except ImportError:
            return []
    done = []
    for name in ("chunk_kda", "fused_recurrent_kda"):
        fn = getattr(module, name, None)
        if fn is None:
            continue
        if getattr(fn, "__kda_dispatch__", None) is None:
            setattr(module, name, dispatch("kda", name)(fn))
        done.append(name)
    return done
