"""The backend dispatch (kda_bt16.dispatch) and the FLA-convention verifiers
(kda_bt16.fla), on the CPU: selection by priority, availability and
verifier, the fallback, positional-argument binding, and the hook that
wraps an FLA module (a stand-in module here: FLA is not installed)."""

from __future__ import annotations

import types

import pytest
import torch

from kda_bt16 import dispatch
from kda_bt16.fla import chunk_kda, verify_chunk_kda, verify_fused_recurrent_kda

OP = "test_op"


class _Fake(dispatch.Backend):
    def __init__(self, name, priority, available=True, accept=True):
        self.name, self.priority = name, priority
        self._available, self._accept = available, accept
        self.calls = []

    def is_available(self):
        return self._available

    def op_fn(self, x, y=0, **kw):
        self.calls.append((x, y, kw))
        return self.name

    def verify_op_fn(self, x, y=0, **kw):
        return None if self._accept and x >= 0 else "declined"


@dispatch.dispatch(OP)
def op_fn(x, y=0, **kw):
    return "fallback"


@pytest.fixture(autouse=True)
def _clean():
    yield
    for b in dispatch.backends(OP):
        dispatch.unregister_backend(OP, b.name)


def test_fallback_without_backends():
    assert op_fn(1) == "fallback"


def test_highest_priority_available_accepting_backend_wins():
    lo, hi = _Fake("lo", 1), _Fake("hi", 5)
    dispatch.register_backend(OP, lo)
    dispatch.register_backend(OP, hi)
    assert op_fn(1, y=2, z=3) == "hi"
    assert hi.calls == [(1, 2, {"z": 3})]
    # declined by every verifier -> fallback
    assert op_fn(-1) == "fallback"


def test_unavailable_or_declining_backends_are_skipped():
    dispatch.register_backend(OP, _Fake("hi_off", 9, available=False))
    dispatch.register_backend(OP, _Fake("mid_no", 5, accept=False))
    dispatch.register_backend(OP, _Fake("lo", 1))
    assert op_fn(3) == "lo"


def test_reregistering_a_name_replaces_it():
    dispatch.register_backend(OP, _Fake("a", 1))
    dispatch.register_backend(OP, _Fake("a", 7, accept=False))
    assert [b.priority for b in dispatch.backends(OP)] == [7]
    assert op_fn(1) == "fallback"


def test_verifier_sees_positional_arguments_by_name():
    seen = {}

    class Rec(_Fake):
        def verify_op_fn(self, **named):
            seen.update(named)
            return None

    dispatch.register_backend(OP, Rec("rec", 1))
    assert op_fn(4, 5, extra=6) == "rec"
    assert seen == {"x": 4, "y": 5, "extra": 6}


def test_backends_are_looked_up_by_the_installed_name():
    """A wrapped function whose __name__ differs from the name it is
    installed under still reaches the backends' implementation."""

    def some_other_name(x, y=0):
        return "fallback"

    wrapped = dispatch.dispatch(OP, "op_fn")(some_other_name)
    dispatch.register_backend(OP, _Fake("be", 1))
    assert wrapped(2) == "be"


def test_install_into_stand_in_fla_module():
    calls = []

    def chunk_kda_fla(q, k, v, g, beta, scale=None, **kw):
        calls.append("fla")
        return "fla"

    mod = types.SimpleNamespace(chunk_kda=chunk_kda_fla)
    assert dispatch.install_into_fla(mod) == ["chunk_kda"]
    wrapped = mod.chunk_kda
    assert dispatch.install_into_fla(mod) == ["chunk_kda"] and mod.chunk_kda is wrapped
    # On the CPU the MI355X backend is unavailable: FLA's own function serves.
    x = torch.zeros(1, 16, 1, 128, dtype=torch.bfloat16)
    assert mod.chunk_kda(x, x, x, x.float(), x[..., 0].float()) == "fla"
    assert calls == ["fla"]


def test_mi355x_backend_registered_and_unavailable_on_cpu():
    names = [b.name for b in dispatch.backends("kda")]
    assert "mi355x_hip" in names
    assert dispatch.MI355X_BACKEND.is_available() is False


def _t(B=1, T=32, H=2, HV=2, dtype=torch.bfloat16):
    q = torch.randn(B, T, H, 128).to(dtype)
    v = torch.randn(B, T, HV, 128).to(dtype)
    return q, q.clone(), v, torch.randn(B, T, HV, 128), torch.randn(B, T, HV)


def test_verifier_bucket_reasons():
    q, k, v, g, b = _t()
    ok_gate = dict(use_gate_in_kernel=True, lower_bound=-5.0, A_log=torch.zeros(2))
    assert verify_chunk_kda(q, k, v, g, b, **ok_gate) == "tensors are not on a ROCm GPU"
    assert "bfloat16" in verify_chunk_kda(q.float(), k, v, g, b, **ok_gate)
    assert "K=V=128" in verify_chunk_kda(*_t()[:2], v[..., :64], g, b, **ok_gate)
    assert "multiple of H" in verify_chunk_kda(*_t(H=2, HV=3), **ok_gate)
    assert "softplus" in verify_chunk_kda(q, k, v, g, b, use_gate_in_kernel=True, A_log=torch.zeros(2))
    assert "A_log" in verify_chunk_kda(q, k, v, g, b, use_gate_in_kernel=True, lower_bound=-5.0)
    assert "safe_gate" in verify_chunk_kda(q, k, v, g, b)
    assert verify_chunk_kda(q, k, v, g, b, safe_gate=True, lower_bound=-5.0) == \
        "tensors are not on a ROCm GPU"
    assert "intermediate" in verify_chunk_kda(q, k, v, g, b, return_intermediate_states=True, **ok_gate)
    assert "context" in verify_chunk_kda(q, k, v, g, b, cp_context=object(), **ok_gate)
    # autograd is served by chunk_kda (the backward kernels), not by the
    # forward-only token recurrence
    qg = q.clone().requires_grad_(False).float().requires_grad_(True).bfloat16()
    assert verify_chunk_kda(qg, k, v, g, b, **ok_gate) == "tensors are not on a ROCm GPU"
    assert "grad" in verify_fused_recurrent_kda(qg, k, v, g, b)
    # the token recurrence takes an unbounded log decay
    assert verify_fused_recurrent_kda(q, k, v, g, b) == "tensors are not on a ROCm GPU"


def test_chunk_kda_raises_outside_its_bucket():
    q, k, v, g, b = _t()
    with pytest.raises(NotImplementedError, match="softplus"):
        chunk_kda(q, k, v, g, b, use_gate_in_kernel=True, A_log=torch.zeros(2))
    with pytest.raises(NotImplementedError, match="ROCm GPU"):
        chunk_kda(q, k, v, g, b, use_gate_in_kernel=True, lower_bound=-5.0, A_log=torch.zeros(2))
