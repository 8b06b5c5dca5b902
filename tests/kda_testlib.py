"""Shared helpers for the test suite: golden fixture loading and error metrics."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "kda_golden.npz"
GOLDEN_CASES = ("state_vfirst", "state_kfirst", "saturated_lb10", "precomputed_g")


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


def load_golden(name: str) -> dict:
    """Inputs (CPU tensors) and fp64-gold outputs of one fixture case."""
    z = np.load(GOLDEN)  # plain arrays only; allow_pickle stays False
    p = name + "/"
    out = {key: _bf16(z[p + key]) for key in ("q", "k", "v")}
    out["g"] = _bf16(z[p + "g_bf16"]) if p + "g_bf16" in z else torch.from_numpy(z[p + "g_f32"])
    out["beta"] = _bf16(z[p + "beta_bf16"])
    out["A_log"] = torch.from_numpy(z[p + "A_log"])
    out["dt_bias"] = torch.from_numpy(z[p + "dt_bias"])
    out["h0"] = torch.from_numpy(z[p + "h0"]) if p + "h0" in z else None
    scale, lb, svf, use_gate = z[p + "cfg"].tolist()
    out.update(scale=scale, lower_bound=lb, state_v_first=bool(svf), use_gate=bool(use_gate))
    out["o_gold"] = torch.from_numpy(z[p + "o_gold"])
    out["ht_gold"] = torch.from_numpy(z[p + "ht_gold"])
    return out


def maxdiff(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def assert_close_rel(name: str, ref: torch.Tensor, got: torch.Tensor, ratio: float) -> None:
    """Relative RMS error check in the style of the reference tests'
    ``assert_close(name, ref, got, ratio)`` (used at tolerances 0.006 / 0.01 /
    0.02 / 0.002 in /root/reference/tests/test_kda_bt16.py:78-200):
    rms(ref - got) / rms(ref) must not exceed ``ratio``, unless the absolute
    error is itself below 1e-6."""
    ref = ref.double().cpu()
    got = got.double().cpu()
    assert torch.isfinite(got).all(), f"{name}: non-finite values"
    diff = (ref - got).abs().max().item()
    err = ((ref - got).pow(2).mean().sqrt() / ref.pow(2).mean().sqrt().clamp_min(1e-30)).item()
    assert diff < 1e-6 or err <= ratio, f"{name}: rms ratio {err:.3e} > {ratio} (max abs {diff:.3e})"
