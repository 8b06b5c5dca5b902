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


REF_FIXTURES = Path(__file__).resolve().parent / "golden" / "kda_ref_fixtures.npz"


def ref_fixture_cases() -> list[str]:
    """Names of the cases written by tests/golden/make_ref_fixtures.py."""
    return [str(x) for x in np.load(REF_FIXTURES)["cases"]]


def load_ref_fixture(name: str) -> dict:
    """One case of the fixtures the reference's own kernels wrote
    (tests/golden/make_ref_fixtures.py): CPU inputs, the flags, and the
    reference's outputs -- ``g``, ``Aqk``, ``A_inv`` from the Triton
    interpreter as installed, ``w``, ``u``, ``o``, ``ht`` from the run with
    its bf16 dot corrected."""
    z = np.load(REF_FIXTURES)  # plain arrays only; allow_pickle stays False
    p = name + "/"
    c = {key: _bf16(z[p + key]) for key in ("q", "k", "v")}
    c["g"] = torch.from_numpy(z[p + "g"])
    c["beta"] = torch.from_numpy(z[p + "beta"])
    c["A_log"] = torch.from_numpy(z[p + "A_log"])
    c["dt_bias"] = torch.from_numpy(z[p + "dt_bias"])
    c["h0"] = _bf16(z[p + "h0"]).float() if p + "h0" in z else None
    scale, lb, svf, use_gate, l2norm, bsig = z[p + "cfg"].tolist()
    c.update(scale=scale, lower_bound=lb, state_v_first=bool(svf), use_gate=bool(use_gate),
             use_l2norm=bool(l2norm), use_beta_sigmoid=bool(bsig))
    c["ref"] = {
        "g": torch.from_numpy(z[p + "interp/g"]),
        "Aqk": _bf16(z[p + "interp/Aqk"]),
        "A_inv": _bf16(z[p + "interp/A_inv"]),
        "w": _bf16(z[p + "dotfix/w"]),
        "u": _bf16(z[p + "dotfix/u"]),
        "o": _bf16(z[p + "dotfix/o"]),
        "ht": torch.from_numpy(z[p + "dotfix/ht"]),
    }
    return c


def _ordered(bits: torch.Tensor, width: int) -> torch.Tensor:
    """Sign-magnitude float bit patterns -> integers in the floats' order."""
    b = bits.to(torch.int64)
    sign = 1 << (width - 1)
    neg = (b & sign) != 0
    mag = b & (sign - 1)
    return torch.where(neg, -mag, mag)


def ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units in the last place between two tensors of the same
    float type (bf16: rounded to bf16 first, fp32: as is): 0 when the bits
    agree (+0 and -0 agree), 1 for neighbours."""
    if a.dtype == torch.float32 and b.dtype == torch.float32:
        ia = _ordered(a.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF, 32)
        ib = _ordered(b.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF, 32)
    else:
        ia = _ordered(a.to(torch.bfloat16).contiguous().view(torch.int16).to(torch.int64) & 0xFFFF, 16)
        ib = _ordered(b.to(torch.bfloat16).contiguous().view(torch.int16).to(torch.int64) & 0xFFFF, 16)
    return (ia - ib).abs()
