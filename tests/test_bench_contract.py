"""bench.py off the GPU: the algorithmic bytes and FLOPs its roofline
divides by, against the per-config figures of the scope table, and its
command-line contract (one GPU only; the workload choices).

The table's bytes are 1282 B per token-head (q, k, v, o in bf16, g in
bf16, beta) plus the fp32 initial and final states of every (sequence,
head), 64 KiB each; its FLOPs are those of the four stage-1 and four stage-2
matrix products.  It counts an initial-state read for every config; the
bench counts one only when the config passes an initial state (c2 and c3 do
not), so there its bytes are one state per (sequence, head) lower.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

# config: (MB with an initial state read, GFLOP), as the scope table gives them
TABLE = {
    "c0": (11.55, 0.973),
    "c1": (86.12, 7.785),
    "c2": (340.28, 31.14),
    "c3": (1020.84, 93.42),
    "c4": (1411.40, 124.55),
}
STATE_BYTES = 128 * 128 * 4


@pytest.mark.parametrize("name", sorted(TABLE))
def test_algorithmic_bytes_and_flops_match_the_table(name):
    c = bench.CONFIGS[name]
    b, t, h = c["B"], c["T"], c["H"]
    k1, k2 = bench.algorithmic_bytes(n_states=b, b=b, t=t, h=h, h0=True)
    assert abs((k1 + k2) / 1e6 - TABLE[name][0]) < 0.01, (name, (k1 + k2) / 1e6)
    # without an initial state the bench counts one state less per (sequence, head)
    n1, n2 = bench.algorithmic_bytes(n_states=b, b=b, t=t, h=h, h0=False)
    assert (k1 + k2) - (n1 + n2) == b * h * STATE_BYTES
    f1, f2 = bench.matmul_flops(b=b, t=t, h=h)
    assert abs((f1 + f2) / 1e9 - TABLE[name][1]) < 0.01, (name, (f1 + f2) / 1e9)


def test_headline_bytes_are_the_roofline_rule():
    """The headline line's alg_bytes (B*T*H*1282 + 64 KiB per final state +
    516 B per head of A_log and dt_bias) at B=1 T=8192 H=32, no h0."""
    k1, k2 = bench.algorithmic_bytes()
    B, T, H = bench.B, bench.T, bench.H
    assert k1 + k2 == B * T * H * 1282 + B * H * STATE_BYTES + 516 * H


def test_roofline_is_the_dominant_kernels():
    """achieved = the forward's algorithmic bytes / the longest kernel's
    mean launch time; traffic = that kernel's bytes per launch; the whole
    forward's figures beside them (c2-like numbers, stage 2 the longer)."""
    kern = {"k1": {"ms": 0.118}, "k2": {"ms": 0.150}}
    traffic = {"k1": 558_000_000, "k2": 362_000_000}
    r = bench._dominant_roofline(kern, traffic, 340_000_000, 31_000_000_000, 0.26, False)
    assert r["kernel"].startswith("stage 2")
    assert r["achieved"] == pytest.approx(340e6 / 0.150 / 1e6, rel=1e-4)
    assert r["frac"] == pytest.approx(r["achieved"] / bench.HBM_PEAK_GBS, rel=1e-3)
    assert r["traffic"] == 362_000_000 and r["kernel_ms_events"] == 0.15
    f = r["forward"]
    assert f["achieved"] == pytest.approx(340e6 / 0.26 / 1e6, rel=1e-4)
    assert f["traffic"] == 920_000_000
    # stage 1 the longer (c3-like); no profile: traffic unknown
    kern = {"k1": {"ms": 0.345}, "k2": {"ms": 0.267}}
    r = bench._dominant_roofline(kern, None, 1_020_000_000, 93e9, 0.61, False)
    assert r["kernel"].startswith("stage 1") and r["traffic"] is None
    assert r["forward"]["traffic"] is None
    # fused: one launch, the forward itself
    r = bench._dominant_roofline({"fused": {"ms": 0.5}}, {"fused": 1_430_000_000}, 1_411_000_000,
                                 124e9, 0.5, True)
    assert r["kernel"].startswith("fused_kernel") and r["traffic"] == 1_430_000_000
    assert r["achieved"] == r["forward"]["achieved"]
    # two stages in two chunk ranges: times and traffic per launch, half the
    # algorithmic bytes a launch; the forward's traffic both ranges'
    kern = {"k1": {"ms": 0.060}, "k2": {"ms": 0.075}}
    traffic = {"k1": 279_000_000, "k2": 181_000_000}
    r = bench._dominant_roofline(kern, traffic, 340_000_000, 31e9, 0.25, False, 2)
    assert r["kernel"].startswith("stage 2") and r["launches_per_forward"] == 2
    assert r["achieved"] == pytest.approx(170e6 / 0.075 / 1e6, rel=1e-4)
    assert r["traffic"] == 181_000_000 and r["kernel_ms_events"] == 0.075
    assert r["forward"]["traffic"] == 920_000_000
    assert r["forward"]["achieved"] == pytest.approx(340e6 / 0.25 / 1e6, rel=1e-4)


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def test_workload_choices():
    r = _run("--workload", "nonesuch")
    assert r.returncode == 2 and "invalid choice" in r.stderr
    for w in ("headline", "config", "varlen", "decode", "train", "dispatch"):
        r = _run("--workload", w, "--gpus", "2")
        assert r.returncode == 2 and "invalid choice" not in r.stderr, w
