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
