"""Write the small golden fixtures in ``kda_golden.npz``.

The reference ships no golden vectors for this path (its correctness tests
compare against FLA at run time, /root/reference/tests/test_kda_bt16.py:26-39).
These fixtures freeze seeded inputs together with the outputs of the fp64
token-by-token recurrence (``oracle.kda_oracle.recurrent_gold``), which is
independent of the chunked algorithm under test.  Cases follow the reference
test list: partial last chunk with a non-zero state in both state layouts
(tests/test_kda_bt16.py:108-125, tests/test_torch_reference.py:390-476), the
saturated gate (tests/test_kda_bt16.py:128-171) and a precomputed log2 gate
cumsum (tests/test_kda_bt16.py:203-237).

Run from the repo root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))

from kda_oracle import BT, RCP_LN2, make_inputs, recurrent_gold  # noqa: E402

OUT = Path(__file__).resolve().parent / "kda_golden.npz"


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _cases():
    # 1) partial chunk, non-zero state, V-first and K-first
    inp = make_inputs(1, 37, 2, seed=7, h0_std=0.05)
    for name, svf in (("state_vfirst", True), ("state_kfirst", False)):
        h0 = inp["h0"] if svf else inp["h0"].transpose(-1, -2).contiguous()
        yield name, inp, dict(scale=0.1, lower_bound=-5.0, state_v_first=svf, h0=h0,
                              use_gate=True)
    # 2) saturated gate: A_log = 0, dt_bias = 0, g = 20, lower_bound = -10
    sat = make_inputs(1, 48, 2, seed=42)
    sat["A_log"] = torch.zeros(2)
    sat["dt_bias"] = torch.zeros(2 * 128)
    sat["g"] = torch.full((1, 48, 2, 128), 20.0).to(torch.bfloat16)
    yield "saturated_lb10", sat, dict(scale=0.1, lower_bound=-10.0, state_v_first=True, h0=None,
                                      use_gate=True)
    # 3) precomputed chunk-local log2 cumsum, no in-kernel gate
    pre = make_inputs(1, 40, 2, seed=11)
    gg = pre["g"].float() + pre["dt_bias"].view(1, 1, 2, 128)
    gate = -5.0 * torch.sigmoid(torch.exp(pre["A_log"]).view(1, 1, 2, 1) * gg)
    G = torch.zeros_like(gate)
    for c0 in range(0, 40, BT):
        G[:, c0:c0 + BT] = torch.cumsum(gate[:, c0:c0 + BT], dim=1) * RCP_LN2
    pre["g"] = G
    yield "precomputed_g", pre, dict(scale=0.1, lower_bound=-5.0, state_v_first=True, h0=None,
                                     use_gate=False)


def main() -> None:
    arrays = {}
    for name, inp, cfg in _cases():
        o, ht = recurrent_gold(
            inp["q"], inp["k"], inp["v"], inp["g"].float(), inp["beta"].float(), cfg["scale"],
            A_log=inp["A_log"], dt_bias=inp["dt_bias"], lower_bound=cfg["lower_bound"],
            initial_state=cfg["h0"], state_v_first=cfg["state_v_first"],
            use_gate=cfg["use_gate"], dtype=torch.float64,
        )
        p = name + "/"
        for key in ("q", "k", "v"):
            arrays[p + key] = _bf16_bits(inp[key])
        g = inp["g"]
        arrays[p + ("g_bf16" if g.dtype == torch.bfloat16 else "g_f32")] = (
            _bf16_bits(g) if g.dtype == torch.bfloat16 else g.numpy().astype(np.float32))
        arrays[p + "beta_bf16"] = _bf16_bits(inp["beta"])
        arrays[p + "A_log"] = inp["A_log"].numpy().astype(np.float32)
        arrays[p + "dt_bias"] = inp["dt_bias"].numpy().astype(np.float32)
        if cfg["h0"] is not None:
            arrays[p + "h0"] = cfg["h0"].numpy().astype(np.float32)
        arrays[p + "cfg"] = np.array([cfg["scale"], cfg["lower_bound"],
                                      float(cfg["state_v_first"]), float(cfg["use_gate"])])
        arrays[p + "o_gold"] = o.numpy().astype(np.float32)
        arrays[p + "ht_gold"] = ht.numpy().astype(np.float32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
