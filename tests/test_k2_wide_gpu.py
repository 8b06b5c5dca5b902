"""Stage 2 with several value tiles per work-group against stage 2 with one
tile per work-group (k2_kernel, csrc/kda_k2.hip), bit for bit: they run the
same arithmetic in the same order (kernels.py:225-302), only the division of
the work differs.

``forward_choice(k2_tiles=...)`` (the ``k2_tiles`` field of the C ABI's
arguments) forces the tiles per work-group (1, 2, 4, 8) over the launch
heuristic, which picks several tiles only when (sequences x heads x 8)
exceeds the CU count.  ``k2_wave_tiles`` picks the kernel for several tiles:
0, the library's choice (a state wave per tile, k2s_kernel in
csrc/kda_k2.hip, at 2 tiles; csrc/kda_k2w.hip's compute waves of one tile
at 4 and of two at 8), or 1 / 2 for kda_k2w.hip's compute waves of that
many tiles.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import forward_choice, kda_bt16_fwd

pytestmark = pytest.mark.gpu

# name, B, T, H, HV, cu_seqlens, state_v_first, h0
CASES = [
    ("one_token", 1, 1, 1, 1, None, True, True),
    ("one_chunk", 1, 16, 1, 2, None, True, True),
    ("partial_T300", 1, 300, 2, 2, None, True, False),
    ("T96_exact", 2, 96, 1, 1, None, True, True),
    ("gva_kfirst_T1037", 2, 1037, 2, 4, None, False, True),
    ("long_T2500", 1, 2500, 1, 1, None, True, True),
    ("varlen_empty", 1, 400, 2, 2, [0, 0, 37, 53, 53, 120, 400], True, True),
    ("varlen_kfirst", 1, 700, 1, 2, [0, 17, 300, 301, 700], False, True),
]


def _inputs(B, T, H, HV, S, seed):
    gen = torch.Generator().manual_seed(seed)
    return dict(
        q=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        k=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        v=torch.randn(B, T, HV, 128, generator=gen).bfloat16(),
        g=torch.randn(B, T, HV, 128, generator=gen).bfloat16(),
        beta=torch.randn(B, T, HV, generator=gen).bfloat16(),
        A_log=torch.log(torch.rand(HV, generator=gen) * 15 + 1),
        dt_bias=torch.randn(HV * 128, generator=gen) * 0.1,
        h0=torch.randn(S, HV, 128, 128, generator=gen) * 0.05,
    )


def _run(c, dev, cu, svf, h0, tiles, wave_tiles=None):
    with forward_choice(k2_tiles=tiles, k2_wave_tiles=wave_tiles or 0):
        init = None
        if h0:
            init = c["h0"] if svf else c["h0"].transpose(-1, -2).contiguous()
            init = init.to(dev)
        o, ht = kda_bt16_fwd(
            *(c[x].to(dev) for x in ("q", "k", "v", "g", "beta")), scale=0.1,
            initial_state=init, output_final_state=True, use_qk_l2norm_in_kernel=True,
            use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, lower_bound=-5.0,
            A_log=c["A_log"].to(dev), dt_bias=c["dt_bias"].to(dev), state_v_first=svf,
            cu_seqlens=None if cu is None else torch.tensor(cu, dtype=torch.int32, device=dev))
        torch.cuda.synchronize()
        return o, ht


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_wide_stage2_equals_one_tile_stage2(case, gpu_device):
    name, B, T, H, HV, cu, svf, h0 = case
    S = B if cu is None else len(cu) - 1
    c = _inputs(B, T, H, HV, S, seed=hash(name) % 1000)
    print(f"[k2 wide] {name}", flush=True)
    o1, ht1 = _run(c, gpu_device, cu, svf, h0, 1)
    assert torch.isfinite(o1.float()).all() and torch.isfinite(ht1).all()
    for tiles in (2, 4, 8):
        for wt in (0, 1, 2):
            o, ht = _run(c, gpu_device, cu, svf, h0, tiles, wt)
            what = f"{name}: {tiles} tiles, {wt} per wave"
            assert torch.equal(o.view(torch.int16), o1.view(torch.int16)), f"{what}: o"
            assert torch.equal(ht.view(torch.int32), ht1.view(torch.int32)), f"{what}: ht"


def test_heuristic_takes_the_wide_kernel_for_many_heads(gpu_device):
    """B=1 T=64 H=96 (768 value tiles) runs several tiles per work-group by
    default and gives the one-tile result."""
    c = _inputs(1, 64, 96, 96, 1, seed=9)
    o1, ht1 = _run(c, gpu_device, None, True, True, 1)
    o, ht = kda_bt16_fwd(
        *(c[x].to(gpu_device) for x in ("q", "k", "v", "g", "beta")), scale=0.1,
        initial_state=c["h0"].to(gpu_device), output_final_state=True,
        use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
        use_beta_sigmoid_in_kernel=True, lower_bound=-5.0, A_log=c["A_log"].to(gpu_device),
        dt_bias=c["dt_bias"].to(gpu_device))
    torch.cuda.synchronize()
    assert torch.equal(o, o1) and torch.equal(ht, ht1)


def test_heuristic_takes_two_tiles_for_forty_heads(gpu_device):
    """B=1 T=200 H=40 (320 value tiles, 2 per work-group by default: the
    state-wave-per-tile kernel) gives the one-tile result, partial last
    chunk included."""
    c = _inputs(1, 200, 40, 40, 1, seed=11)
    o1, ht1 = _run(c, gpu_device, None, True, True, 1)
    o, ht = _run(c, gpu_device, None, True, True, 0)
    assert torch.equal(o, o1) and torch.equal(ht, ht1)
