"""The built library keeps every MFMA accumulation chain in one shape.

On gfx950 an MFMA accumulating onto the result of an MFMA of the other
shape (16x16x16 <-> 16x16x32 bf16) fewer than 5 wait states later reads two
stale accumulator registers, and the compiler inserts no wait there.  This
was the cause of wrong gradients for one-chunk sequences: the backward's
dv_new chain began with a 16x16x16 product that the first 16x16x32 product
accumulated onto with no instruction between them.  CPU-only: it reads the
library's gfx950 machine code (tests/isa_check.py).
"""

from __future__ import annotations

import pytest

import isa_check
from kda_bt16 import _build

pytestmark = pytest.mark.skipif(not isa_check.tools_available(), reason="ROCm LLVM tools not found")


def _listing(lines: str):
    """A disassembly in llvm-objdump's format from instruction lines (one
    instruction a line, 4 bytes each, from 0x1000; "-> k+0xN" names a
    branch target)."""
    out = ["0000000000001000 <k>:"]
    for n, line in enumerate(lines.strip().splitlines()):
        ins, _, target = line.partition("->")
        tail = f" <{target.strip()}>" if target else ""
        out.append(f"\t{ins.strip():60s}// {0x1000 + 4 * n:012X}: 00000000{tail}")
    return "\n".join(out)


def test_checker_finds_a_planted_pair_and_respects_wait_states():
    near = _listing("""
        v_mfma_f32_16x16x16_bf16 v[8:11], v[2:3], v[4:5], 0
        v_mfma_f32_16x16x32_bf16 v[8:11], v[12:15], v[16:19], v[8:11]
        s_endpgm""")
    bad = isa_check.check(isa_check.parse(near)[0])
    assert len(bad) == 1 and bad[0].waits == 0
    # the other order, partial overlap of SrcC, through a taken branch
    other = _listing("""
        v_mfma_f32_16x16x32_bf16 v[8:11], v[12:15], v[16:19], 0
        s_branch 1 -> k+0xc
        s_nop 7
        v_mfma_f32_16x16x16_bf16 v[10:13], v[2:3], v[4:5], v[10:13]
        s_endpgm""")
    bad = isa_check.check(isa_check.parse(other)[0])
    assert len(bad) == 1 and bad[0].waits == 1
    far = _listing("""
        v_mfma_f32_16x16x16_bf16 v[8:11], v[2:3], v[4:5], 0
        s_nop 7
        v_mfma_f32_16x16x32_bf16 v[8:11], v[12:15], v[16:19], v[8:11]
        s_endpgm""")
    assert not isa_check.check(isa_check.parse(far)[0])
    same = _listing("""
        v_mfma_f32_16x16x32_bf16 v[8:11], v[2:5], v[4:7], 0
        v_mfma_f32_16x16x32_bf16 v[8:11], v[12:15], v[16:19], v[8:11]
        s_endpgm""")
    assert not isa_check.check(isa_check.parse(same)[0])


def test_library_has_no_mixed_shape_accumulation():
    lib = _build.LIB_PATH if hasattr(_build, "LIB_PATH") else None
    if lib is None or not lib.exists():
        pytest.skip("library not built")
    n, bad = isa_check.check_library(str(lib))
    assert n > 1000, f"only {n} MFMAs found: the disassembly did not cover the kernels"
    assert not bad, "\n".join(str(v) for v in bad[:10])


def test_no_kernel_uses_scratch():
    """Every kernel of the built library keeps its state in registers and
    LDS: no private (scratch) segment, which register spills and
    non-inlined calls would need.  A non-inlined helper in the fused kernel
    once gave it 688 bytes of scratch per lane and made it ~3x slower with
    the same results; this catches such a change on the CPU."""
    res = isa_check.kernel_resources(str(_build.LIB_PATH))
    assert len(res) >= 30, sorted(res)
    assert any("fused_kernel" in n for n in res) and any("k2_kernel" in n for n in res)
    spill = {n: r["scratch"] for n, r in res.items() if r["scratch"]}
    assert not spill, spill
