"""Host-side contract of kda_bt16_fwd / kda_bt16_debug (CPU only).

Messages and exception types follow _validate_kda_inputs,
/root/reference/src/kda_bt16/kernels.py:609-749; the first three cases are
the reference's own test_kda_bt16_input_validation
(/root/reference/tests/test_torch_reference.py:354-387).
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import (
    kda_bt16_debug,
    kda_bt16_fwd,
    kda_bt16_kernel_fused,
    kda_decode_step,
    kda_recurrent_fwd,
)

B, T, H, D = 1, 32, 2, 128


def _inputs():
    q = torch.randn(B, T, H, D, dtype=torch.bfloat16)
    k = torch.randn(B, T, H, D, dtype=torch.bfloat16)
    v = torch.randn(B, T, H, D, dtype=torch.bfloat16)
    g = torch.randn(B, T, H, D, dtype=torch.float32)
    beta = torch.randn(B, T, H, dtype=torch.float32)
    return q, k, v, g, beta


@pytest.mark.parametrize("fn", [kda_bt16_fwd, kda_bt16_debug])
def test_reference_validation_cases(fn):
    q, k, v, g, beta = _inputs()
    with pytest.raises(ValueError, match="q must be contiguous"):
        fn(q.transpose(1, 2), k, v, g, beta, scale=0.0883)
    with pytest.raises(TypeError, match="k must be bfloat16"):
        fn(q, k.float(), v, g, beta, scale=0.0883)
    v_wrong = torch.randn(B, T, H, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="prototype targets K=V=128"):
        fn(q, k, v_wrong, g, beta, scale=0.0883)


def test_shape_and_rank_errors():
    q, k, v, g, beta = _inputs()
    with pytest.raises(ValueError, match="q must be 4D"):
        kda_bt16_fwd(q[0], k, v, g, beta)
    with pytest.raises(ValueError, match="beta must be 3D"):
        kda_bt16_fwd(q, k, v, g, beta[..., None])
    with pytest.raises(ValueError, match="q dimensions must be positive"):
        kda_bt16_fwd(q[:, :0], k[:, :0], v[:, :0], g[:, :0], beta[:, :0])
    with pytest.raises(ValueError, match="k.shape"):
        kda_bt16_fwd(q, k[:, :16], v, g, beta)
    with pytest.raises(ValueError, match="g.shape"):
        kda_bt16_fwd(q, k, v, g[:, :16], beta)
    with pytest.raises(ValueError, match="beta.shape"):
        kda_bt16_fwd(q, k, v, g, beta[:, :16])
    with pytest.raises(ValueError, match="beta must be contiguous"):
        kda_bt16_fwd(q, k, v, g, beta.transpose(1, 2).contiguous().transpose(1, 2))


def test_dtype_errors():
    q, k, v, g, beta = _inputs()
    with pytest.raises(TypeError, match="q must be bfloat16"):
        kda_bt16_fwd(q.half(), k, v, g, beta)
    with pytest.raises(TypeError, match="v must be bfloat16"):
        kda_bt16_fwd(q, k, v.float(), g, beta)
    with pytest.raises(TypeError, match="g must be float32 when use_gate_in_kernel=True"):
        kda_bt16_fwd(q, k, v, g.half(), beta, use_gate_in_kernel=True, A_log=torch.zeros(H))
    with pytest.raises(TypeError, match="beta must be float32 or bfloat16"):
        kda_bt16_fwd(q, k, v, g, beta.double())
    with pytest.raises(TypeError, match="beta must be float32 or bfloat16"):
        kda_bt16_fwd(q, k, v, g, beta.half())


def test_g_of_any_float_dtype_without_the_in_kernel_gate():
    """kernels.py:673-674: only the in-kernel gate restricts g's dtype; the
    kernels widen any other g to fp32.  Validation passes, and these CPU
    tensors are then refused by the GPU check."""
    q, k, v, g, beta = _inputs()
    for dt in (torch.float16, torch.float64, torch.bfloat16):
        with pytest.raises(ValueError, match="runs on a ROCm GPU"):
            kda_bt16_fwd(q, k, v, g.to(dt), beta)
    # bf16 beta is accepted too (a superset of the reference's fp32)
    with pytest.raises(ValueError, match="runs on a ROCm GPU"):
        kda_bt16_fwd(q, k, v, g, beta.bfloat16())


def test_state_and_gate_parameter_errors():
    q, k, v, g, beta = _inputs()
    h0 = torch.zeros(B, H, D, D)
    with pytest.raises(TypeError, match="initial_state must be float32"):
        kda_bt16_fwd(q, k, v, g, beta, initial_state=h0.bfloat16())
    with pytest.raises(ValueError, match="initial_state.shape"):
        kda_bt16_fwd(q, k, v, g, beta, initial_state=torch.zeros(B, H, D, 64))
    with pytest.raises(ValueError, match="initial_state must be contiguous"):
        kda_bt16_fwd(q, k, v, g, beta, initial_state=h0.transpose(-1, -2))
    with pytest.raises(ValueError, match="A_log.shape"):
        kda_bt16_fwd(q, k, v, g, beta, A_log=torch.zeros(H + 1))
    with pytest.raises(TypeError, match="A_log must be float32"):
        kda_bt16_fwd(q, k, v, g, beta, A_log=torch.zeros(H, dtype=torch.float64))
    with pytest.raises(ValueError, match="dt_bias.shape"):
        kda_bt16_fwd(q, k, v, g, beta, dt_bias=torch.zeros(H))
    with pytest.raises(ValueError, match="use_gate_in_kernel requires safe_gate=True"):
        kda_bt16_fwd(q, k, v, g, beta, use_gate_in_kernel=True, safe_gate=False, A_log=torch.zeros(H))
    with pytest.raises(ValueError, match="lower_bound must be in range"):
        kda_bt16_fwd(q, k, v, g, beta, use_gate_in_kernel=True, lower_bound=-11.0, A_log=torch.zeros(H))
    with pytest.raises(ValueError, match="lower_bound must be in range"):
        kda_bt16_fwd(q, k, v, g, beta, use_gate_in_kernel=True, lower_bound=0.0, A_log=torch.zeros(H))
    with pytest.raises(ValueError, match="use_gate_in_kernel requires A_log"):
        kda_bt16_fwd(q, k, v, g, beta, use_gate_in_kernel=True)


def test_grouped_value_heads():
    """HV a multiple of H is accepted (the reference rejects HV != H,
    kernels.py:729-730); anything else is refused."""
    q, k, v, g, beta = _inputs()
    v2 = torch.randn(B, T, 2 * H, D, dtype=torch.bfloat16)
    g2 = torch.randn(B, T, 2 * H, D)
    b2 = torch.randn(B, T, 2 * H)
    with pytest.raises(ValueError, match="ROCm GPU"):
        kda_bt16_fwd(q, k, v2, g2, b2)
    v3 = torch.randn(B, T, 3, D, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HV must be a multiple of H"):
        kda_bt16_fwd(q, k, v3, torch.randn(B, T, 3, D), torch.randn(B, T, 3))


def test_varlen_contract():
    """cu_seqlens: FLA's varlen convention and messages."""
    q, k, v, g, beta = _inputs()
    cu = torch.tensor([0, 5, 32], dtype=torch.int64)
    with pytest.raises(ValueError, match="ROCm GPU"):
        kda_bt16_fwd(q, k, v, g, beta, cu_seqlens=cu)
    with pytest.raises(ValueError, match="ROCm GPU"):
        kda_bt16_fwd(q, k, v, g, beta, cu_seqlens=cu.int(),
                     initial_state=torch.zeros(2, H, D, D))
    with pytest.raises(ValueError, match="The batch size is expected to be 1"):
        kda_bt16_fwd(*(torch.cat([x, x]) for x in (q, k, v, g, beta)), cu_seqlens=cu)
    with pytest.raises(ValueError, match="number of initial states"):
        kda_bt16_fwd(q, k, v, g, beta, cu_seqlens=cu, initial_state=torch.zeros(1, H, D, D))
    with pytest.raises(TypeError, match="cu_seqlens must be int32 or int64"):
        kda_bt16_fwd(q, k, v, g, beta, cu_seqlens=cu.float())
    with pytest.raises(ValueError, match="cu_seqlens must be 1D"):
        kda_bt16_fwd(q, k, v, g, beta, cu_seqlens=cu[:1])
    with pytest.raises(ValueError, match="number of initial states"):
        kda_recurrent_fwd(q, k, v, g, beta, cu_seqlens=cu, initial_state=torch.zeros(3, H, D, D))


def test_valid_cpu_inputs_are_refused_before_launch():
    """Valid shapes on the CPU: refused with a clear error, no launch and no
    CPU fallback."""
    q, k, v, g, beta = _inputs()
    with pytest.raises(ValueError, match="ROCm GPU"):
        kda_bt16_fwd(q, k, v, g, beta, use_gate_in_kernel=True, A_log=torch.zeros(H))


def test_bf16_gate_and_beta_are_accepted_by_validation():
    q, k, v, g, beta = _inputs()
    with pytest.raises(ValueError, match="ROCm GPU"):
        kda_bt16_fwd(q, k, v, g.bfloat16(), beta.bfloat16(), use_gate_in_kernel=True,
                     A_log=torch.zeros(H))


def test_fused_kernel_symbol_raises():
    with pytest.raises(NotImplementedError):
        kda_bt16_kernel_fused()


def _gva_inputs(HV):
    q, k, _, _, _ = _inputs()
    v = torch.randn(B, T, HV, D, dtype=torch.bfloat16)
    g = torch.randn(B, T, HV, D)
    beta = torch.randn(B, T, HV)
    return q, k, v, g, beta


def test_recurrent_accepts_grouped_value_heads():
    """kda_recurrent_fwd takes HV a multiple of H; valid CPU inputs are then
    refused only for want of a GPU."""
    q, k, v, g, beta = _gva_inputs(2 * H)
    with pytest.raises(ValueError, match="ROCm GPU"):
        kda_recurrent_fwd(q, k, v, g, beta, use_gate_in_kernel=True, A_log=torch.zeros(2 * H))
    with pytest.raises(ValueError, match="A_log.shape"):
        kda_recurrent_fwd(q, k, v, g, beta, use_gate_in_kernel=True, A_log=torch.zeros(H))
    q3, k3, v3, g3, b3 = _gva_inputs(3)
    with pytest.raises(ValueError, match="HV must be a multiple of H"):
        kda_recurrent_fwd(q3, k3, v3, g3, b3)


def test_recurrent_host_errors():
    q, k, v, g, beta = _inputs()
    with pytest.raises(TypeError, match="output_dtype"):
        kda_recurrent_fwd(q, k, v, g, beta, output_dtype=torch.float16)
    with pytest.raises(ValueError, match="inplace_final_state requires initial_state"):
        kda_recurrent_fwd(q, k, v, g, beta, inplace_final_state=True)
    with pytest.raises(ValueError, match="initial_state.shape"):
        kda_decode_step(q[:, :1], k[:, :1], v[:, :1], g[:, :1], beta[:, :1],
                        torch.zeros(B, H, D, 64))
    with pytest.raises(ValueError, match="ROCm GPU"):
        kda_decode_step(q[:, :1], k[:, :1], v[:, :1], g[:, :1], beta[:, :1],
                        torch.zeros(B, H, D, D))


def test_max_seqlen_is_checked_before_the_device():
    """The varlen hint: a non-negative int or None (chunk_kda's max_seqlen)."""
    q, k, v, g, beta = _inputs()
    for bad in (-1, 3.5, "16"):
        with pytest.raises(ValueError, match="max_seqlen must be a non-negative int or None"):
            kda_bt16_fwd(q, k, v, g, beta, max_seqlen=bad)
    with pytest.raises(ValueError, match="ROCm GPU"):
        kda_bt16_fwd(q, k, v, g, beta, max_seqlen=16)


def test_forward_choice_rejects_unknown_widths():
    from kda_bt16 import forward_choice

    for kw, msg in ((dict(k2_tiles=3), "k2_tiles must be 0, 1, 2, 4 or 8"),
                    (dict(k2_tiles=16), "k2_tiles must be 0, 1, 2, 4 or 8"),
                    (dict(k2_wave_tiles=4), "k2_wave_tiles must be 0, 1 or 2")):
        with pytest.raises(ValueError, match=msg):
            with forward_choice(**kw):
                pass


def test_forward_choice_reaches_the_abi_arguments():
    """forward_choice sets the ABI 4 flags and fields of the arguments the
    forward passes on (built here from CPU tensors; nothing is launched),
    nests, restores the enclosing choice, and is per thread."""
    import threading

    from kda_bt16 import _hip, forward_choice
    from kda_bt16.kernels import _make_args

    q, k, v, g, beta = _inputs()

    def args(flags=0):
        return _make_args(q, k, v, g, beta, 0.088, -5.0, None, None, None, None, None, None, 0,
                          flags)

    a = args()
    assert not a.flags & (_hip.FUSED_KERNEL | _hip.TWO_STAGE) and a.k2_tiles == a.k2_wave_tiles == 0
    with forward_choice(fused=False, k2_tiles=4, k2_wave_tiles=1):
        a = args()
        assert a.flags & _hip.TWO_STAGE and not a.flags & _hip.FUSED_KERNEL
        assert (a.k2_tiles, a.k2_wave_tiles) == (4, 1)
        # use_fused_kernel=True (the flag) wins over fused=False
        a = args(_hip.FUSED_KERNEL)
        assert a.flags & _hip.FUSED_KERNEL and not a.flags & _hip.TWO_STAGE
        with forward_choice(fused=True):
            a = args()
            assert a.flags & _hip.FUSED_KERNEL and not a.flags & _hip.TWO_STAGE
            assert (a.k2_tiles, a.k2_wave_tiles) == (0, 0)
        a = args()
        assert a.flags & _hip.TWO_STAGE and a.k2_tiles == 4
        seen = []
        t = threading.Thread(target=lambda: seen.append(args()))
        t.start()
        t.join()
        assert not seen[0].flags & (_hip.FUSED_KERNEL | _hip.TWO_STAGE)
        assert seen[0].k2_tiles == 0
    a = args()
    assert not a.flags & (_hip.FUSED_KERNEL | _hip.TWO_STAGE) and a.k2_tiles == 0
