"""The parity helpers themselves (CPU): the per-row bound catches an error
confined to one row that the aggregate relative norm lets through. The error
is planted in a copy of the oracle's own gradient."""
import pytest
import torch

from memory_efficient_attn_layer_amd.synthetic import Workload, make_inputs
from oracle import block as ob
from tests.parity_util import assert_grad_close, assert_rows_close


def test_a_planted_row_error_fails_the_row_bound():
    w = Workload(99, "plant", 1, 256, 256, 4, 64)
    inp = make_inputs(w)
    ref = ob.block_grads(inp, w.H, w.N, dtype=torch.float32, with_intermediates=True)["inter_grad"]["a_q"]
    bad = ref.clone()
    bad[0, 100, 2] *= 1.3  # one (token, head) row of 1024, 30% off
    assert_grad_close("aggregate", bad, ref)  # within the aggregate tolerance
    with pytest.raises(AssertionError):
        assert_rows_close("planted", bad, ref)


def test_row_bound_accepts_bf16_rounding():
    g = torch.Generator().manual_seed(0)
    ref = torch.randn(512, 64, generator=g)
    ref[7] *= 1e-4  # a nearly cancelled row: judged against the floor
    got = ref.bfloat16().float()
    assert assert_rows_close("bf16", got, ref) < 1e-2


def test_a_planted_error_in_an_early_query_row_fails():
    """The first 16 query rows of da_q are held to the normal row bound against
    the kernel-operand reference: a 10% error in row t = 3 of one head fails
    it, while the aggregate norm of those rows would let it through."""
    from tests.parity_util import early_daq_reference, q_chain
    from tests.test_flash_numerics import simulate_kernel_dq

    w = Workload(99, "plant-early", 1, 64, 256, 4, 64)
    inp = make_inputs(w)
    ref = ob.block_grads(inp, w.H, w.N, dtype=torch.float32, with_intermediates=True)
    it, ig = ref["inter"], ref["inter_grad"]
    B, T, H, N, E = w.B, w.T, w.H, w.N, 16
    hm = lambda t: t.double().reshape(B, T, H, N).permute(0, 2, 1, 3)  # noqa: E731
    dO = hm(ig["o"])
    dq_sim, O_sim = simulate_kernel_dq(hm(it["q"]), hm(it["k"]), hm(it["v"]), dO, N)
    rx = torch.rsqrt(inp["x"].double().pow(2).mean(-1) + 1e-6)
    got = q_chain(it, dq_sim[:, :, :E], inp["f1"], inp["f2"], rx)
    pinned = early_daq_reference(it, dO.bfloat16(), O_sim.permute(0, 2, 1, 3).reshape(B, T, H * N), inp["f1"],
                                 inp["f2"], rx, H, N, E)
    assert assert_rows_close("simulated kernel", got, pinned) < 0.01
    bad = got.clone()
    g = torch.Generator().manual_seed(3)
    d = torch.randn(N, generator=g, dtype=torch.float64)
    bad[0, 2, 3] += 0.1 * got[0, 2, 3].norm() * d / d.norm()  # 10% of row t = 3 of head 2
    assert_grad_close("aggregate", bad, pinned)
    with pytest.raises(AssertionError):
        assert_rows_close("planted t = 3", bad, pinned)
