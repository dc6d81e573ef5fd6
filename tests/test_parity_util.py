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
