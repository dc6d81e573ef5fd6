"""Pins the YaRN table builder (yarn.py) against what YaRN's "NTK-by-parts"
interpolation fixes in closed form (Peng et al. 2023, "YaRN: Efficient
Context Window Extension of Large Language Models", eqs. for gamma and h):

  * dimension i has wavelength lambda_i = 2 pi / theta_i and makes
    r_i = L0 / lambda_i turns over the original context L0;
  * r_i > beta (high frequency): the frequency is kept;
  * r_i < alpha (low frequency): the frequency is divided by the scale s;
  * in between: a blend whose share of the kept frequency grows with r_i;
  * attention temperature m = 0.1 ln s + 1 multiplies both tables.

The region boundaries below are solved by hand from theta_i =
base^(-2i/N): r_i > beta  <=>  i < (N/2) ln(L0 / (2 pi beta)) / ln(base),
so a swapped alpha/beta, a ramp running the wrong way or a misplaced 2 pi
moves them.
"""
import math

import pytest
import torch

from memory_efficient_attn_layer_amd.yarn import rotary_tables, yarn_frequencies, yarn_mscale


def _bounds(N, base, L0, alpha=1.0, beta=32.0):
    """(last index kept, first index fully interpolated), solved in closed form."""
    half = N / 2
    i_keep = half * math.log(L0 / (2 * math.pi * beta)) / math.log(base)   # r_i = beta
    i_interp = half * math.log(L0 / (2 * math.pi * alpha)) / math.log(base)  # r_i = alpha
    return math.ceil(i_keep) - 1, math.floor(i_interp) + 1


@pytest.mark.parametrize("N,s,L0", [(64, 4.0, 8192), (128, 8.0, 16384), (64, 8.0, 2048)],
                         ids=["long-context-s4", "prefill-s8", "n64-s8-short"])
def test_ntk_by_parts_regions(N, s, L0):
    base = 10000.0
    th = torch.tensor([base ** (-2.0 * i / N) for i in range(N // 2)], dtype=torch.float64)
    got = yarn_frequencies(N, base, s, L0)
    last_keep, first_interp = _bounds(N, base, L0)
    assert 0 <= last_keep < first_interp <= N // 2
    # s=4 over 8192 at N=64: dims 0..12 kept, 25..31 interpolated.
    if (N, s, L0) == (64, 4.0, 8192):
        assert (last_keep, first_interp) == (12, 25)
    for i in range(N // 2):
        if i <= last_keep:
            assert got[i] == th[i], i
        elif i >= first_interp:
            assert torch.isclose(got[i], th[i] / s, rtol=1e-14, atol=0), i
        else:
            assert th[i] / s < got[i] < th[i], i
    # Share of the kept frequency: 1 above beta, falling to 0 below alpha,
    # monotone in i (r_i decreases with i).
    share = ((got - th / s) / (th - th / s)).tolist()
    assert all(a >= b for a, b in zip(share, share[1:]))
    assert share[0] == 1.0 and share[-1] == 0.0


def test_temperature_and_table_layout():
    assert yarn_mscale(1.0) == 1.0
    assert math.isclose(yarn_mscale(4.0), 1.1386294361119891, rel_tol=1e-15)
    assert math.isclose(yarn_mscale(8.0), 1.2079441541679836, rel_tol=1e-15)
    N, T, s, L0 = 64, 40, 4.0, 16
    f1, f2 = rotary_tables(T, N, scale=s, original_context=L0, dtype=torch.float64)
    th = yarn_frequencies(N, 10000.0, s, L0)
    m = yarn_mscale(s)
    t = torch.arange(T, dtype=torch.float64)[:, None]
    # Adjacent pairs (fast_triton_attn.py:132-141): f1 = m cos, f2 = (-m sin, +m sin).
    assert torch.allclose(f1[:, 0::2], m * torch.cos(t * th), atol=1e-14)
    assert torch.equal(f1[:, 0::2], f1[:, 1::2])
    assert torch.allclose(f2[:, 1::2], m * torch.sin(t * th), atol=1e-14)
    assert torch.equal(f2[:, 0::2], -f2[:, 1::2])
    # Every pair block is m times a rotation: determinant m^2.
    det = f1[:, 0::2] * f1[:, 1::2] - f2[:, 0::2] * f2[:, 1::2]
    assert torch.allclose(det, torch.full_like(det, m * m), rtol=1e-13)


def test_unscaled_tables_are_plain_rope():
    th = yarn_frequencies(128, 10000.0, 1.0, None)
    assert torch.equal(th, torch.tensor([10000.0 ** (-2.0 * i / 128) for i in range(64)], dtype=torch.float64))
    with pytest.raises(ValueError):
        yarn_frequencies(64, 10000.0, 4.0, None)
