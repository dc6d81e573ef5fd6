"""Pins the oracle (CPU) before it is trusted as the parity reference.

Each check is chosen so that a plausible slip in the oracle (a dropped term,
a wrong sign or pair index, a transposed operand, a missing eps) fails it:
library routines, closed forms, invariants, known answers, brute force and
finite differences. None of them re-types the oracle's own formula.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from memory_efficient_attn_layer_amd.yarn import rotary_tables
from oracle import block as ob
from oracle import exact_bwd as eb



@pytest.fixture(autouse=True)
def _float64_default():
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(prev)


def _inputs(B=2, T=24, C=32, H=2, N=8, scale=1.0, L0=None, seed=0, wo_zero=False, wg_zero=False, wq_zero=False):
    g = torch.Generator().manual_seed(seed)
    bnd = 0.5 / math.sqrt(C)
    u = lambda *s: (torch.rand(*s, generator=g) * 2 - 1) * bnd  # noqa: E731
    d = dict(x=torch.randn(B, T, C, generator=g), wq=u(H * N, C), wk=u(H * N, C), wv=u(H * N, C),
             wg=u(H * N, C), wo=u(C, H * N), dy=torch.randn(B, T, C, generator=g))
    if wo_zero:
        d["wo"].zero_()
    if wg_zero:
        d["wg"].zero_()
    if wq_zero:
        d["wq"].zero_()
    d["f1"], d["f2"] = rotary_tables(T, N, scale=scale, original_context=L0, dtype=torch.float64)
    return d


def _fwd(d, H, N, eps=1e-6):
    return ob.block_intermediates(d["x"], d["wq"], d["wk"], d["wv"], d["wg"], d["wo"], d["f1"], d["f2"], H, N, eps)


# --------------------------------------------------------------------------- norm
def test_rms_norm_matches_formula_and_invariants():
    x = torch.randn(5, 7, 64)
    eps = 1e-6
    ref = x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)
    assert torch.allclose(ob.rms_norm(x, eps), ref, rtol=1e-13, atol=0)
    y = ob.rms_norm(x, 0.0)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(5, 7), rtol=1e-12)
    assert torch.allclose(ob.rms_norm(3.7 * x, 0.0), y, rtol=1e-12)
    # eps sits inside the square root: a zero row maps to zero, not NaN.
    assert torch.all(ob.rms_norm(torch.zeros(1, 64), eps) == 0)


# --------------------------------------------------------------------------- rotary
def test_swap_even_odd():
    t = torch.arange(8.0)
    assert ob.swap_even_odd(t).tolist() == [1, 0, 3, 2, 5, 4, 7, 6]
    assert torch.equal(ob.swap_even_odd(ob.swap_even_odd(t)), t)
    assert np.array_equal(eb.swap(t.numpy()), ob.swap_even_odd(t).numpy())


@pytest.mark.parametrize("scale,L0", [(1.0, None), (4.0, 64), (8.0, 128)])
def test_rotary_is_complex_multiplication(scale, L0):
    """Adjacent-pair rotary == (t[2i] + i t[2i+1]) * m * exp(i pos theta_i)."""
    T, H, N = 40, 3, 16
    f1, f2 = rotary_tables(T, N, scale=scale, original_context=L0, dtype=torch.float64)
    t = torch.randn(2, T, H, N)
    out = ob.rotary(t, f1, f2)
    z = torch.complex(t[..., 0::2], t[..., 1::2])
    m = 1.0 if scale == 1.0 else 0.1 * math.log(scale) + 1.0
    ang = torch.atan2(f2[:, 1::2], f1[:, 0::2])           # pos * theta_i
    rot = m * torch.exp(1j * ang)[:, None, :]
    zr = z * rot
    assert torch.allclose(out[..., 0::2], zr.real, atol=1e-12)
    assert torch.allclose(out[..., 1::2], zr.imag, atol=1e-12)
    # f1^2 + f2^2 == m^2 per lane, and pairs share the cosine.
    assert torch.allclose(f1 * f1 + f2 * f2, torch.full_like(f1, m * m), atol=1e-12)
    assert torch.equal(f1[:, 0::2], f1[:, 1::2]) and torch.equal(f2[:, 0::2], -f2[:, 1::2])


def test_rotary_identity_at_zero_and_relative_position():
    T, N = 64, 16
    f1, f2 = rotary_tables(T, N, dtype=torch.float64)
    q = torch.randn(1, 1, 1, N).expand(1, T, 1, N)
    k = torch.randn(1, 1, 1, N).expand(1, T, 1, N)
    rq, rk = ob.rotary(q, f1, f2)[0, :, 0], ob.rotary(k, f1, f2)[0, :, 0]
    assert torch.allclose(rq[0], q[0, 0, 0], atol=1e-15)          # position 0 is the identity
    dots = rq @ rk.T                                              # <R_t q, R_s k>
    for delta in (0, 1, 5, 17):
        diag = torch.diagonal(dots, offset=-delta)                # t - s = delta
        assert torch.allclose(diag, diag[0].expand_as(diag), atol=1e-10)


def test_adjacent_pairs_equal_rotate_half_with_permuted_heads():
    """Adjacent-pair RoPE with W rows permuted (even lanes first) equals NeoX
    rotate-half RoPE: the output y is identical."""
    B, T, C, H, N = 2, 20, 32, 2, 16
    d = _inputs(B, T, C, H, N)
    y = _fwd(d, H, N)["y"]
    perm = torch.cat([torch.arange(0, N, 2), torch.arange(1, N, 2)])   # half-layout lane -> pair lane
    rows = torch.cat([h * N + perm for h in range(H)])
    wq, wk = d["wq"][rows], d["wk"][rows]
    xh = ob.rms_norm(d["x"], 1e-6)
    q = ob.rms_norm(F.linear(xh, wq).view(B, T, H, N), 1e-6)
    k = ob.rms_norm(F.linear(xh, wk).view(B, T, H, N), 1e-6)
    theta = 10000.0 ** (-2.0 * torch.arange(N // 2) / N)
    ang = torch.arange(T)[:, None] * theta[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[:, None, :]
    rot_half = lambda t: torch.cat([-t[..., N // 2:], t[..., : N // 2]], -1)  # noqa: E731
    q, k = q * cos + rot_half(q) * sin, k * cos + rot_half(k) * sin
    v = F.linear(xh, d["wv"]).view(B, T, H, N)
    o = ob.causal_attention(q, k, v).reshape(B, T, H * N)
    y2 = F.linear(o * torch.sigmoid(F.linear(xh, d["wg"])), d["wo"])
    assert torch.allclose(y, y2, atol=1e-12)


# --------------------------------------------------------------------------- attention
def test_attention_matches_brute_force():
    B, T, H, N = 2, 33, 3, 8
    q, k, v = (torch.randn(B, T, H, N) for _ in range(3))
    o = ob.causal_attention(q, k, v)
    s = torch.einsum("bthn,buhn->bhtu", q, k) / math.sqrt(N)
    s = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), float("-inf"))
    ref = torch.einsum("bhtu,buhn->bthn", torch.softmax(s, -1), v)
    assert torch.allclose(o, ref, atol=1e-12)


def test_attention_known_answers():
    B, T, H, N = 1, 9, 2, 8
    v = torch.randn(B, T, H, N)
    # T = 1: the output is v.
    assert torch.allclose(ob.causal_attention(*(torch.randn(B, 1, H, N) for _ in range(2)), v[:, :1]), v[:, :1])
    # q = 0: uniform weights over the causal prefix -> prefix means of v.
    o = ob.causal_attention(torch.zeros(B, T, H, N), torch.randn(B, T, H, N), v)
    pref = torch.cumsum(v, 1) / torch.arange(1, T + 1)[None, :, None, None]
    assert torch.allclose(o, pref, atol=1e-12)


def test_block_wq_zero_gives_prefix_means():
    B, T, C, H, N = 1, 12, 32, 2, 8
    d = _inputs(B, T, C, H, N, wq_zero=True)
    it = _fwd(d, H, N)
    assert torch.all(it["q"] == 0)
    pref = torch.cumsum(it["v"], 1) / torch.arange(1, T + 1)[None, :, None, None]
    assert torch.allclose(it["o"].view(B, T, H, N), pref, atol=1e-12)


def test_block_is_causal_and_batch_equivariant():
    B, T, C, H, N = 3, 16, 32, 2, 8
    d = _inputs(B, T, C, H, N)
    y = _fwd(d, H, N)["y"]
    d2 = dict(d)
    d2["x"] = d["x"].clone()
    d2["x"][:, 10:] += torch.randn(B, T - 10, C)
    y2 = _fwd(d2, H, N)["y"]
    assert torch.equal(y[:, :10], y2[:, :10])
    assert not torch.allclose(y[:, 10:], y2[:, 10:])
    perm = torch.tensor([2, 0, 1])
    d3 = dict(d)
    d3["x"] = d["x"][perm]
    assert torch.allclose(_fwd(d3, H, N)["y"], y[perm], atol=1e-14)


def test_gate_and_init_known_answers():
    B, T, C, H, N = 2, 10, 32, 2, 8
    d = _inputs(B, T, C, H, N, wg_zero=True)
    it = _fwd(d, H, N)
    assert torch.all(it["sig"] == 0.5)
    assert torch.allclose(it["y"], 0.5 * F.linear(it["o"], d["wo"]), atol=1e-14)
    # README.md:35 initialises o_proj to zero: y = 0 and only dWo is nonzero.
    d = _inputs(B, T, C, H, N, wo_zero=True)
    g = ob.block_grads(d, H, N, dtype=torch.float64)
    assert torch.all(g["y"] == 0)
    for k in ("dx", "dwq", "dwk", "dwv", "dwg", "df1", "df2"):
        assert torch.all(g[k] == 0), k
    assert g["dwo"].abs().max() > 0


# --------------------------------------------------------------------------- gradients
def test_oracle_gradcheck_fp64():
    B, T, C, H, N = 1, 6, 16, 2, 4
    d = _inputs(B, T, C, H, N, scale=4.0, L0=2)
    names = ("x", "wq", "wk", "wv", "wg", "wo", "f1", "f2")
    args = tuple(d[n].clone().requires_grad_(True) for n in names)
    fn = lambda *a: ob.block_forward(*a, H, N, 1e-6)  # noqa: E731
    assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("scale,L0", [(1.0, None), (4.0, 8), (8.0, 16)])
def test_numpy_exact_backward_matches_autograd(scale, L0):
    """Two independent derivations of the gradients: hand-written numpy
    (oracle.exact_bwd) vs torch autograd through library ops (oracle.block)."""
    B, T, C, H, N = 2, 21, 32, 2, 8
    d = _inputs(B, T, C, H, N, scale=scale, L0=L0)
    g = ob.block_grads(d, H, N, dtype=torch.float64)
    npd = {k: v.numpy() for k, v in d.items()}
    fw = eb.forward(npd["x"], npd["wq"], npd["wk"], npd["wv"], npd["wg"], npd["wo"], npd["f1"], npd["f2"], H, N)
    assert np.allclose(fw["y"], g["y"].numpy(), atol=1e-13)
    bw = eb.backward(fw, npd["dy"], npd["wq"], npd["wk"], npd["wv"], npd["wg"], npd["wo"], H, N)
    for k in ("dx", "dwq", "dwk", "dwv", "dwg", "dwo", "df1", "df2"):
        ref = g[k].numpy()
        err = np.abs(bw[k] - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err < 1e-10, (k, err)


def test_numpy_exact_backward_finite_differences():
    """Directional derivative of sum(y*dy) along random directions."""
    B, T, C, H, N = 1, 9, 16, 2, 4
    d = {k: v.numpy() for k, v in _inputs(B, T, C, H, N, scale=4.0, L0=2, seed=3).items()}
    names = ("x", "wq", "wk", "wv", "wg", "wo", "f1", "f2")
    fw = eb.forward(*(d[n] for n in names), H, N)
    bw = eb.backward(fw, d["dy"], d["wq"], d["wk"], d["wv"], d["wg"], d["wo"], H, N)
    rng = np.random.default_rng(0)
    for n in names:
        u = rng.standard_normal(d[n].shape)
        h = 1e-6
        dp = dict(d)
        dp[n] = d[n] + h * u
        dm = dict(d)
        dm[n] = d[n] - h * u
        lp = (eb.forward(*(dp[m] for m in names), H, N)["y"] * d["dy"]).sum()
        lm = (eb.forward(*(dm[m] for m in names), H, N)["y"] * d["dy"]).sum()
        fd = (lp - lm) / (2 * h)
        an = (bw["d" + n] * u).sum()
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (n, fd, an)


def test_reference_shortcut_exact_only_for_unit_tables():
    """The reference's rotated-space q/k chain (fast_triton_attn.py:603-634)
    equals the exact chain for plain RoPE and departs from it once the YaRN
    temperature is folded into the tables."""
    B, T, C, H, N = 2, 17, 32, 2, 8
    for scale, L0, exact in ((1.0, None, True), (4.0, 8, False)):
        d = {k: v.numpy() for k, v in _inputs(B, T, C, H, N, scale=scale, L0=L0).items()}
        fw = eb.forward(d["x"], d["wq"], d["wk"], d["wv"], d["wg"], d["wo"], d["f1"], d["f2"], H, N)
        bw = eb.backward(fw, d["dy"], d["wq"], d["wk"], d["wv"], d["wg"], d["wo"], H, N)
        da_q, da_k, df1, df2 = eb.reference_qk_shortcut(fw, bw["dq"], bw["dk"], N)
        rel = lambda a, b: np.linalg.norm(a - b) / np.linalg.norm(b)  # noqa: E731
        errs = [rel(da_q, bw["da_q"]), rel(da_k, bw["da_k"]), rel(df1, bw["df1"]), rel(df2, bw["df2"])]
        if exact:
            assert max(errs) < 1e-10, errs
        else:
            assert min(errs) > 1e-3, errs
