"""What bf16 flash-attention backward numerics give at the first query rows
(CPU, float64 arithmetic on the oracle's own values). A flash backward keeps
the attention output O in bf16 and forms delta_t = dO_t . O_t from it; with
exact O, sum_j dS_tj = sum_j P_tj (dP_tj - delta_t) = 0 and dQ_t =
sum_j dS_tj k_j is a combination of key differences. With bf16 O the sum is
dO_t . (O_t - bf16(O_t)), of relative size 2^-9, and dQ_t gains that much
of the probability-weighted mean key. When query t sees only two or three
keys nothing averages this out; this pins how large it gets on the 2x256
workload, so the GPU parity tests can bound those rows separately."""
import math

import torch

from memory_efficient_attn_layer_amd.synthetic import WORKLOADS, make_inputs
from oracle import block as ob


def _bwd_dq(q, k, v, dO, O, N):
    T = q.shape[2]
    s = q @ k.transpose(-1, -2) / math.sqrt(N)
    s = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), float("-inf"))
    p = torch.softmax(s, -1)
    ds = p * (dO @ v.transpose(-1, -2) - (dO * O).sum(-1, keepdim=True))
    return ds @ k / math.sqrt(N)


def _fwd(q, k, v, N):
    T = q.shape[2]
    s = q @ k.transpose(-1, -2) / math.sqrt(N)
    s = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), float("-inf"))
    return torch.softmax(s, -1) @ v


def simulate_kernel_dq(q, k, v, dO, N):
    """The dQ of the gfx950 kernels' arithmetic, float64 otherwise: q stored as
    bf16(c q) with c = log2(e)/sqrt(N), bf16 k, v and dO; the forward rounds P
    to bf16 for the PV product and its row sum (the fixed-offset softmax), and
    O to bf16; the backward recomputes P = exp(s - lse), forms delta from the
    bf16 dO and O, and rounds dS to bf16 for the dQ product. Returns dQ and
    the bf16 O, (B, H, T, N)."""
    c = math.log2(math.e) / math.sqrt(N)
    bf = lambda t: t.bfloat16().double()  # noqa: E731
    q = bf(q * c) / c
    k, v, dO = bf(k), bf(v), bf(dO)
    T = q.shape[2]
    s = q @ k.transpose(-1, -2) / math.sqrt(N)
    s = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), float("-inf"))
    m = s.amax(-1, keepdim=True)
    pb = bf(torch.exp(s - m))
    l = pb.sum(-1, keepdim=True)
    O = bf((pb @ v) / l)
    p = torch.exp(s - m - torch.log(l))
    ds = bf(p * (dO @ v.transpose(-1, -2) - (dO * O).sum(-1, keepdim=True)))
    return ds @ k / math.sqrt(N), O


def _row_ratio(got, ref):
    g, r = got.reshape(-1, got.shape[-1]), ref.reshape(-1, ref.shape[-1])
    sc = r.norm(dim=1)
    return (g - r).norm(dim=1) / sc.clamp_min(0.1 * sc.pow(2).mean().sqrt())


def test_bf16_saved_output_dominates_the_first_rows_of_dq():
    w = WORKLOADS[0]
    ref = ob.block_grads(make_inputs(w), w.H, w.N, dtype=torch.float64, with_intermediates=True)
    it, ig = ref["inter"], ref["inter_grad"]
    B, T, H, N = 2, w.T, w.H, w.N
    hm = lambda t: t.reshape(B, T, H, N).permute(0, 2, 1, 3)  # noqa: E731
    q, k, v, o, dO = hm(it["q"]), hm(it["k"]), hm(it["v"]), hm(it["o"]), hm(ig["o"])
    exact = _bwd_dq(q, k, v, dO, o, N)
    assert torch.allclose(exact, hm(ig["q"]), atol=1e-12)  # the restatement is autograd's dQ
    bf = lambda t: t.bfloat16().double()  # noqa: E731
    qb, kb, vb, dOb = bf(q), bf(k), bf(v), bf(dO)
    flash = _bwd_dq(qb, kb, vb, dOb, bf(_fwd(qb, kb, vb, N)), N)        # bf16 O in delta
    exact_o = _bwd_dq(qb, kb, vb, dOb, _fwd(qb, kb, vb, N), N)           # unrounded O in delta
    r_flash = _row_ratio(flash, exact).reshape(B, H, T)
    r_exact_o = _row_ratio(exact_o, exact).reshape(B, H, T)
    assert float(r_flash[..., :16].max()) > 0.05           # an early row far above the rest ...
    assert float(r_flash[..., 16:].max()) < 0.03           # ... which stay within a few 1e-3
    assert float(r_exact_o[..., :16].max()) < float(r_flash[..., :16].max()) / 2  # the bf16 O is the cause


def test_kernel_operand_reference_pins_the_first_rows():
    """What the GPU stage test compares the first 16 rows of da_q with
    (parity_util.early_daq_reference): the kernel's own operands and saved O
    in float64. Against the simulated kernel it agrees to under 1% (0.35%
    here), far inside the 6% row bound, where the exact oracle and a reference
    that only borrows the kernel's O for delta (keeping the oracle's fp32 q,
    k, v, dO) both differ by more than ten times that (5.4% and 6.4%): with
    the oracle's P V and the kernel's O in delta, sum_j dS_tj is off by
    dO . (O_kernel - O_oracle), the same size as the effect being removed."""
    from tests.parity_util import early_daq_reference, q_chain

    w = WORKLOADS[0]
    inp = make_inputs(w)
    ref = ob.block_grads(inp, w.H, w.N, dtype=torch.float32, with_intermediates=True)
    it, ig = ref["inter"], ref["inter_grad"]
    B, T, H, N, E = w.B, w.T, w.H, w.N, 16
    hm = lambda t: t.double().reshape(B, T, H, N).permute(0, 2, 1, 3)  # noqa: E731
    q, k, v, dO = hm(it["q"]), hm(it["k"]), hm(it["v"]), hm(ig["o"])
    dq_sim, O_sim = simulate_kernel_dq(q, k, v, dO, N)
    rx = torch.rsqrt(inp["x"].double().pow(2).mean(-1) + 1e-6)
    f1, f2 = inp["f1"], inp["f2"]
    got = q_chain(it, dq_sim[:, :, :E], f1, f2, rx)
    o_save = O_sim.permute(0, 2, 1, 3).reshape(B, T, H * N)
    pinned = early_daq_reference(it, dO.bfloat16(), o_save, f1, f2, rx, H, N, E)
    exact = rx[:, None, :E, None] * hm(ig["a_q"])[:, :, :E]
    borrowed_o = q_chain(it, _bwd_dq(q, k, v, dO, O_sim, N)[:, :, :E], f1, f2, rx)
    pin = float(_row_ratio(got, pinned).max())
    assert pin < 0.01
    assert float(_row_ratio(got, exact).max()) > 10 * pin
    assert float(_row_ratio(got, borrowed_o).max()) > 10 * pin
