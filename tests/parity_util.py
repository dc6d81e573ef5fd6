"""Shared helpers of the GPU parity tests (not collected by pytest).

Tolerances (the block's stated contract, against the fp32 eager oracle on
identical bf16-rounded inputs):
  * bf16 outputs (y and stage outputs): max |gpu - ref| <= 2e-2 * max |ref|
    and relative Frobenius error <= 2e-2;
  * gradients (dx, all five weight gradients, both table gradients):
    relative Frobenius error ||gpu - ref|| / ||ref|| <= 3e-2;
  * per row (one token of y and dx; one (b, h, t) row of an attention
    gradient): ||gpu_r - ref_r|| <= ROW_TOL * max(||ref_r||, ROW_FLOOR *
    rms_r ||ref_r||). The floor keeps rows whose exact value nearly cancels
    from demanding more than bf16 operands give; an error confined to a few
    rows or one key block fails this bound even where the aggregate norm
    above would not notice it.
"""
from __future__ import annotations

import math

import torch

from memory_efficient_attn_layer_amd.attention import FusedAttentionFunction
from memory_efficient_attn_layer_amd.synthetic import Workload, make_inputs
from oracle import block as ob

OUT_TOL = 2e-2
GRAD_TOL = 3e-2
ROW_TOL = 6e-2
ROW_FLOOR = 0.1


def rel_fro(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def assert_out_close(name: str, got: torch.Tensor, ref: torch.Tensor, tol: float = OUT_TOL):
    assert torch.isfinite(got.float()).all(), f"{name}: non-finite values"
    mr, rf = max_rel(got, ref), rel_fro(got, ref)
    assert mr <= tol and rf <= tol, f"{name}: max-abs/max|ref| = {mr:.3e}, rel-fro = {rf:.3e} (tol {tol})"


def assert_rows_close(name: str, got: torch.Tensor, ref: torch.Tensor, tol: float = ROW_TOL,
                      floor: float = ROW_FLOOR) -> float:
    """Per-row bound (rows = last dimension); returns the worst ratio."""
    g = got.detach().double().cpu().reshape(-1, got.shape[-1])
    r = ref.detach().double().cpu().reshape(-1, ref.shape[-1])
    assert g.shape == r.shape, (name, tuple(got.shape), tuple(ref.shape))
    assert torch.isfinite(g).all(), f"{name}: non-finite values"
    err = (g - r).norm(dim=1)
    scale = r.norm(dim=1)
    fl = floor * float(scale.pow(2).mean().sqrt())
    ratio = err / scale.clamp_min(max(fl, 1e-30))
    worst = int(ratio.argmax())
    w = float(ratio[worst])
    print(f"  rows {name}: worst {w:.3e} at row {worst} of {g.shape[0]}, median {float(ratio.median()):.3e}")
    assert w <= tol, f"{name}: row {worst} of {g.shape[0]}: error / scale = {w:.3e} (tol {tol})"
    return w


def assert_grad_close(name: str, got: torch.Tensor, ref: torch.Tensor, tol: float = GRAD_TOL,
                      scale: torch.Tensor | None = None):
    """Relative Frobenius error <= tol. Where the exact gradient is identically
    zero (e.g. dWq with a single key), the error is measured against the norm
    of ``scale`` (a nonzero gradient of the same case) instead."""
    assert torch.isfinite(got.float()).all(), f"{name}: non-finite values"
    if float(ref.detach().double().norm()) == 0.0 and scale is not None:
        rf = float(got.detach().double().cpu().norm() / scale.detach().double().cpu().norm())
    else:
        rf = rel_fro(got, ref)
    assert rf <= tol, f"{name}: rel-fro = {rf:.3e} (tol {tol})"


def gpu_block(inp: dict, H: int, N: int, table_grad: bool = True, eps: float = 1e-6):
    """fused_attn forward + backward on the GPU with loss = sum(y * dy)."""
    names = ("x", "wq", "wk", "wv", "wg", "wo", "f1", "f2")
    leaf = {n: inp[n].detach().cuda().clone().requires_grad_(table_grad or n not in ("f1", "f2")) for n in names}
    y = FusedAttentionFunction.apply(*(leaf[n] for n in names), H, N, eps)
    y.backward(inp["dy"].cuda())
    torch.cuda.synchronize()
    out = {"y": y.detach()}
    for n in names:
        out["d" + n] = None if leaf[n].grad is None else leaf[n].grad.detach()
    return out


def check_block(w: Workload, B: int | None = None, seed: int | None = None, table_grad: bool = True, **over):
    """Full block parity on workload ``w`` (optionally a batch slice)."""
    inp = make_inputs(w, dtype=torch.bfloat16, B=B, seed=seed)
    inp.update(over)
    got = gpu_block(inp, w.H, w.N, table_grad=table_grad)
    ref = ob.block_grads(inp, w.H, w.N, dtype=torch.float32)
    assert_out_close("y", got["y"], ref["y"])
    for k in ("dx", "dwq", "dwk", "dwv", "dwg", "dwo"):
        assert_grad_close(k, got[k], ref[k], scale=ref["dwv"])
    if float(ref["dx"].norm()) > 0:
        assert_rows_close("y per token", got["y"], ref["y"])
        assert_rows_close("dx per token", got["dx"], ref["dx"])
    if table_grad:
        T = inp["x"].shape[1]
        assert_grad_close("df1", got["df1"][:T], ref["df1"][:T], scale=ref["dwv"])
        assert_grad_close("df2", got["df2"][:T], ref["df2"][:T], scale=ref["dwv"])
    return got, ref


def early_daq_reference(inter: dict, dO: torch.Tensor, o_save: torch.Tensor, f1: torch.Tensor, f2: torch.Tensor,
                        rx: torch.Tensor, H: int, N: int, E: int, eps: float = 1e-6) -> torch.Tensor:
    """rx * dL/da_q for the query rows t < E, in float64, from the operands the
    attention backward consumes: q as stored (bf16(c q) / c with
    c = log2(e) / sqrt(N)), bf16 k and v (from the oracle's intermediates
    ``inter``), the kernel's own dO (B, H, T, N) and its saved bf16 attention
    output o_save (B, T, H*N) in delta = rowsum(dO * O). A flash backward's
    delta comes from the bf16-rounded O, so sum_j dS_tj is not exactly zero and
    a query that sees only a few keys keeps an error of relative size ~2^-9
    times the cancellation of its dQ (up to 12% at t < 16); with every operand
    taken as the kernel holds it, that error is in the reference too and the
    rows agree to the normal row tolerance. Rows t < E depend on keys
    0 .. E-1 only, so this costs E x E per head."""
    B, T = rx.shape
    E = min(E, T)
    c = 1.4426950408889634 / math.sqrt(N)

    def heads(t):  # (B, T, H, N) or (B, T, H*N) -> (B, H, E, N) float64
        return t.detach().double().cpu().reshape(B, T, H, N)[:, :E].permute(0, 2, 1, 3)

    def bf(t):
        return t.bfloat16().double()

    q = bf(heads(inter["q"]) * c) / c
    k, v = bf(heads(inter["k"])), bf(heads(inter["v"]))
    do = dO.detach().double().cpu()[:, :, :E]
    o = heads(o_save)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(N)
    s = s.masked_fill(~torch.ones(E, E, dtype=torch.bool).tril(), float("-inf"))
    p = torch.softmax(s, -1)
    ds = p * (do @ v.transpose(-1, -2) - (do * o).sum(-1, keepdim=True))
    dq = (ds @ k) / math.sqrt(N)                                       # (B, H, E, N)
    return q_chain(inter, dq, f1, f2, rx, eps)


def q_chain(inter: dict, dq: torch.Tensor, f1: torch.Tensor, f2: torch.Tensor, rx: torch.Tensor,
            eps: float = 1e-6) -> torch.Tensor:
    """rx * dL/da_q (B, H, E, N) for dL/dq = dq (B, H, E, N) on the first E
    rows: autograd through the oracle's head RMSNorm and rotary of a_q."""
    B, T = rx.shape
    E = dq.shape[2]
    a_q = inter["a_q"].detach().double().cpu()[:, :E].clone().requires_grad_(True)  # (B, E, H, N)
    qr = ob.rotary(ob.rms_norm(a_q, eps), f1[:E].detach().double().cpu(), f2[:E].detach().double().cpu())
    (g,) = torch.autograd.grad(qr, a_q, dq.detach().double().cpu().permute(0, 2, 1, 3))
    return rx.detach().double().cpu()[:, None, :E, None] * g.permute(0, 2, 1, 3)
