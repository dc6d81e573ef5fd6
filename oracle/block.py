"""CPU restatement of the reference block's eager path — TEST INFRASTRUCTURE ONLY.

Follows the commented eager code the reference states is equivalent to
``fused_attn`` (README.md:3, README.md:42-64):

    x  = norm(x)                                   README.md:43
    q, k, v = Linear(x).view(B, T, H, N)           README.md:45-47
    g  = Linear(x)                                 README.md:48
    q, k = rotary(norm(q)), rotary(norm(k))        README.md:50
    o  = SDPA(q, k, v, is_causal=True)             README.md:56-62
    y  = o_proj(o * sigmoid(g))                    README.md:64

with the pieces the reference's kernels fix:
  * norm is an RMSNorm over the last dim, no weight, eps inside the rsqrt,
    eps = 1e-6 (fast_triton_attn.py:29-32, :102-106, :681);
  * rotary pairs lanes n and n^1: t*f1 + swap_even_odd(t)*f2
    (fast_triton_attn.py:132-141, :497-498);
  * the softmax scale is 1/sqrt(N) (fast_triton_attn.py:426);
  * the gate is o * sigmoid(g) laid out (B, T, H*N) (fast_triton_attn.py:123, :171-175);
  * no bias anywhere (README.md:25-29).

Everything runs in the dtype of the inputs (float32 or float64) with
library routines; gradients come from autograd.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def rms_norm(x: torch.Tensor, eps: float) -> torch.Tensor:
    """fast_triton_attn.py:29-32 — x * rsqrt(mean(x^2) + eps) over the last dim."""
    return F.rms_norm(x, (x.shape[-1],), eps=eps)


def swap_even_odd(t: torch.Tensor) -> torch.Tensor:
    """fast_triton_attn.py:497-498 — t[..., n] -> t[..., n ^ 1]."""
    n = t.shape[-1]
    return t.reshape(*t.shape[:-1], n // 2, 2).flip(-1).reshape(t.shape)


def rotary(t: torch.Tensor, f1: torch.Tensor, f2: torch.Tensor) -> torch.Tensor:
    """fast_triton_attn.py:132-141 for t of shape (B, T, H, N), tables (T, N)."""
    return t * f1[:, None, :] + swap_even_odd(t) * f2[:, None, :]


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """README.md:56-62 — SDPA, causal, default scale 1/sqrt(N); (B, T, H, N) in and out.
    The math backend is forced so float64 stays float64."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel(SDPBackend.MATH):
        o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True)
    return o.transpose(1, 2)


def block_intermediates(x, wq, wk, wv, wg, wo, f1, f2, H: int, N: int, eps: float = 1e-6) -> dict:
    """Forward of the block; returns every intermediate by name."""
    B, T, C = x.shape
    f1, f2 = f1[:T], f2[:T]
    xh = rms_norm(x, eps)
    a_q = F.linear(xh, wq).view(B, T, H, N)
    a_k = F.linear(xh, wk).view(B, T, H, N)
    a_v = F.linear(xh, wv).view(B, T, H, N)
    a_g = F.linear(xh, wg)
    qh, kh = rms_norm(a_q, eps), rms_norm(a_k, eps)
    q, k = rotary(qh, f1, f2), rotary(kh, f1, f2)
    o = causal_attention(q, k, a_v).reshape(B, T, H * N)
    sig = torch.sigmoid(a_g)
    y = F.linear(o * sig, wo)
    return dict(xh=xh, a_q=a_q, a_k=a_k, a_v=a_v, a_g=a_g, qh=qh, kh=kh, q=q, k=k, v=a_v, o=o, sig=sig, y=y)


def block_forward(x, wq, wk, wv, wg, wo, f1, f2, H: int, N: int, eps: float = 1e-6) -> torch.Tensor:
    return block_intermediates(x, wq, wk, wv, wg, wo, f1, f2, H, N, eps)["y"]


def block_grads(inputs: dict, H: int, N: int, eps: float = 1e-6, dtype=torch.float32, with_intermediates=False):
    """Forward + backward with loss = sum(y * dy). ``inputs`` holds x, wq, wk,
    wv, wg, wo, f1, f2, dy (any dtype, any device); everything is upcast to
    ``dtype`` on the CPU. Returns dict(y, dx, dwq, dwk, dwv, dwg, dwo, df1, df2)
    [+ intermediates and their gradients]."""
    names = ("x", "wq", "wk", "wv", "wg", "wo", "f1", "f2")
    leaf = {n: inputs[n].detach().to("cpu", dtype).clone().requires_grad_(True) for n in names}
    dy = inputs["dy"].detach().to("cpu", dtype)
    inter = block_intermediates(*(leaf[n] for n in names), H, N, eps)
    if with_intermediates:
        for t in inter.values():
            if t.requires_grad:
                t.retain_grad()
    (inter["y"] * dy).sum().backward()
    out = {"y": inter["y"].detach()}
    for n in names:
        out["d" + n] = leaf[n].grad.detach()
    if with_intermediates:
        out["inter"] = {k: v.detach() for k, v in inter.items()}
        out["inter_grad"] = {k: v.grad.detach() for k, v in inter.items() if v.grad is not None}
    return out
