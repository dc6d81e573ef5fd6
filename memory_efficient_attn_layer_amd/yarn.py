"""Rotary / YaRN tables in the adjacent-pair layout the block consumes.

The reference takes its tables from an external ``yarn`` module that is not
part of it (fast_triton_attn.py:692-693, README.md:50). The layout it needs
is fixed by the kernel: lane n is paired with lane n^1 and

    out[n] = t[n] * factor1[pos, n] + t[n ^ 1] * factor2[pos, n]

(fast_triton_attn.py:132-141), which is the complex product
(t[2i] + i t[2i+1]) * m * exp(i pos theta_i) when

    factor1[pos, 2i] = factor1[pos, 2i+1] = m cos(pos theta_i)
    factor2[pos, 2i] = -m sin(pos theta_i),  factor2[pos, 2i+1] = +m sin(pos theta_i).

Frequencies follow RoPE (theta_i = base^(-2i/N)) with YaRN's "NTK-by-parts"
interpolation and attention temperature (Peng et al., 2023, "YaRN: Efficient
Context Window Extension of Large Language Models"): for scale s over an
original context L0, with r_i = L0 * theta_i / (2 pi) and the ramp
gamma(r) = clamp((r - alpha) / (beta - alpha), 0, 1),

    theta'_i = (1 - gamma(r_i)) * theta_i / s + gamma(r_i) * theta_i
    m = 0.1 ln(s) + 1    (1 when s == 1)

The softmax scale of the block is fixed at 1/sqrt(N) (fast_triton_attn.py:426),
so the temperature is folded into both q and k tables (logits scale by m^2).
"""
from __future__ import annotations

import math

import torch
from torch import nn


def yarn_frequencies(N: int, base: float = 10000.0, scale: float = 1.0, original_context: int | None = None,
                     alpha: float = 1.0, beta: float = 32.0) -> torch.Tensor:
    """theta'_i for i in [0, N/2), float64."""
    if N % 2:
        raise ValueError("N must be even")
    i = torch.arange(N // 2, dtype=torch.float64)
    theta = base ** (-2.0 * i / N)
    if scale == 1.0:
        return theta
    if original_context is None:
        raise ValueError("YaRN scaling needs the original context length")
    r = original_context * theta / (2.0 * math.pi)
    gamma = ((r - alpha) / (beta - alpha)).clamp(0.0, 1.0)
    return (1.0 - gamma) * theta / scale + gamma * theta


def yarn_mscale(scale: float) -> float:
    return 1.0 if scale <= 1.0 else 0.1 * math.log(scale) + 1.0


def rotary_tables(T_max: int, N: int, base: float = 10000.0, scale: float = 1.0,
                  original_context: int | None = None, dtype=torch.bfloat16, device=None):
    """(factor1, factor2), each (T_max, N), in the adjacent-pair layout."""
    theta = yarn_frequencies(N, base, scale, original_context)
    m = yarn_mscale(scale)
    pos = torch.arange(T_max, dtype=torch.float64)[:, None]
    ang = pos * theta[None, :]
    c, s = m * torch.cos(ang), m * torch.sin(ang)
    f1 = torch.stack((c, c), dim=-1).reshape(T_max, N)
    f2 = torch.stack((-s, s), dim=-1).reshape(T_max, N)
    return f1.to(device=device, dtype=dtype), f2.to(device=device, dtype=dtype)


def swap_even_odd(t: torch.Tensor) -> torch.Tensor:
    """t[..., n] -> t[..., n ^ 1] (fast_triton_attn.py:497-498)."""
    n = t.shape[-1]
    return t.reshape(*t.shape[:-1], n // 2, 2).flip(-1).reshape(t.shape)


class Yarn(nn.Module):
    """Table holder with the interface the block reads: ``factor1``,
    ``factor2`` and ``rotary(t)`` for t of shape (B, T, H, N)."""

    def __init__(self, N: int, T_max: int, base: float = 10000.0, scale: float = 1.0,
                 original_context: int | None = None, dtype=torch.bfloat16, device=None):
        super().__init__()
        f1, f2 = rotary_tables(T_max, N, base, scale, original_context, dtype=dtype, device=device)
        self.register_buffer("factor1", f1, persistent=False)
        self.register_buffer("factor2", f2, persistent=False)
        self.N, self.T_max, self.scale = N, T_max, scale

    def rotary(self, t: torch.Tensor) -> torch.Tensor:
        T = t.shape[1]
        f1 = self.factor1[:T, None, :].to(t.dtype)
        f2 = self.factor2[:T, None, :].to(t.dtype)
        return t * f1 + swap_even_odd(t) * f2
