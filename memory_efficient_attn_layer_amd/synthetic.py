"""Seeded synthetic workloads for the block's five shape configurations.

Draw order per configuration (CPU generator seeded with 1000 + id):
x ~ N(0, 1) (B, T, C); Wq, Wk, Wv, Wg ~ U(+-0.5/sqrt(C)) (H*N, C);
Wo ~ U(+-0.5/sqrt(C)) (C, H*N) (nonzero, so every gradient flows);
dy ~ N(0, 1) (B, T, C). Values are drawn in fp32 and rounded to bf16, so an
fp32 reference evaluated on the rounded values sees exactly the kernel inputs.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .yarn import rotary_tables


@dataclass(frozen=True)
class Workload:
    wid: int
    name: str
    B: int
    T: int
    C: int
    H: int
    N: int
    yarn_scale: float = 1.0
    original_context: int | None = None
    backward: bool = True

    @property
    def tokens(self) -> int:
        return self.B * self.T

    def flops_fwd(self) -> float:
        """Algorithmic forward flops: projections, causal attention (exact
        T(T+1)/2 pairs), output projection."""
        M, HN = self.tokens, self.H * self.N
        attn = 4.0 * self.B * self.H * self.N * self.T * (self.T + 1) / 2
        return 2.0 * M * self.C * 4 * HN + attn + 2.0 * M * HN * self.C

    def flops_attn_fwd(self) -> float:
        return 4.0 * self.B * self.H * self.N * self.T * (self.T + 1) / 2


WORKLOADS = {
    0: Workload(0, "cpu-reference B2 T256 C256 H4 N64", 2, 256, 256, 4, 64),
    1: Workload(1, "pretrain-50M B64 T4096 C512 H8 N64", 64, 4096, 512, 8, 64),
    2: Workload(2, "long-context-yarn4 B8 T32768 C512 H8 N64", 8, 32768, 512, 8, 64, 4.0, 8192),
    3: Workload(3, "wide-head B16 T8192 C1024 H8 N128", 16, 8192, 1024, 8, 128),
    4: Workload(4, "prefill-yarn8 B1 T131072 C2048 H16 N128", 1, 131072, 2048, 16, 128, 8.0, 16384, False),
    # Not one of the five configurations: the pretrain width with 32-wide
    # heads (the native N = 32 kernels), for the benchmark only.
    5: Workload(5, "narrow-head B32 T4096 C512 H16 N32", 32, 4096, 512, 16, 32),
}


def make_inputs(w: Workload, device="cpu", dtype=torch.bfloat16, seed: int | None = None, B: int | None = None):
    """Returns dict(x, wq, wk, wv, wg, wo, f1, f2, dy). ``B`` overrides the
    batch (a batch slice of the same per-sequence shape)."""
    g = torch.Generator("cpu").manual_seed(1000 + w.wid if seed is None else seed)
    Bv = w.B if B is None else B
    HN, C = w.H * w.N, w.C
    bound = 0.5 / C ** 0.5

    def unif(*shape):
        return (torch.rand(*shape, generator=g) * 2.0 - 1.0) * bound

    x = torch.randn(Bv, w.T, C, generator=g)
    wq, wk, wv, wg = (unif(HN, C) for _ in range(4))
    wo = unif(C, HN)
    dy = torch.randn(Bv, w.T, C, generator=g)
    f1, f2 = rotary_tables(w.T, w.N, scale=w.yarn_scale, original_context=w.original_context, dtype=torch.float32)
    out = dict(x=x, wq=wq, wk=wk, wv=wv, wg=wg, wo=wo, dy=dy)
    out = {k: v.to(dtype).to(device) for k, v in out.items()}
    out["f1"] = f1.to(dtype).to(device)
    out["f2"] = f2.to(dtype).to(device)
    return out
