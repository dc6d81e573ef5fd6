"""``CausalSoftmaxAttention``: the module the reference's README wraps around
``fused_attn`` (README.md:6-68), with the same constructor, initialisation and
forward signature."""
from __future__ import annotations

import torch
from torch import nn

from .attention import fused_attn
from .decode import KVCache, decode_step, prefill


class CausalSoftmaxAttention(nn.Module):
    def __init__(self, input_dim: int, num_heads: int, head_dim: int):
        super().__init__()
        self.head_dim = head_dim
        self.num_heads = num_heads
        N, H, C = head_dim, num_heads, input_dim
        with torch.no_grad():
            init_bounds = 0.5 / (C ** 0.5)
            self.q_proj = nn.Linear(C, H * N, bias=False)
            self.k_proj = nn.Linear(C, H * N, bias=False)
            self.v_proj = nn.Linear(C, H * N, bias=False)
            self.g_proj = nn.Linear(C, H * N, bias=False)
            self.o_proj = nn.Linear(H * N, C, bias=False)
            self.q_proj.weight.data.uniform_(-init_bounds, init_bounds)
            self.k_proj.weight.data.uniform_(-init_bounds, init_bounds)
            self.v_proj.weight.data.uniform_(-init_bounds, init_bounds)
            self.g_proj.weight.data.uniform_(-init_bounds, init_bounds)
            self.o_proj.weight.data.zero_()

    def forward(self, x, yarn):
        return fused_attn(x, self.q_proj, self.k_proj, self.v_proj, self.g_proj, self.o_proj, yarn,
                          self.num_heads, self.head_dim)

    # Inference with a KV cache (no counterpart in the reference, which
    # trains only): the prompt fills the cache, then one token per sequence
    # per step.
    def new_cache(self, batch: int, capacity: int, device=None) -> KVCache:
        dev = self.q_proj.weight.device if device is None else device
        return KVCache.empty(batch, self.num_heads, self.head_dim, capacity, dev)

    def prefill(self, x, yarn, cache: KVCache):
        return prefill(x, *self._weights(), yarn.factor1, yarn.factor2, self.num_heads, self.head_dim, cache)

    def decode(self, x, yarn, pos, cache: KVCache):
        return decode_step(x, *self._weights(), yarn.factor1, yarn.factor2, self.num_heads, self.head_dim,
                           pos, cache)

    def _weights(self):
        return (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.g_proj.weight,
                self.o_proj.weight)
