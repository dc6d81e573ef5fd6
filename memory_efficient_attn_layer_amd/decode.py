"""KV-cache inference for the block: ``prefill`` a prompt into a cache, then
``decode_step`` one new token per sequence.

The reference trains only and has no decode path; these run the same block
math (README.md:42-64) through ``mea_prefill`` / ``mea_decode`` of libmea.so.
The cache holds, per (batch, head), the k rows exactly as the attention uses
them (RMS-normalised over N and rotated) and the plain v rows, bf16, in a
``(B, cache_heads(N, H), capacity, cache_width(N, H))`` layout (heads of 16
dimensions are held zero-padded to 32, and an odd number of 16- or 32-wide
heads with one zero head more). Sequence b's new token sits at position
``pos[b]``: it reads rotary row ``pos[b]``, its k / v are written to cache row
``pos[b]``, and it attends to rows ``0 .. pos[b]``, so sequences of a batch may
have different lengths.

Rotary tables are read in fp32 rows ``0 .. capacity-1``; pass fp32 tables to
avoid a conversion per step.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .attention import MAX_C_FORWARD, SUPPORTED_HEAD_DIMS, _pad_heads, _validate, storage_shape


def cache_width(N: int, H: int) -> int:
    """Width of a cache row for H heads of N dimensions: the head width the
    library runs (storage_shape; 16-wide heads zero-padded to 32, as in
    fused_attn)."""
    return storage_shape(H, N)[1]


def cache_heads(N: int, H: int) -> int:
    """Heads of a cache for H heads of N dimensions (storage_shape: an odd
    number of 16- or 32-wide heads carries one zero head more)."""
    return storage_shape(H, N)[0]


@dataclass
class KVCache:
    """Per-layer cache: ``k`` and ``v`` of shape (B, cache_heads(N, H), capacity,
    cache_width(N, H)), bf16 (narrow heads as zero-padded rows, an odd number
    of them with one zero head more; see storage_shape)."""

    k: torch.Tensor
    v: torch.Tensor

    @classmethod
    def empty(cls, B: int, H: int, N: int, capacity: int, device) -> "KVCache":
        shape = (B, cache_heads(N, H), capacity, cache_width(N, H))
        return cls(torch.zeros(shape, device=device, dtype=torch.bfloat16),
                   torch.zeros(shape, device=device, dtype=torch.bfloat16))

    @property
    def capacity(self) -> int:
        return self.k.shape[2]

    def check(self, B: int, H: int, N: int, device) -> None:
        W, Hc = cache_width(N, H), cache_heads(N, H)
        for name, t in (("k", self.k), ("v", self.v)):
            if tuple(t.shape) != (B, Hc, self.capacity, W):
                raise ValueError(f"cache.{name} has shape {tuple(t.shape)}, expected {(B, Hc, self.capacity, W)}")
            if t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise ValueError(f"cache.{name} must be a contiguous bfloat16 tensor")
            if t.device != device:
                raise ValueError(f"cache.{name} is on {t.device}, x is on {device}")


def _padded(H: int, N: int, weights, factor1, factor2):
    """(weights, tables, H, N, N_active) as the library takes them: narrow
    heads zero-padded to storage_shape(H, N) (no gradient is taken here)."""
    Hs, Ns = storage_shape(H, N)
    if (Hs, Ns) == (H, N):
        return weights, factor1, factor2, H, N, 0
    with torch.no_grad():
        w, f1, f2 = _pad_heads(H, N, weights, factor1, factor2, Ns, Hs)
    return w, f1, f2, Hs, Ns, N if Ns != N else 0


def _tables(factor1, factor2, rows: int):
    if factor1.shape[0] < rows:
        raise ValueError(f"rotary tables have {factor1.shape[0]} rows, fewer than the cache capacity {rows}")
    return factor1[:rows].float().contiguous(), factor2[:rows].float().contiguous()


def prefill(x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2, H: int, N: int,
            cache: KVCache, eps: float = 1e-6) -> torch.Tensor:
    """Inference forward of a prompt ``x`` (B, T, C); writes its k / v rows to
    rows 0..T-1 of ``cache`` and returns y (B, T, C)."""
    H, N, eps = int(H), int(N), float(eps)
    weights = (q_weight, k_weight, v_weight, g_weight, o_weight)
    _validate(x, weights, factor1, factor2, H, N, eps, False)
    B, T, C = x.shape
    cache.check(B, H, N, x.device)
    weights, factor1, factor2, H, N, n_active = _padded(H, N, weights, factor1, factor2)
    Tc = cache.capacity
    if Tc < T:
        raise ValueError(f"cache capacity {Tc} is smaller than the prompt length {T}")
    lib = _lib.load()
    dev = x.device
    xc = x.contiguous()
    wc = [w.contiguous() for w in weights]
    tb16 = factor1.dtype == torch.bfloat16 and factor2.dtype == torch.bfloat16
    f1, f2 = _tables(factor1, factor2, Tc)
    d = _lib.desc(B, T, C, H, N, Tc, eps, n_active, tb16)
    y = torch.empty((B, T, C), device=dev, dtype=torch.bfloat16)
    ws_bytes = lib.mea_workspace_bytes(d, _lib.MEA_PASS_FWD)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        rc = lib.mea_prefill(d, xc.data_ptr(), *[w.data_ptr() for w in wc], f1.data_ptr(), f2.data_ptr(),
                             y.data_ptr(), cache.k.data_ptr(), cache.v.data_ptr(), Tc, ws.data_ptr(), ws_bytes,
                             _lib.stream_of(dev))
    _lib.check(rc, "mea_prefill")
    return y


def decode_step(x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2, H: int, N: int,
                pos, cache: KVCache, eps: float = 1e-6) -> torch.Tensor:
    """One new token per sequence: ``x`` (B, C) or (B, 1, C) at positions
    ``pos`` (B,) (an int32 device tensor or a sequence of ints, each in
    [0, capacity)); returns y with the shape of ``x``."""
    H, N, eps = int(H), int(N), float(eps)
    weights = (q_weight, k_weight, v_weight, g_weight, o_weight)
    squeeze = x.dim() == 2
    x3 = x.unsqueeze(1) if squeeze else x
    if x3.dim() != 3 or x3.shape[1] != 1:
        raise ValueError(f"x must be (B, C) or (B, 1, C), got {tuple(x.shape)}")
    _validate(x3, weights, factor1, factor2, H, N, eps, False)
    B, _, C = x3.shape
    dev = x3.device
    cache.check(B, H, N, dev)
    weights, factor1, factor2, H, N, n_active = _padded(H, N, weights, factor1, factor2)
    return _decode_launch(x3, weights, factor1, factor2, H, N, n_active, pos, cache, eps, squeeze)


def _decode_launch(x3, weights, factor1, factor2, H, N, n_active, pos, cache, eps, squeeze):
    """The library call of one decode step (weights and tables as the
    library takes them, see _padded)."""
    B, _, C = x3.shape
    dev = x3.device
    Tc = cache.capacity
    if not isinstance(pos, torch.Tensor):
        pos = torch.tensor(list(pos), dtype=torch.int32, device=dev)
    if pos.shape != (B,) or pos.dtype != torch.int32 or pos.device != dev:
        raise ValueError(f"pos must be an int32 tensor of shape ({B},) on {dev}")
    lib = _lib.load()
    xc = x3.contiguous()
    wc = [w.contiguous() for w in weights]
    posc = pos.contiguous()
    f1, f2 = _tables(factor1, factor2, Tc)
    d = _lib.desc(B, Tc, C, H, N, Tc, eps, n_active)
    y = torch.empty((B, 1, C), device=dev, dtype=torch.bfloat16)
    ws_bytes = lib.mea_decode_workspace_bytes(d)
    if ws_bytes == 0:
        raise ValueError("unsupported decode shape")
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        rc = lib.mea_decode(d, xc.data_ptr(), *[w.data_ptr() for w in wc], f1.data_ptr(), f2.data_ptr(),
                            posc.data_ptr(), cache.k.data_ptr(), cache.v.data_ptr(), y.data_ptr(), ws.data_ptr(),
                            ws_bytes, _lib.stream_of(dev))
    _lib.check(rc, "mea_decode")
    return y[:, 0] if squeeze else y


class DecodeGraph:
    """``decode_step`` captured once in a HIP graph for a fixed batch, cache and
    set of weights, then replayed: one graph launch per step instead of five
    kernel launches and the Python around them. ``step(x, pos)`` copies x
    (B, C) and pos (B,) into the graph's static inputs, replays, and returns
    the static output (overwritten by the next step; clone it to keep it).
    Nothing in the captured step clears memory with a memset.

    Construction does not touch ``cache``: the warm-up steps run on a scratch
    cache of the same shape (freed afterwards), and capturing records the
    step without executing it. The cache may therefore be prefilled before
    or after the graph is built."""

    def __init__(self, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2, H: int, N: int,
                 cache: KVCache, eps: float = 1e-6, warmup: int = 2):
        B, dev = cache.k.shape[0], cache.k.device
        C = q_weight.shape[1]
        H, N = int(H), int(N)
        weights = (q_weight, k_weight, v_weight, g_weight, o_weight)
        _validate(torch.empty((B, 1, C), device=dev, dtype=torch.bfloat16), weights, factor1, factor2, H, N,
                  float(eps), False)
        cache.check(B, H, N, dev)
        # Padded once here, so the captured step allocates nothing.
        weights, factor1, factor2, Hl, Nl, n_active = _padded(H, N, weights, factor1, factor2)
        self._w = [w.contiguous() for w in weights]
        self._f1, self._f2 = _tables(factor1, factor2, cache.capacity)
        self._args = (Hl, Nl, n_active)
        self._cache, self._eps = cache, float(eps)
        self.x = torch.zeros((B, C), device=dev, dtype=torch.bfloat16)
        self.pos = torch.zeros((B,), device=dev, dtype=torch.int32)
        # Warm-up (allocator and library state) on a side stream and a scratch
        # cache, then capture on the caller's cache.
        scratch = KVCache(torch.empty_like(cache.k), torch.empty_like(cache.v))
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(max(1, warmup)):
                self._run(scratch)
        torch.cuda.current_stream(dev).wait_stream(side)
        del scratch
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.y = self._run(self._cache)

    def _run(self, cache: KVCache):
        H, Nl, n_active = self._args
        return _decode_launch(self.x.unsqueeze(1), self._w, self._f1, self._f2, H, Nl, n_active, self.pos, cache,
                              self._eps, True)

    def step(self, x, pos) -> torch.Tensor:
        self.x.copy_(x)
        self.pos.copy_(pos if isinstance(pos, torch.Tensor) else torch.tensor(list(pos), dtype=torch.int32))
        self.graph.replay()
        return self.y


__all__ = ["KVCache", "DecodeGraph", "prefill", "decode_step", "cache_width", "cache_heads", "SUPPORTED_HEAD_DIMS",
           "MAX_C_FORWARD"]
