"""KV-cache prefill + decode (mea_prefill / mea_decode) against the fp32 oracle.

The oracle has no cache: the expected output of a decode step at position t
is the last row of the oracle's forward over the sequence's first t tokens
followed by the new token. Sequences of a batch may sit at different
positions, and a position below the cached length rewinds (later cache rows
are ignored and row t is overwritten).
"""
import math

import pytest
import torch

from memory_efficient_attn_layer_amd.decode import KVCache, decode_step, prefill
from memory_efficient_attn_layer_amd.yarn import rotary_tables
from oracle import block as ob
from tests.parity_util import assert_out_close

pytestmark = pytest.mark.gpu


def _params(C, H, N, capacity, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    HN, bound = H * N, 0.5 / math.sqrt(C)
    ws = [((torch.rand(HN, C, generator=g) * 2 - 1) * bound).bfloat16() for _ in range(4)]
    ws.append(((torch.rand(C, HN, generator=g) * 2 - 1) * bound).bfloat16())
    f1, f2 = rotary_tables(capacity, N, scale=scale, original_context=max(capacity // 4, 16), dtype=torch.float32)
    return ws, f1, f2, g


def _oracle_last(seq, ws, f1, f2, H, N):
    """y of the last token of one sequence seq (T, C) under the oracle."""
    y = ob.block_forward(seq[None].float(), *(w.float() for w in ws), f1, f2, H, N)
    return y[0, -1]


class _Block:
    def __init__(self, ws, f1, f2, H, N):
        self.ws = [w.cuda() for w in ws]
        self.f1, self.f2 = f1.cuda(), f2.cuda()
        self.H, self.N = H, N

    def prefill(self, x, cache):
        return prefill(x.cuda(), *self.ws, self.f1, self.f2, self.H, self.N, cache)

    def decode(self, x, pos, cache):
        out = decode_step(x.cuda(), *self.ws, self.f1, self.f2, self.H, self.N, pos, cache)
        torch.cuda.synchronize()
        return out


@pytest.mark.parametrize(
    "C,H,N",
    [(256, 2, 64), (512, 4, 128), (512, 2, 256), (96, 3, 32), (64, 4, 16), (256, 8, 32)],
    ids=["c256-h2-n64", "c512-h4-n128", "c512-h2-n256", "c96-h3-n32-padded", "c64-h4-n16-padded", "c256-h8-n32"],
)
def test_prefill_then_decode_matches_oracle(C, H, N):
    B, T0, steps, cap = 2, 37, 3, 64
    ws, f1, f2, g = _params(C, H, N, cap, seed=3)
    blk = _Block(ws, f1, f2, H, N)
    x = torch.randn(B, T0 + steps, C, generator=g).bfloat16()
    cache = KVCache.empty(B, H, N, cap, "cuda")
    y0 = blk.prefill(x[:, :T0], cache)
    ref0 = ob.block_forward(x[:, :T0].float(), *(w.float() for w in ws), f1, f2, H, N)
    assert_out_close("prefill y", y0, ref0)
    for s in range(steps):
        t = T0 + s
        y = blk.decode(x[:, t], [t] * B, cache)
        for b in range(B):
            assert_out_close(f"decode b{b} t{t}", y[b], _oracle_last(x[b, :t + 1], ws, f1, f2, H, N))
    # Sequence 1 rewinds to position 20: rows 20.. of its cache are ignored and
    # row 20 is overwritten; sequence 0 continues.
    xr = torch.randn(B, C, generator=g).bfloat16()
    y = blk.decode(xr, [T0 + steps, 20], cache)
    assert_out_close("ragged b0", y[0], _oracle_last(torch.cat([x[0], xr[0:1]]), ws, f1, f2, H, N))
    assert_out_close("ragged b1", y[1], _oracle_last(torch.cat([x[1, :20], xr[1:2]]), ws, f1, f2, H, N))


def test_decode_at_position_zero_is_the_token_alone():
    C, H, N, cap = 256, 2, 64, 128
    ws, f1, f2, g = _params(C, H, N, cap, seed=5)
    blk = _Block(ws, f1, f2, H, N)
    x = torch.randn(3, C, generator=g).bfloat16()
    cache = KVCache.empty(3, H, N, cap, "cuda")
    y = blk.decode(x, [0, 0, 0], cache)
    for b in range(3):
        assert_out_close(f"b{b}", y[b], _oracle_last(x[b:b + 1], ws, f1, f2, H, N))


def test_decode_batch_past_one_token_tile():
    # B = 70 new tokens: the decode products take a second 64-token tile, and
    # 140 (b, h) pairs each get their own position (rewinds included).
    C, H, N, B, T0, cap = 128, 2, 64, 70, 24, 32
    ws, f1, f2, g = _params(C, H, N, cap, seed=17)
    blk = _Block(ws, f1, f2, H, N)
    x = torch.randn(B, T0, C, generator=g).bfloat16()
    cache = KVCache.empty(B, H, N, cap, "cuda")
    blk.prefill(x, cache)
    pos = torch.randint(0, T0 + 1, (B,), generator=g).tolist()
    xn = torch.randn(B, C, generator=g).bfloat16()
    y = blk.decode(xn, pos, cache)
    for b in range(B):
        p = pos[b]
        ref = _oracle_last(torch.cat([x[b, :p], xn[b:b + 1]]), ws, f1, f2, H, N)
        assert_out_close(f"b{b} pos {p}", y[b], ref)


def test_decode_long_cache_across_split_boundaries():
    # 3000 cache rows over B * H = 4 heads: 48 splits of 64 keys, so these
    # positions put the last key first, last and inside a split, and the
    # step after the prefill spans 40 splits.
    C, H, N, B, T0, cap = 256, 2, 64, 2, 2500, 3000
    ws, f1, f2, g = _params(C, H, N, cap, seed=7, scale=4.0)
    blk = _Block(ws, f1, f2, H, N)
    x = torch.randn(B, T0, C, generator=g).bfloat16()
    cache = KVCache.empty(B, H, N, cap, "cuda")
    blk.prefill(x, cache)
    for pos in ([T0, T0], [63, 64], [65, 127], [128, 2047]):
        xn = torch.randn(B, C, generator=g).bfloat16()
        y = blk.decode(xn, pos, cache)
        for b in range(B):
            p = pos[b]
            ref = _oracle_last(torch.cat([x[b, :p], xn[b:b + 1]]), ws, f1, f2, H, N)
            assert_out_close(f"pos {p} b{b}", y[b], ref)
        # the step overwrote row pos[b]; restore the prompt's rows for the
        # next rewind
        blk.prefill(x, cache)


def test_decode_matches_prefill_rows():
    # Decoding token t over a cache of the first t prompt tokens reproduces
    # row t of the prefill output (the two use different attention kernels:
    # agreement to the output tolerance).
    C, H, N, B, T0, cap = 512, 4, 128, 2, 300, 320
    ws, f1, f2, g = _params(C, H, N, cap, seed=11)
    blk = _Block(ws, f1, f2, H, N)
    x = torch.randn(B, T0, C, generator=g).bfloat16()
    cache = KVCache.empty(B, H, N, cap, "cuda")
    y_pre = blk.prefill(x, cache)
    for t in (0, 1, 150, 299):
        y = blk.decode(x[:, t], [t] * B, cache)
        assert_out_close(f"t{t}", y, y_pre[:, t])


@pytest.mark.parametrize("C,H,N", [(256, 2, 64), (512, 4, 128)], ids=["n64", "n128"])
def test_prefill_with_bf16_tables_is_bitwise_the_fp32_copy(C, H, N):
    # bf16 tables take the packed-table projection; their fp32 copy the plain
    # one. Same values, so the outputs and both caches agree bitwise.
    B, T0, cap = 2, 75, 96
    ws, f1, f2, g = _params(C, H, N, cap, seed=23)
    f1b, f2b = f1.bfloat16(), f2.bfloat16()
    x = torch.randn(B, T0, C, generator=g).bfloat16()
    outs = []
    for t1, t2 in ((f1b, f2b), (f1b.float(), f2b.float())):
        cache = KVCache.empty(B, H, N, cap, "cuda")
        y = prefill(x.cuda(), *[w.cuda() for w in ws], t1.cuda(), t2.cuda(), H, N, cache)
        torch.cuda.synchronize()
        outs.append((y, cache.k.clone(), cache.v.clone()))
    for name, a, b in zip(("y", "k_cache", "v_cache"), outs[0], outs[1]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), name
    ref = ob.block_forward(x.float(), *(w.float() for w in ws), f1b.float(), f2b.float(), H, N)
    assert_out_close("y", outs[0][0], ref)


@pytest.mark.parametrize("C,H,N", [(512, 4, 128), (128, 4, 32), (96, 3, 32)], ids=["n128", "n32", "n32-padded"])
def test_decode_graph_replays_match_eager_steps(C, H, N):
    # Captured decode steps, replayed several times with eager work and
    # synchronisation between the replays; every replay must equal the eager
    # step on the same inputs bitwise (same kernels, same cache contents).
    from memory_efficient_attn_layer_amd.decode import DecodeGraph

    B, T0, cap = 3, 100, 160
    ws, f1, f2, g = _params(C, H, N, cap, seed=13)
    blk = _Block(ws, f1, f2, H, N)
    x = torch.randn(B, T0 + 6, C, generator=g).bfloat16()
    cache_e = KVCache.empty(B, H, N, cap, "cuda")
    cache_g = KVCache.empty(B, H, N, cap, "cuda")
    blk.prefill(x[:, :T0], cache_e)
    blk.prefill(x[:, :T0], cache_g)
    before_k, before_v = cache_g.k.clone(), cache_g.v.clone()
    graph = DecodeGraph(*blk.ws, blk.f1, blk.f2, H, N, cache_g)
    torch.cuda.synchronize()
    # Building the graph (warm-up + capture) leaves the prefilled cache untouched.
    assert torch.equal(cache_g.k, before_k) and torch.equal(cache_g.v, before_v)
    del before_k, before_v
    for s in range(6):
        pos = [T0 + s, T0 + s, max(0, T0 - 40 + 7 * s)]
        y_e = blk.decode(x[:, T0 + s], pos, cache_e)
        y_g = graph.step(x[:, T0 + s].cuda(), torch.tensor(pos, dtype=torch.int32, device="cuda")).clone()
        torch.cuda.synchronize()
        _ = (torch.randn(1000, device="cuda") * 2).sum().item()  # eager work between replays
        assert torch.equal(y_g, y_e), f"replay {s}"
        assert torch.equal(cache_g.k, cache_e.k) and torch.equal(cache_g.v, cache_e.v), f"cache after replay {s}"
