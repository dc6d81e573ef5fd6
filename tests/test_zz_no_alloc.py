"""mea_decode_static (the decode step with the library's static scratch
buffer, no workspace argument) against mea_decode (caller workspace), both
through the C ABI: two calls in a row, the second on a smaller shape, each
must equal mea_decode's output and cache update bitwise (same kernels, same
inputs; only the scratch address differs)."""
import ctypes
import math

import pytest
import torch

from memory_efficient_attn_layer_amd import _lib
from memory_efficient_attn_layer_amd.decode import KVCache, prefill
from memory_efficient_attn_layer_amd.yarn import rotary_tables

pytestmark = pytest.mark.gpu


def _case(B, C, H, N, cap, T0, seed):
    g = torch.Generator().manual_seed(seed)
    HN, bound = H * N, 0.5 / math.sqrt(C)
    ws = [((torch.rand(HN, C, generator=g) * 2 - 1) * bound).bfloat16().cuda() for _ in range(4)]
    ws.append(((torch.rand(C, HN, generator=g) * 2 - 1) * bound).bfloat16().cuda())
    f1, f2 = rotary_tables(cap, N, scale=4.0, original_context=cap // 4, dtype=torch.float32)
    f1, f2 = f1.cuda(), f2.cuda()
    x = torch.randn(B, T0, C, generator=g).bfloat16().cuda()
    xt = torch.randn(B, C, generator=g).bfloat16().cuda()
    caches = []
    for _ in range(2):
        c = KVCache.empty(B, H, N, cap, "cuda")
        prefill(x, *ws, f1, f2, H, N, c)
        caches.append(c)
    pos = torch.tensor([T0 - 3 * b for b in range(B)], dtype=torch.int32, device="cuda")
    return ws, f1, f2, xt, pos, caches


def _decode_both(B, C, H, N, cap, T0, seed):
    print(f"\nmea_decode vs mea_decode_static: B={B} C={C} H={H} N={N} capacity={cap}", flush=True)
    lib = _lib.load()
    ws, f1, f2, xt, pos, (ce, cs) = _case(B, C, H, N, cap, T0, seed)
    d = _lib.desc(B, cap, C, H, N, cap, 1e-6)
    s = _lib.stream_of(torch.device("cuda"))
    need = lib.mea_decode_workspace_bytes(ctypes.byref(d))
    assert 0 < need <= _lib.MEA_STATIC_SCRATCH_BYTES
    wsb = torch.empty(need, dtype=torch.uint8, device="cuda")
    ye = torch.empty(B, C, dtype=torch.bfloat16, device="cuda")
    ys = torch.empty(B, C, dtype=torch.bfloat16, device="cuda")
    wp = [w.data_ptr() for w in ws]
    rc = lib.mea_decode(ctypes.byref(d), xt.data_ptr(), *wp, f1.data_ptr(), f2.data_ptr(), pos.data_ptr(),
                        ce.k.data_ptr(), ce.v.data_ptr(), ye.data_ptr(), wsb.data_ptr(), need, s)
    assert rc == 0, _lib.strerror(rc)
    rc = lib.mea_decode_static(ctypes.byref(d), xt.data_ptr(), *wp, f1.data_ptr(), f2.data_ptr(), pos.data_ptr(),
                               cs.k.data_ptr(), cs.v.data_ptr(), ys.data_ptr(), s)
    assert rc == 0, _lib.strerror(rc)
    torch.cuda.synchronize()
    assert torch.isfinite(ys.float()).all()
    assert torch.equal(ys, ye)
    assert torch.equal(cs.k, ce.k) and torch.equal(cs.v, ce.v)


def test_static_scratch_decode_matches_workspace_decode_twice():
    _decode_both(B=8, C=1024, H=8, N=128, cap=4096, T0=3000, seed=1)  # the larger scratch first
    _decode_both(B=2, C=256, H=2, N=64, cap=256, T0=100, seed=2)      # then a smaller shape
