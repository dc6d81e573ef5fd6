"""The C ABI on the GPU: outputs surrounded by guard regions (no out-of-bounds
writes), workspace sized exactly by mea_workspace_bytes, ragged shapes, and
the NULL-table-gradient path."""
import ctypes

import pytest
import torch

from memory_efficient_attn_layer_amd import _lib
from memory_efficient_attn_layer_amd.synthetic import Workload, make_inputs
from oracle import block as ob
from tests.parity_util import assert_grad_close, assert_out_close

pytestmark = pytest.mark.gpu

GUARD = 4096  # elements on each side
PAT_BF16 = 0x7FA1  # a NaN pattern nothing writes
PAT_F32 = 0x7FC0DEAD


def _guarded(n, dtype):
    if dtype == torch.bfloat16:
        buf = torch.full((n + 2 * GUARD,), PAT_BF16, dtype=torch.int16, device="cuda")
    else:
        buf = torch.full((n + 2 * GUARD,), PAT_F32, dtype=torch.int32, device="cuda")
    return buf, buf[GUARD:GUARD + n].view(dtype)


def _intact(buf):
    pat = PAT_BF16 if buf.dtype == torch.int16 else PAT_F32
    return bool((buf[:GUARD] == pat).all() and (buf[-GUARD:] == pat).all())


CASES = [Workload(99, "ragged", 3, 77, 256, 2, 64), Workload(99, "n128", 2, 200, 512, 4, 128),
         Workload(99, "c1024", 1, 130, 1024, 8, 64), Workload(99, "c2048", 1, 96, 2048, 16, 128)]


@pytest.mark.parametrize("w", CASES, ids=[f"B{w.B}-T{w.T}-C{w.C}-H{w.H}-N{w.N}" for w in CASES])
def test_guarded_forward_backward(w):
    lib = _lib.load()
    inp = make_inputs(w)
    g = {k: v.cuda().contiguous() for k, v in inp.items()}
    f1, f2 = g["f1"].float().contiguous(), g["f2"].float().contiguous()
    B, T, C, H, N = w.B, w.T, w.C, w.H, w.N
    HN, M = H * N, B * T
    d = _lib.desc(B, T, C, H, N, T, 1e-6)
    s = _lib.stream_of(torch.device("cuda"))

    yb, y = _guarded(M * C, torch.bfloat16)
    ob_, o = _guarded(M * HN, torch.bfloat16)
    lb, lse = _guarded(B * H * T, torch.float32)
    wsf = lib.mea_workspace_bytes(ctypes.byref(d), 0)
    wsf_t = torch.empty(wsf, dtype=torch.uint8, device="cuda")
    rc = lib.mea_fwd(ctypes.byref(d), g["x"].data_ptr(), *(g[n].data_ptr() for n in ("wq", "wk", "wv", "wg", "wo")),
                     f1.data_ptr(), f2.data_ptr(), y.data_ptr(), o.data_ptr(), lse.data_ptr(), wsf_t.data_ptr(),
                     wsf, s)
    assert rc == 0, _lib.strerror(rc)
    torch.cuda.synchronize()
    for name, buf in (("y", yb), ("o", ob_), ("lse", lb)):
        assert _intact(buf), f"guard overwritten around {name}"

    dxb, dx = _guarded(M * C, torch.bfloat16)
    dwbufs = [_guarded(HN * C, torch.bfloat16) for _ in range(4)] + [_guarded(C * HN, torch.bfloat16)]
    df1b, df1 = _guarded(T * N, torch.float32)
    df2b, df2 = _guarded(T * N, torch.float32)
    wsb = lib.mea_workspace_bytes(ctypes.byref(d), _lib.MEA_PASS_BWD_TABLES)  # df1 / df2 are written
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    rc = lib.mea_bwd(ctypes.byref(d), g["dy"].data_ptr(), g["x"].data_ptr(),
                     *(g[n].data_ptr() for n in ("wq", "wk", "wv", "wg", "wo")), f1.data_ptr(), f2.data_ptr(),
                     o.data_ptr(), lse.data_ptr(), dx.data_ptr(), *(t.data_ptr() for _, t in dwbufs),
                     df1.data_ptr(), df2.data_ptr(), ws.data_ptr(), wsb, s)
    assert rc == 0, _lib.strerror(rc)
    torch.cuda.synchronize()
    for name, buf in [("dx", dxb), ("df1", df1b), ("df2", df2b)] + [(f"dw{i}", b) for i, (b, _) in enumerate(dwbufs)]:
        assert _intact(buf), f"guard overwritten around {name}"

    ref = ob.block_grads(inp, H, N)
    assert_out_close("y", y.view(B, T, C), ref["y"])
    assert_grad_close("dx", dx.view(B, T, C), ref["dx"])
    for (_, t), k, shp in zip(dwbufs, ("dwq", "dwk", "dwv", "dwg", "dwo"), [(HN, C)] * 4 + [(C, HN)]):
        assert_grad_close(k, t.view(shp), ref[k])
    assert_grad_close("df1", df1.view(T, N), ref["df1"])
    assert_grad_close("df2", df2.view(T, N), ref["df2"])
