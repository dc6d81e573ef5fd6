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
         Workload(99, "c1024", 1, 130, 1024, 8, 64), Workload(99, "c2048", 1, 96, 2048, 16, 128),
         Workload(99, "c8192", 1, 40, 8192, 8, 128)]


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


PACK_CASES = [Workload(99, "n64", 2, 200, 256, 2, 64), Workload(99, "n128", 1, 130, 512, 4, 128),
              Workload(99, "n256", 1, 96, 512, 2, 256)]
WS_GUARD = 4096  # bytes on each side of the workspace (a multiple of 256 keeps it aligned)


def _ws_guarded(nbytes):
    buf = torch.full((nbytes + 2 * WS_GUARD,), 0xA5, dtype=torch.uint8, device="cuda")
    return buf, buf[WS_GUARD:WS_GUARD + nbytes]


def _ws_intact(buf):
    return bool((buf[:WS_GUARD] == 0xA5).all() and (buf[-WS_GUARD:] == 0xA5).all())


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def _run_block(lib, g, f1, f2, w, tables_bf16, var=None, n_active=0, table_grad=True):
    """mea_fwd + mea_bwd (or their varlen forms with var = (cu, nseq, max_len))
    with table gradients (NULL df1 / df2 without table_grad); workspaces
    guarded. Returns every output."""
    B, T, C, H, N = w.B, w.T, w.C, w.H, w.N
    HN, M = H * N, B * T
    t_max = var[2] if var is not None else T
    d = _lib.desc(B, T, C, H, N, t_max, 1e-6, n_active, tables_bf16)
    d_ws = _lib.desc(B, T, C, H, N, T, 1e-6, n_active, tables_bf16)
    s = _lib.stream_of(torch.device("cuda"))
    wts = [g[n].data_ptr() for n in ("wq", "wk", "wv", "wg", "wo")]
    y = torch.empty(M * C, dtype=torch.bfloat16, device="cuda")
    o = torch.empty(M * HN, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B * H * T, dtype=torch.float32, device="cuda")
    nf = lib.mea_workspace_bytes(ctypes.byref(d_ws), _lib.MEA_PASS_FWD)
    wsf_buf, wsf = _ws_guarded(nf)
    head = (var[0].data_ptr(), var[1], var[2]) if var is not None else ()
    fwd = lib.mea_fwd_varlen if var is not None else lib.mea_fwd
    rc = fwd(ctypes.byref(d), *head, g["x"].data_ptr(), *wts, f1.data_ptr(), f2.data_ptr(), y.data_ptr(),
             o.data_ptr(), lse.data_ptr(), wsf.data_ptr(), nf, s)
    assert rc == 0, _lib.strerror(rc)
    rows = t_max
    dx = torch.empty(M * C, dtype=torch.bfloat16, device="cuda")
    dws = [torch.empty(HN * C, dtype=torch.bfloat16, device="cuda") for _ in range(5)]
    df1 = torch.empty(rows * N, dtype=torch.float32, device="cuda") if table_grad else None
    df2 = torch.empty(rows * N, dtype=torch.float32, device="cuda") if table_grad else None
    nb = lib.mea_workspace_bytes(ctypes.byref(d_ws), _lib.MEA_PASS_BWD_TABLES if table_grad else _lib.MEA_PASS_BWD)
    wsb_buf, wsb = _ws_guarded(nb)
    bwd = lib.mea_bwd_varlen if var is not None else lib.mea_bwd
    rc = bwd(ctypes.byref(d), *head, g["dy"].data_ptr(), g["x"].data_ptr(), *wts, f1.data_ptr(), f2.data_ptr(),
             o.data_ptr(), lse.data_ptr(), dx.data_ptr(), *(t.data_ptr() for t in dws), _lib.ptr(df1),
             _lib.ptr(df2), wsb.data_ptr(), nb, s)
    assert rc == 0, _lib.strerror(rc)
    torch.cuda.synchronize()
    assert _ws_intact(wsf_buf) and _ws_intact(wsb_buf), "write past the workspace"
    return dict(y=y, o=o, lse=lse, dx=dx, dwq=dws[0], dwk=dws[1], dwv=dws[2], dwg=dws[3], dwo=dws[4],
                df1=df1, df2=df2)


@pytest.mark.parametrize("w", PACK_CASES, ids=[f"B{w.B}-T{w.T}-C{w.C}-H{w.H}-N{w.N}" for w in PACK_CASES])
def test_packed_bf16_tables_bitwise(w):
    """tables_bf16 = 1 (the projection reads a packed bf16 copy of tables whose
    values are bf16 numbers) gives bitwise the outputs of tables_bf16 = 0 in
    the forward and the backward, inside the workspace it asks for."""
    lib = _lib.load()
    inp = make_inputs(w)  # bf16 tables
    g = {k: v.cuda().contiguous() for k, v in inp.items()}
    f1, f2 = g["f1"].float().contiguous(), g["f2"].float().contiguous()
    plain = _run_block(lib, g, f1, f2, w, False)
    packed = _run_block(lib, g, f1, f2, w, True)
    for k in plain:
        assert torch.equal(_bits(plain[k]), _bits(packed[k])), f"{k} differs with packed tables"
    assert torch.isfinite(plain["y"].float()).all()


def test_packed_bf16_tables_varlen_bitwise():
    """The packed-sequence forms with tables_bf16 = 1 (per-token rotary rows
    read from the packed copy of max_len rows) match tables_bf16 = 0 bitwise."""
    lib = _lib.load()
    lens = [70, 0, 131, 33]
    w = Workload(99, "varlen", 1, sum(lens), 256, 2, 64)
    inp = make_inputs(w)
    g = {k: v.cuda().contiguous() for k, v in inp.items()}
    max_len = max(lens)
    f1, f2 = g["f1"][:max_len].float().contiguous(), g["f2"][:max_len].float().contiguous()
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
    var = (cu, len(lens), max_len)
    plain = _run_block(lib, g, f1, f2, w, False, var)
    packed = _run_block(lib, g, f1, f2, w, True, var)
    for k in plain:
        assert torch.equal(_bits(plain[k]), _bits(packed[k])), f"{k} differs with packed tables"


@pytest.mark.parametrize("pad", ["identity", "zero"])
@pytest.mark.parametrize("table_grad", [False, True], ids=["no-table-grad", "table-grad"])
@pytest.mark.parametrize("n,ns", [(32, 64), (16, 32), (32, 32)], ids=["n32-in-64", "n16-in-32", "n32-native"])
def test_narrow_heads_through_the_abi(n, ns, pad, table_grad):
    """Narrow heads through the C ABI as the header describes them. Native:
    N = 32 with an even H, no padding. Padded: N = ns, N_active = n, the
    last ns - n rows of every head of Wq, Wk, Wv, Wg and columns of Wo zero,
    and the padding columns of the rotary tables holding identity pairs
    (f1 = 1, f2 = 0) or zeros. All give the oracle's N = n block (no NaN
    from the zero pair blocks in the backward)."""
    from memory_efficient_attn_layer_amd.attention import _pad_heads

    if ns == n and pad == "zero":
        pytest.skip("no padding columns")
    lib = _lib.load()
    w = Workload(99, f"n{n}", 2, 150, 256, 4, n, 4.0, 64)
    inp = make_inputs(w)
    ref = ob.block_grads(inp, w.H, w.N)
    g = {k: v.cuda().contiguous() for k, v in inp.items()}
    if ns != n:
        wts, f1p, f2p = _pad_heads(w.H, w.N, [g[m] for m in ("wq", "wk", "wv", "wg", "wo")], g["f1"], g["f2"], ns)
        if pad == "zero":
            f1p, f2p = f1p.clone(), f2p.clone()
            f1p[:, w.N:] = 0
        gp = dict(g, **{m: t.contiguous() for m, t in zip(("wq", "wk", "wv", "wg", "wo"), wts)})
    else:
        gp, f1p, f2p = g, g["f1"], g["f2"]
    wp = Workload(99, f"n{n}p", w.B, w.T, w.C, w.H, ns)
    out = _run_block(lib, gp, f1p[:w.T].float().contiguous(), f2p[:w.T].float().contiguous(), wp, False,
                     n_active=0 if ns == n else w.N, table_grad=table_grad)
    B, T, C, H, N = w.B, w.T, w.C, w.H, w.N
    for k, v in out.items():
        if v is not None:
            assert torch.isfinite(v.float()).all(), f"{k}: non-finite values"
    assert_out_close("y", out["y"].view(B, T, C), ref["y"])
    assert_grad_close("dx", out["dx"].view(B, T, C), ref["dx"])
    for k in ("dwq", "dwk", "dwv", "dwg"):
        got = out[k].view(H, ns, C)
        assert torch.all(got[:, N:] == 0), f"{k}: padding rows nonzero"
        assert_grad_close(k, got[:, :N].reshape(H * N, C), ref[k])
    assert_grad_close("dwo", out["dwo"].view(C, H, ns)[:, :, :N].reshape(C, H * N), ref["dwo"])
    if table_grad:
        assert_grad_close("df1", out["df1"].view(T, ns)[:, :N], ref["df1"][:T])
        assert_grad_close("df2", out["df2"].view(T, ns)[:, :N], ref["df2"][:T])
