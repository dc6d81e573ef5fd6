"""Thin wrappers over the per-stage C ABI entry points.

They expose the intermediate results of the forward (rotated q/k, v,
sigmoid(g), the attention output and its lse) so each stage can be checked on
its own. They allocate their outputs with torch and run on the current
stream.
"""
from __future__ import annotations

import torch

from . import _lib


def _d(x_shape, H, N, eps=1e-6):
    B, T, C = x_shape
    return _lib.desc(B, T, C, H, N, T, eps)


def qkvg_proj(x, wq, wk, wv, wg, factor1, factor2, H, N, eps=1e-6, stats=False):
    """Returns q, k, v (B, H, T, N), sig (B, T, H*N) [, rx (B, T), rq, rk (B, H, T)]."""
    lib = _lib.load()
    B, T, C = x.shape
    dev = x.device
    f1 = factor1[:T].float().contiguous()
    f2 = factor2[:T].float().contiguous()
    q, k, v = (torch.empty((B, H, T, N), device=dev, dtype=torch.bfloat16) for _ in range(3))
    sig = torch.empty((B, T, H * N), device=dev, dtype=torch.bfloat16)
    rx = torch.empty((B, T), device=dev, dtype=torch.float32) if stats else None
    rq = torch.empty((B, H, T), device=dev, dtype=torch.float32) if stats else None
    rk = torch.empty((B, H, T), device=dev, dtype=torch.float32) if stats else None
    d = _d(x.shape, H, N, eps)
    with torch.cuda.device(dev):
        rc = lib.mea_qkvg_proj(
            d, x.contiguous().data_ptr(), wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), wg.data_ptr(),
            f1.data_ptr(), f2.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), sig.data_ptr(),
            _lib.ptr(rx), _lib.ptr(rq), _lib.ptr(rk), _lib.stream_of(dev),
        )
    _lib.check(rc, "mea_qkvg_proj")
    return (q, k, v, sig, rx, rq, rk) if stats else (q, k, v, sig)


def attn_fwd(q, k, v, C=None):
    """Causal attention of (B, H, T, N) q/k/v; returns o (B, T, H*N) and lse (B, H, T)."""
    lib = _lib.load()
    B, H, T, N = q.shape
    dev = q.device
    o = torch.empty((B, T, H * N), device=dev, dtype=torch.bfloat16)
    lse = torch.empty((B, H, T), device=dev, dtype=torch.float32)
    d = _d((B, T, C if C is not None else 256), H, N)
    with torch.cuda.device(dev):
        rc = lib.mea_attn_fwd(d, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                              _lib.stream_of(dev))
    _lib.check(rc, "mea_attn_fwd")
    return o, lse


def gate_oproj(o, sig, wo, H, N):
    """y = (o * sig) Wo^T with o, sig (B, T, H*N)."""
    lib = _lib.load()
    B, T, HN = o.shape
    C = wo.shape[0]
    dev = o.device
    y = torch.empty((B, T, C), device=dev, dtype=torch.bfloat16)
    d = _d((B, T, C), H, N)
    with torch.cuda.device(dev):
        rc = lib.mea_gate_oproj(d, o.data_ptr(), sig.data_ptr(), wo.data_ptr(), y.data_ptr(), _lib.stream_of(dev))
    _lib.check(rc, "mea_gate_oproj")
    return y


def bwd_grads(x, wq, wk, wv, wg, wo, factor1, factor2, o_save, lse, dy, H, N, eps=1e-6, table_grad=False):
    """The first half of the backward (mea_bwd_stage_grads) from the saved O
    and lse of a training forward. Returns a dict of
    daq, dak, dav (B, H, T, N), dag (B, T, H*N) -- each rx * dL/da_p with
    rx = 1/rms(x) per token -- dO (B, H, T, N), delta (B, H, T) and, with
    table_grad, df1 / df2 (T, N)."""
    lib = _lib.load()
    B, T, C = x.shape
    dev = x.device
    HN = H * N
    f1 = factor1[:T].float().contiguous()
    f2 = factor2[:T].float().contiguous()
    out = {k: torch.empty((B, H, T, N), device=dev, dtype=torch.bfloat16) for k in ("daq", "dak", "dav", "dO")}
    out["dag"] = torch.empty((B, T, HN), device=dev, dtype=torch.bfloat16)
    out["delta"] = torch.empty((B, H, T), device=dev, dtype=torch.float32)
    df1 = torch.empty((T, N), device=dev, dtype=torch.float32) if table_grad else None
    df2 = torch.empty((T, N), device=dev, dtype=torch.float32) if table_grad else None
    d = _d(x.shape, H, N, eps)
    ws_bytes = lib.mea_workspace_bytes(d, _lib.MEA_PASS_BWD_TABLES if table_grad else _lib.MEA_PASS_BWD)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    ws_w = [w.contiguous() for w in (wq, wk, wv, wg, wo)]
    with torch.cuda.device(dev):
        rc = lib.mea_bwd_stage_grads(
            d, dy.contiguous().data_ptr(), x.contiguous().data_ptr(), *[w.data_ptr() for w in ws_w],
            f1.data_ptr(), f2.data_ptr(), o_save.data_ptr(), lse.data_ptr(), out["daq"].data_ptr(),
            out["dak"].data_ptr(), out["dav"].data_ptr(), out["dag"].data_ptr(), out["dO"].data_ptr(),
            out["delta"].data_ptr(), _lib.ptr(df1), _lib.ptr(df2), ws.data_ptr(), ws_bytes, _lib.stream_of(dev),
        )
    _lib.check(rc, "mea_bwd_stage_grads")
    if table_grad:
        out["df1"], out["df2"] = df1, df2
    return out


def fwd_saved(x, wq, wk, wv, wg, wo, factor1, factor2, H, N, eps=1e-6):
    """Training forward through mea_fwd; returns y (B, T, C), the saved
    attention output o_save (B, T, H*N) and lse (B, H, T)."""
    lib = _lib.load()
    B, T, C = x.shape
    dev = x.device
    f1 = factor1[:T].float().contiguous()
    f2 = factor2[:T].float().contiguous()
    y = torch.empty((B, T, C), device=dev, dtype=torch.bfloat16)
    o = torch.empty((B, T, H * N), device=dev, dtype=torch.bfloat16)
    lse = torch.empty((B, H, T), device=dev, dtype=torch.float32)
    d = _d(x.shape, H, N, eps)
    ws_bytes = lib.mea_workspace_bytes(d, _lib.MEA_PASS_FWD)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    ws_w = [w.contiguous() for w in (wq, wk, wv, wg, wo)]
    with torch.cuda.device(dev):
        rc = lib.mea_fwd(d, x.contiguous().data_ptr(), *[w.data_ptr() for w in ws_w], f1.data_ptr(), f2.data_ptr(),
                         y.data_ptr(), o.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(dev))
    _lib.check(rc, "mea_fwd")
    return y, o, lse
