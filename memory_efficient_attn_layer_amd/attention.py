"""The drop-in attention block: ``FusedAttentionFunction`` and ``fused_attn``.

Same call, arguments and autograd contract as the reference
(fast_triton_attn.py:373-697):

    fused_attn(x, q_proj, k_proj, v_proj, g_proj, o_proj, yarn_module, H, N, eps=1e-6)
    FusedAttentionFunction.apply(x, Wq, Wk, Wv, Wg, Wo, factor1, factor2, H, N, eps)

The forward saves x, the weights, the rotary tables, the attention output and
its log-sum-exp (fast_triton_attn.py:463-466); the backward recomputes
everything else. All work runs in libmea.so (gfx950 HIP kernels) on the
current stream; there is no eager or CPU fallback.

Differences from the reference, all deliberate:
  * The q/k RMSNorm + rotary backward is exact for any rotary table with
    invertible pair blocks (YaRN tables with a temperature included); the
    reference's rotated-space shortcut (:603-634) is exact only when
    f1^2 + f2^2 == 1.
  * Table gradients are computed only when a table requires grad.
  * Rotary tables may be bf16, fp16 or fp32 (the reference accepts only bf16).
  * Without a gradient requirement the forward keeps no activations.
  * Unsupported shapes raise ValueError before any launch.
"""
from __future__ import annotations

import torch

from . import _lib

SUPPORTED_HEAD_DIMS = (64, 128)
MAX_C_FORWARD = 4096
MAX_C_BACKWARD = 1024


def _validate(x, weights, factor1, factor2, H: int, N: int, eps: float, need_backward: bool) -> None:
    if not isinstance(x, torch.Tensor) or x.dim() != 3:
        raise ValueError("x must be a (B, T, C) tensor")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16, got {x.dtype}")
    B, T, C = x.shape
    if B < 1 or T < 1:
        raise ValueError(f"empty input: x.shape={tuple(x.shape)}")
    if N not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head width N={N} not supported (supported: {SUPPORTED_HEAD_DIMS})")
    if H < 1:
        raise ValueError(f"H={H} must be >= 1")
    if C % 256 != 0 or C > MAX_C_FORWARD:
        raise ValueError(f"model width C={C} must be a multiple of 256 and <= {MAX_C_FORWARD}")
    if need_backward and C > MAX_C_BACKWARD:
        raise ValueError(f"backward supports C <= {MAX_C_BACKWARD}, got C={C}")
    HN = H * N
    names = ("q_proj", "k_proj", "v_proj", "g_proj", "o_proj")
    shapes = ((HN, C),) * 4 + ((C, HN),)
    for name, w, shp in zip(names, weights, shapes):
        if tuple(w.shape) != shp:
            raise ValueError(f"{name}.weight has shape {tuple(w.shape)}, expected {shp}")
        if w.dtype != torch.bfloat16:
            raise TypeError(f"{name}.weight must be bfloat16, got {w.dtype}")
        if w.device != x.device:
            raise ValueError(f"{name}.weight is on {w.device}, x is on {x.device}")
    for name, f in (("factor1", factor1), ("factor2", factor2)):
        if f.dim() != 2 or f.shape[1] != N:
            raise ValueError(f"{name} must be (T_max, N={N}), got {tuple(f.shape)}")
        if f.shape[0] < T:
            raise ValueError(f"{name} has {f.shape[0]} rows, fewer than T={T}")
        if f.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise TypeError(f"{name} must be a floating tensor, got {f.dtype}")
        if f.device != x.device:
            raise ValueError(f"{name} is on {f.device}, x is on {x.device}")
    if factor1.shape != factor2.shape:
        raise ValueError("factor1 and factor2 must have the same shape")
    if not (eps > 0.0) or eps != eps or eps == float("inf"):
        raise ValueError(f"eps={eps} must be finite and positive")
    if not x.is_cuda:
        raise RuntimeError("fused_attn runs only on a ROCm GPU device (there is no CPU path)")


def _tables32(factor1: torch.Tensor, factor2: torch.Tensor, T: int):
    return factor1[:T].float().contiguous(), factor2[:T].float().contiguous()


class FusedAttentionFunction(torch.autograd.Function):
    """Autograd op of the block (fast_triton_attn.py:373-675)."""

    @staticmethod
    def forward(ctx, x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2, H, N, eps):
        H, N, eps = int(H), int(N), float(eps)
        weights = (q_weight, k_weight, v_weight, g_weight, o_weight)
        need_bwd = any(ctx.needs_input_grad[:8])
        _validate(x, weights, factor1, factor2, H, N, eps, need_bwd)
        lib = _lib.load()
        B, T, C = x.shape
        dev = x.device
        xc = x.contiguous()
        wc = [w.contiguous() for w in weights]
        f1, f2 = _tables32(factor1, factor2, T)
        d = _lib.desc(B, T, C, H, N, T, eps)
        y = torch.empty((B, T, C), device=dev, dtype=torch.bfloat16)
        if need_bwd:
            o_save = torch.empty((B, T, H * N), device=dev, dtype=torch.bfloat16)
            lse = torch.empty((B, H, T), device=dev, dtype=torch.float32)
        else:
            o_save = lse = None
        ws_bytes = lib.mea_workspace_bytes(d, _lib.MEA_PASS_FWD)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            rc = lib.mea_fwd(
                d, xc.data_ptr(), *[w.data_ptr() for w in wc], f1.data_ptr(), f2.data_ptr(), y.data_ptr(),
                _lib.ptr(o_save), _lib.ptr(lse), ws.data_ptr(), ws_bytes, _lib.stream_of(dev),
            )
        _lib.check(rc, "mea_fwd")
        if need_bwd:
            ctx.save_for_backward(xc, *wc, factor1, factor2, o_save, lse)
        ctx.H, ctx.N, ctx.eps = H, N, eps
        return y

    @staticmethod
    def backward(ctx, grad_output):
        x, wq, wk, wv, wg, wo, factor1, factor2, o_save, lse = ctx.saved_tensors
        H, N, eps = ctx.H, ctx.N, ctx.eps
        lib = _lib.load()
        B, T, C = x.shape
        dev = x.device
        dy = grad_output.to(torch.bfloat16).contiguous()
        f1, f2 = _tables32(factor1, factor2, T)
        d = _lib.desc(B, T, C, H, N, T, eps)
        dx = torch.empty_like(x)
        dws = [torch.empty_like(w) for w in (wq, wk, wv, wg, wo)]
        want_f = ctx.needs_input_grad[6] or ctx.needs_input_grad[7]
        if want_f:
            df1 = torch.empty((T, N), device=dev, dtype=torch.float32)
            df2 = torch.empty((T, N), device=dev, dtype=torch.float32)
        else:
            df1 = df2 = None
        ws_bytes = lib.mea_workspace_bytes(d, _lib.MEA_PASS_BWD)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            rc = lib.mea_bwd(
                d, dy.data_ptr(), x.data_ptr(), wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), wg.data_ptr(),
                wo.data_ptr(), f1.data_ptr(), f2.data_ptr(), o_save.data_ptr(), lse.data_ptr(), dx.data_ptr(),
                *[w.data_ptr() for w in dws], _lib.ptr(df1), _lib.ptr(df2), ws.data_ptr(), ws_bytes,
                _lib.stream_of(dev),
            )
        _lib.check(rc, "mea_bwd")
        gf1 = gf2 = None
        if want_f:
            # Rows >= T receive no gradient (fast_triton_attn.py:636-639).
            gf1 = torch.zeros_like(factor1)
            gf2 = torch.zeros_like(factor2)
            gf1[:T] = df1.to(factor1.dtype)
            gf2[:T] = df2.to(factor2.dtype)
        return (dx, *dws, gf1, gf2, None, None, None)


def fused_attn(x, q_proj, k_proj, v_proj, g_proj, o_proj, yarn_module, H, N, eps=1e-6):
    """Drop-in for the reference wrapper (fast_triton_attn.py:681-697)."""
    return FusedAttentionFunction.apply(
        x,
        q_proj.weight,
        k_proj.weight,
        v_proj.weight,
        g_proj.weight,
        o_proj.weight,
        yarn_module.factor1,
        yarn_module.factor2,
        H,
        N,
        eps,
    )
