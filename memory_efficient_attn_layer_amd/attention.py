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
  * Heads of 32 dimensions run natively; heads of 16 run zero-padded to 32
    (zero weight rows and o_proj columns, identity rotary pairs), and an
    odd number of 16- or 32-wide heads gets one zero head more (the kernels
    take 32-wide heads in pairs); the head RMSNorm and the attention scale
    use the true head width, so results are those of the unpadded block.
"""
from __future__ import annotations

import torch

from . import _lib

SUPPORTED_HEAD_DIMS = (16, 32, 64, 128, 256)


def storage_shape(H: int, N: int) -> tuple[int, int]:
    """(heads, head width) the library runs for H heads of N dimensions. The
    kernels are built for widths 32, 64, 128 and 256, and 32-wide heads come
    in pairs (the projection tiles hold head pairs): heads of 16 dimensions
    run zero-padded to 32, and an odd number of 16- or 32-wide heads gets one
    zero head more."""
    if N >= 64 or N not in SUPPORTED_HEAD_DIMS:
        return H, N
    return H + (H & 1), 32


def storage_n(H: int, N: int) -> int:
    """Head width the library runs (storage_shape)."""
    return storage_shape(H, N)[1]
MAX_C_FORWARD = 16384
MAX_C_BACKWARD = 16384
MAX_HN_C = 1 << 29  # H * N * C below this: 32-bit element indices into the stacked weights


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
    if C < 32 or C % 32 != 0 or C > MAX_C_FORWARD:
        raise ValueError(f"model width C={C} must be a multiple of 32 in [32, {MAX_C_FORWARD}]")
    if need_backward and C > MAX_C_BACKWARD:
        raise ValueError(f"backward supports C <= {MAX_C_BACKWARD}, got C={C}")
    HN = H * N
    if HN * C >= MAX_HN_C:
        raise ValueError(f"H*N*C = {HN * C} must be below 2^29")
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


def _pad_heads(H: int, N: int, weights, factor1, factor2, pad_n: int, pad_h: int | None = None):
    """Zero-pads every head from N to pad_n dimensions and the head count
    from H to pad_h (zero heads), differentiably (the gradients of the
    caller's tensors are the slices of the padded ones): rows of Wq, Wk, Wv,
    Wg and columns of Wo get zeros; the rotary tables get identity pairs
    (factor1 = 1, factor2 = 0), which keep the padded q and k dimensions at
    zero and the pair blocks invertible for the backward. A zero head has
    q = k = v = 0 and a zero column block in Wo: it adds nothing to y, and
    every gradient it produces is zero (dZ = dy Wo is zero on it)."""
    wq, wk, wv, wg, wo = weights
    pad_h = H if pad_h is None else pad_h
    P, Q = pad_n - N, pad_h - H

    def rows(w):
        C = w.shape[1]
        w3 = torch.cat([w.reshape(H, N, C), w.new_zeros(H, P, C)], dim=1)
        return torch.cat([w3, w.new_zeros(Q, pad_n, C)], dim=0).reshape(pad_h * pad_n, C)

    C = wo.shape[0]
    wo3 = torch.cat([wo.reshape(C, H, N), wo.new_zeros(C, H, P)], dim=2)
    wo_p = torch.cat([wo3, wo.new_zeros(C, Q, pad_n)], dim=1).reshape(C, pad_h * pad_n)
    f1_p = torch.cat([factor1, factor1.new_ones(factor1.shape[0], P)], dim=1)
    f2_p = torch.cat([factor2, factor2.new_zeros(factor2.shape[0], P)], dim=1)
    return (rows(wq), rows(wk), rows(wv), rows(wg), wo_p), f1_p, f2_p


def _tables32(factor1: torch.Tensor, factor2: torch.Tensor, T: int):
    return factor1[:T].float().contiguous(), factor2[:T].float().contiguous()


def _bf16_tables(factor1: torch.Tensor, factor2: torch.Tensor) -> bool:
    """Whether the fp32 copies of the tables hold bf16 numbers only (the
    library then reads a packed bf16 copy in the projection; same results)."""
    return factor1.dtype == torch.bfloat16 and factor2.dtype == torch.bfloat16


def _wants_grad(*tensors) -> bool:
    """Whether autograd will record the op: grad mode is on and an input
    requires grad. Decided by the caller of ``Function.apply``: inside
    ``forward`` grad mode is always off and ``ctx.needs_input_grad`` ignores
    it (a Parameter reports True even under ``torch.no_grad()``)."""
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


class FusedAttentionFunction(torch.autograd.Function):
    """Autograd op of the block (fast_triton_attn.py:373-675).

    ``apply(x, Wq, Wk, Wv, Wg, Wo, factor1, factor2, H, N, eps)`` as in the
    reference (:685-697). Without a gradient requirement (grad mode off, or
    no input requiring grad) the forward saves nothing and writes no O / lse.
    """

    @classmethod
    def apply(cls, x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2, H, N, eps=1e-6):
        save = _wants_grad(x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2)
        weights = (q_weight, k_weight, v_weight, g_weight, o_weight)
        H, N = int(H), int(N)
        Hs, Ns = storage_shape(H, N)
        if (Hs, Ns) != (H, N):
            _validate(x, weights, factor1, factor2, H, N, float(eps), save)
            weights, factor1, factor2 = _pad_heads(H, N, weights, factor1, factor2, Ns, Hs)
            return super().apply(x, *weights, factor1, factor2, Hs, Ns, eps, save, N if Ns != N else 0)
        return super().apply(x, *weights, factor1, factor2, H, N, eps, save, 0)

    @staticmethod
    def forward(ctx, x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2, H, N, eps, save,
                n_active):
        H, N, eps, n_active = int(H), int(N), float(eps), int(n_active)
        weights = (q_weight, k_weight, v_weight, g_weight, o_weight)
        need_bwd = bool(save)
        _validate(x, weights, factor1, factor2, H, N, eps, need_bwd)
        lib = _lib.load()
        B, T, C = x.shape
        dev = x.device
        xc = x.contiguous()
        wc = [w.contiguous() for w in weights]
        f1, f2 = _tables32(factor1, factor2, T)
        d = _lib.desc(B, T, C, H, N, T, eps, n_active, _bf16_tables(factor1, factor2))
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
            # The fp32 table rows too: the backward reuses them instead of casting again.
            ctx.save_for_backward(xc, *wc, factor1, factor2, f1, f2, o_save, lse)
        ctx.H, ctx.N, ctx.eps, ctx.n_active = H, N, eps, n_active
        return y

    @staticmethod
    def backward(ctx, grad_output):
        x, wq, wk, wv, wg, wo, factor1, factor2, f1, f2, o_save, lse = ctx.saved_tensors
        H, N, eps = ctx.H, ctx.N, ctx.eps
        lib = _lib.load()
        B, T, C = x.shape
        dev = x.device
        dy = grad_output.to(torch.bfloat16).contiguous()
        d = _lib.desc(B, T, C, H, N, T, eps, ctx.n_active, _bf16_tables(factor1, factor2))
        dx = torch.empty_like(x)
        dws = [torch.empty_like(w) for w in (wq, wk, wv, wg, wo)]
        want_f = ctx.needs_input_grad[6] or ctx.needs_input_grad[7]
        if want_f:
            df1 = torch.empty((T, N), device=dev, dtype=torch.float32)
            df2 = torch.empty((T, N), device=dev, dtype=torch.float32)
        else:
            df1 = df2 = None
        ws_bytes = lib.mea_workspace_bytes(d, _lib.MEA_PASS_BWD_TABLES if want_f else _lib.MEA_PASS_BWD)
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
        return (dx, *dws, gf1, gf2, None, None, None, None, None)


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


class FusedAttentionVarlenFunction(torch.autograd.Function):
    """The block over packed variable-length sequences: x is (total, C), the
    sequences lie back to back with offsets cu_seqlens (nseq + 1, int32, on
    the device); attention is causal inside each sequence and the rotary row
    of a token is its position in its sequence. The reference's aten call
    carries the (unused) cum_seq slots for this (fast_triton_attn.py:431-432).
    Gradients as in FusedAttentionFunction; table gradients cover rows
    0 .. max_len - 1."""

    @classmethod
    def apply(cls, x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2, cu_seqlens, max_len, H, N,
              eps=1e-6):
        save = _wants_grad(x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2)
        weights = (q_weight, k_weight, v_weight, g_weight, o_weight)
        H, N = int(H), int(N)
        Hs, Ns = storage_shape(H, N)
        if (Hs, Ns) != (H, N):
            if not isinstance(x, torch.Tensor) or x.dim() != 2:
                raise ValueError("x must be a (total_tokens, C) tensor")
            _validate(x[:1].unsqueeze(0), weights, factor1, factor2, H, N, float(eps), save)
            weights, factor1, factor2 = _pad_heads(H, N, weights, factor1, factor2, Ns, Hs)
            return super().apply(x, *weights, factor1, factor2, cu_seqlens, max_len, Hs, Ns, eps, save,
                                 N if Ns != N else 0)
        return super().apply(x, *weights, factor1, factor2, cu_seqlens, max_len, H, N, eps, save, 0)

    @staticmethod
    def forward(ctx, x, q_weight, k_weight, v_weight, g_weight, o_weight, factor1, factor2, cu_seqlens, max_len, H,
                N, eps, save, n_active):
        H, N, eps, max_len, n_active = int(H), int(N), float(eps), int(max_len), int(n_active)
        weights = (q_weight, k_weight, v_weight, g_weight, o_weight)
        if not isinstance(x, torch.Tensor) or x.dim() != 2:
            raise ValueError("x must be a (total_tokens, C) tensor")
        need_bwd = bool(save)
        # Dtypes, devices, widths and weight shapes (tables: rows checked against max_len below).
        _validate(x[:1].unsqueeze(0), weights, factor1, factor2, H, N, eps, need_bwd)
        total, C = x.shape
        if (cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2
                or cu_seqlens.device != x.device):
            raise ValueError("cu_seqlens must be a 1-D int32 tensor of nseq + 1 offsets on the device of x")
        nseq = cu_seqlens.numel() - 1
        if not 1 <= max_len <= total:
            raise ValueError(f"max_len={max_len} must be in [1, {total}]")
        if factor1.shape[0] < max_len:
            raise ValueError(f"rotary tables have {factor1.shape[0]} rows, fewer than max_len={max_len}")
        lib = _lib.load()
        dev = x.device
        xc = x.contiguous()
        wc = [w.contiguous() for w in weights]
        cu = cu_seqlens.contiguous()
        f1, f2 = _tables32(factor1, factor2, max_len)
        tb16 = _bf16_tables(factor1, factor2)
        d = _lib.desc(1, total, C, H, N, max_len, eps, n_active, tb16)
        d_ws = _lib.desc(1, total, C, H, N, total, eps, n_active, tb16)
        y = torch.empty((total, C), device=dev, dtype=torch.bfloat16)
        if need_bwd:
            o_save = torch.empty((total, H * N), device=dev, dtype=torch.bfloat16)
            lse = torch.empty((H, total), device=dev, dtype=torch.float32)
        else:
            o_save = lse = None
        ws_bytes = lib.mea_workspace_bytes(d_ws, _lib.MEA_PASS_FWD)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            rc = lib.mea_fwd_varlen(
                d, cu.data_ptr(), nseq, max_len, xc.data_ptr(), *[w.data_ptr() for w in wc], f1.data_ptr(),
                f2.data_ptr(), y.data_ptr(), _lib.ptr(o_save), _lib.ptr(lse), ws.data_ptr(), ws_bytes,
                _lib.stream_of(dev),
            )
        _lib.check(rc, "mea_fwd_varlen")
        if need_bwd:
            ctx.save_for_backward(xc, *wc, factor1, factor2, f1, f2, cu, o_save, lse)
        ctx.H, ctx.N, ctx.eps, ctx.max_len, ctx.n_active = H, N, eps, max_len, n_active
        return y

    @staticmethod
    def backward(ctx, grad_output):
        x, wq, wk, wv, wg, wo, factor1, factor2, f1, f2, cu, o_save, lse = ctx.saved_tensors
        H, N, eps, max_len = ctx.H, ctx.N, ctx.eps, ctx.max_len
        if x.shape[1] > MAX_C_BACKWARD:
            raise ValueError(f"backward supports C <= {MAX_C_BACKWARD}")
        lib = _lib.load()
        total, C = x.shape
        dev = x.device
        nseq = cu.numel() - 1
        dy = grad_output.to(torch.bfloat16).contiguous()
        tb16 = _bf16_tables(factor1, factor2)
        d = _lib.desc(1, total, C, H, N, max_len, eps, ctx.n_active, tb16)
        d_ws = _lib.desc(1, total, C, H, N, total, eps, ctx.n_active, tb16)
        dx = torch.empty_like(x)
        dws = [torch.empty_like(w) for w in (wq, wk, wv, wg, wo)]
        want_f = ctx.needs_input_grad[6] or ctx.needs_input_grad[7]
        if want_f:
            df1 = torch.empty((max_len, N), device=dev, dtype=torch.float32)
            df2 = torch.empty((max_len, N), device=dev, dtype=torch.float32)
        else:
            df1 = df2 = None
        ws_bytes = lib.mea_workspace_bytes(d_ws, _lib.MEA_PASS_BWD_TABLES if want_f else _lib.MEA_PASS_BWD)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            rc = lib.mea_bwd_varlen(
                d, cu.data_ptr(), nseq, max_len, dy.data_ptr(), x.data_ptr(), wq.data_ptr(), wk.data_ptr(),
                wv.data_ptr(), wg.data_ptr(), wo.data_ptr(), f1.data_ptr(), f2.data_ptr(), o_save.data_ptr(),
                lse.data_ptr(), dx.data_ptr(), *[w.data_ptr() for w in dws], _lib.ptr(df1), _lib.ptr(df2),
                ws.data_ptr(), ws_bytes, _lib.stream_of(dev),
            )
        _lib.check(rc, "mea_bwd_varlen")
        gf1 = gf2 = None
        if want_f:
            gf1 = torch.zeros_like(factor1)
            gf2 = torch.zeros_like(factor2)
            gf1[:max_len] = df1.to(factor1.dtype)
            gf2[:max_len] = df2.to(factor2.dtype)
        return (dx, *dws, gf1, gf2, None, None, None, None, None, None, None)


def check_offsets(offsets, total: int) -> int:
    """Host-side check of packed-sequence offsets: at least two entries,
    starting at 0, nondecreasing, ending at ``total``. Returns the longest
    sequence length."""
    if len(offsets) < 2:
        raise ValueError("cu_seqlens needs nseq + 1 >= 2 offsets")
    if offsets[0] != 0 or offsets[-1] != total:
        raise ValueError(f"cu_seqlens must run from 0 to {total} (got {offsets[0]} .. {offsets[-1]})")
    lens = [b - a for a, b in zip(offsets[:-1], offsets[1:])]
    if min(lens) < 0:
        raise ValueError("cu_seqlens must be nondecreasing")
    return max(lens)


def fused_attn_varlen(x, q_proj, k_proj, v_proj, g_proj, o_proj, yarn_module, H, N, cu_seqlens, max_len=None,
                      eps=1e-6):
    """``fused_attn`` over packed sequences: x (total, C), cu_seqlens the
    nseq + 1 int32 offsets (a device tensor, a CPU tensor or a list of ints).
    max_len defaults to the longest sequence (read from the offsets on the
    host). Whenever the offsets are on the host (a list or a CPU tensor, or
    read back because max_len was left out) they are checked: nondecreasing
    from 0 to x.shape[0], and max_len at least the longest sequence (a
    smaller one would leave that sequence's last rows unwritten). Offsets
    passed on the device with an explicit max_len are trusted, as the C ABI
    trusts them."""
    if not isinstance(cu_seqlens, torch.Tensor):
        host = [int(v) for v in cu_seqlens]
        cu_seqlens = torch.tensor(host, dtype=torch.int32, device=x.device)
    elif cu_seqlens.device.type == "cpu":
        host = [int(v) for v in cu_seqlens.tolist()]
        cu_seqlens = cu_seqlens.to(device=x.device, dtype=torch.int32)
    else:
        host = None
    if max_len is None and host is None:
        host = [int(v) for v in cu_seqlens.tolist()]
    if host is not None:
        longest = check_offsets(host, x.shape[0])
        if max_len is None:
            max_len = longest
        elif int(max_len) < longest:
            raise ValueError(f"max_len={int(max_len)} is below the longest sequence ({longest} tokens)")
    return FusedAttentionVarlenFunction.apply(
        x, q_proj.weight, k_proj.weight, v_proj.weight, g_proj.weight, o_proj.weight, yarn_module.factor1,
        yarn_module.factor2, cu_seqlens, max_len, H, N, eps,
    )
