"""Hand-derived float64 numpy restatement of the block — TEST INFRASTRUCTURE ONLY.

Independent of torch autograd and of SDPA: attention is brute force with an
explicit causal mask. The backward is written out term by term; the
tests check it against torch autograd of oracle.block (two derivations that
share no code) and against finite differences.

Forward (README.md:42-64 with the kernel details of fast_triton_attn.py):
    xh  = r_x x,  r_x = (mean_C x^2 + eps)^-1/2              :29-32
    a_p = xh W_p^T                                           :87-100
    qh  = r_q a_q, kh = r_k a_k  (per head over N)           :102-106
    q   = F1*qh + F2*S(qh),  k likewise                      :132-141
    o   = softmax(q k^T / sqrt(N) + causal) v                :425-444
    y   = (o * sigmoid(a_g)) Wo^T                            :146-176, :460

Exact backward (valid for any F1, F2):
    dZ = dy Wo,  dWo = dy^T Z,  Z = o * s
    do = dZ * s,  da_g = dZ * o * s (1 - s)
    dP = do v^T, dS = P (dP - rowsum(do * o)), dq = dS k / sqrt(N),
    dk = dS^T q / sqrt(N), dv = P^T do
    dqh = F1*dq + S(F2*dq),  da_q = r_q (dqh - qh (dqh . qh) / N)
    dF1 = sum_{b,h} dq*qh + dk*kh,  dF2 = sum_{b,h} dq*S(qh) + dk*S(kh)
    dW_p = da_p^T xh,  dxh = sum_p da_p W_p
    dx = r_x (dxh - xh (dxh . xh) / C)

``reference_qk_shortcut`` restates the reference's rotated-space q/k chain
(fast_triton_attn.py:603-634) for comparison.
"""
from __future__ import annotations

import numpy as np


def swap(t: np.ndarray) -> np.ndarray:
    """t[..., n] -> t[..., n ^ 1] (fast_triton_attn.py:497-498)."""
    n = t.shape[-1]
    return t.reshape(*t.shape[:-1], n // 2, 2)[..., ::-1].reshape(t.shape)


def _rms(t, eps):
    return 1.0 / np.sqrt(np.mean(t * t, axis=-1, keepdims=True) + eps)


def forward(x, wq, wk, wv, wg, wo, f1, f2, H, N, eps=1e-6):
    """Returns a dict of every forward intermediate (float64, heads as (B, H, T, N))."""
    x = np.asarray(x, np.float64)
    B, T, C = x.shape
    f1, f2 = np.asarray(f1, np.float64)[:T], np.asarray(f2, np.float64)[:T]
    rx = _rms(x, eps)                                        # (B, T, 1)
    xh = x * rx
    heads = lambda a: a.reshape(B, T, H, N).transpose(0, 2, 1, 3)  # noqa: E731
    a_q, a_k, a_v = (heads(xh @ np.asarray(w, np.float64).T) for w in (wq, wk, wv))
    a_g = xh @ np.asarray(wg, np.float64).T                  # (B, T, HN)
    rq, rk = _rms(a_q, eps), _rms(a_k, eps)                  # (B, H, T, 1)
    qh, kh = a_q * rq, a_k * rk
    q = qh * f1 + swap(qh) * f2
    k = kh * f1 + swap(kh) * f2
    scale = 1.0 / np.sqrt(N)
    s = np.einsum("bhtn,bhun->bhtu", q, k) * scale
    mask = np.tril(np.ones((T, T), bool))
    s = np.where(mask, s, -np.inf)
    mx = s.max(-1, keepdims=True)
    e = np.exp(s - mx)
    l = e.sum(-1, keepdims=True)
    P = e / l
    lse = (mx + np.log(l))[..., 0]                           # (B, H, T)
    o = P @ a_v                                              # (B, H, T, N)
    o_flat = o.transpose(0, 2, 1, 3).reshape(B, T, H * N)
    sg = 1.0 / (1.0 + np.exp(-a_g))
    Z = o_flat * sg
    y = Z @ np.asarray(wo, np.float64).T
    return dict(x=x, rx=rx, xh=xh, a_q=a_q, a_k=a_k, a_v=a_v, a_g=a_g, rq=rq, rk=rk, qh=qh, kh=kh, q=q, k=k,
                P=P, lse=lse, o=o, o_flat=o_flat, sig=sg, Z=Z, y=y, f1=f1, f2=f2, scale=scale)


def backward(fw: dict, dy, wq, wk, wv, wg, wo, H, N, T_max=None):
    """Exact gradients of sum(y * dy). Returns dx, dwq..dwo, df1, df2 (T_max rows)."""
    dy = np.asarray(dy, np.float64)
    B, T, C = dy.shape
    wo = np.asarray(wo, np.float64)
    Z, sg, o_flat = fw["Z"], fw["sig"], fw["o_flat"]
    dZ = dy @ wo                                             # (B, T, HN)
    dwo = np.einsum("btc,btj->cj", dy, Z)
    do_flat = dZ * sg
    da_g = dZ * o_flat * sg * (1.0 - sg)
    do = do_flat.reshape(B, T, H, N).transpose(0, 2, 1, 3)
    P, q, k, v, o = fw["P"], fw["q"], fw["k"], fw["a_v"], fw["o"]
    dP = do @ v.transpose(0, 1, 3, 2)
    delta = (do * o).sum(-1, keepdims=True)
    dS = P * (dP - delta)
    dq = (dS @ k) * fw["scale"]
    dk = (dS.transpose(0, 1, 3, 2) @ q) * fw["scale"]
    dv = P.transpose(0, 1, 3, 2) @ do
    f1, f2 = fw["f1"], fw["f2"]

    def qk_chain(dr, xh, r):
        dh = f1 * dr + swap(f2 * dr)
        return r * (dh - xh * (dh * xh).sum(-1, keepdims=True) / N)

    da_q = qk_chain(dq, fw["qh"], fw["rq"])
    da_k = qk_chain(dk, fw["kh"], fw["rk"])
    T_max = T if T_max is None else T_max
    df1 = np.zeros((T_max, N))
    df2 = np.zeros((T_max, N))
    df1[:T] = (dq * fw["qh"] + dk * fw["kh"]).sum((0, 1))
    df2[:T] = (dq * swap(fw["qh"]) + dk * swap(fw["kh"])).sum((0, 1))
    flat = lambda a: a.transpose(0, 2, 1, 3).reshape(B, T, H * N)  # noqa: E731
    das = [flat(da_q), flat(da_k), flat(dv), da_g]
    xh = fw["xh"]
    dws = [np.einsum("btj,btc->jc", da, xh) for da in das]
    dxh = sum(da @ np.asarray(w, np.float64) for da, w in zip(das, (wq, wk, wv, wg)))
    dx = fw["rx"] * (dxh - xh * (dxh * xh).sum(-1, keepdims=True) / C)
    return dict(dx=dx, dwq=dws[0], dwk=dws[1], dwv=dws[2], dwg=dws[3], dwo=dwo, df1=df1, df2=df2,
                dq=dq, dk=dk, dv=dv, da_q=da_q, da_k=da_k, da_g=da_g, delta=delta[..., 0])


def reference_qk_shortcut(fw: dict, dq, dk, N):
    """The reference's q/k gradient chain (fast_triton_attn.py:603-634), which
    normalises in the rotated space. Returns da_q, da_k, df1, df2 (T rows)."""
    f1, f2 = fw["f1"], fw["f2"]

    def rotated(dr, r_out, r):                               # :606-609
        return r * (dr - (r_out / N) * (dr * r_out).sum(-1, keepdims=True))

    gq = rotated(dq, fw["q"], fw["rq"])                      # :611
    gk = rotated(dk, fw["k"], fw["rk"])                      # :612
    da_q = gq * f1 + swap(gq * f2)                           # :618
    da_k = gk * f1 + swap(gk * f2)                           # :619
    q, k = fw["q"], fw["k"]
    dgq = (dq * q).sum((0, 1))                               # :625
    dgk = (dk * k).sum((0, 1))                               # :626
    dgqs = (dq * swap(q)).sum((0, 1))                        # :627
    dgks = (dk * swap(k)).sum((0, 1))                        # :628
    df1 = (dgq + dgk) * f1 - (dgqs + dgks) * f2              # :633
    df2 = (dgqs + dgks) * f1 + (dgq + dgk) * f2              # :634
    return da_q, da_k, df1, df2
