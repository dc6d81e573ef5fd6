"""Packed variable-length sequences (mea_fwd_varlen / mea_bwd_varlen).

Expected values come from the fp32 oracle run on every sequence alone: its
output and dx rows per sequence, weight and table gradients summed over the
sequences (they are sums over tokens). Sequences of equal length packed
back to back must also reproduce the batched block exactly.
"""
import math

import pytest
import torch

from memory_efficient_attn_layer_amd.attention import FusedAttentionFunction, FusedAttentionVarlenFunction
from memory_efficient_attn_layer_amd.yarn import rotary_tables
from oracle import block as ob
from tests.parity_util import assert_grad_close, assert_out_close

pytestmark = pytest.mark.gpu

WNAMES = ("wq", "wk", "wv", "wg", "wo")


def _inputs(lens, C, H, N, t_max, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    HN, bound = H * N, 0.5 / math.sqrt(C)
    total = sum(lens)
    inp = {
        "x": torch.randn(total, C, generator=g).bfloat16(),
        "dy": torch.randn(total, C, generator=g).bfloat16(),
    }
    for n in WNAMES[:4]:
        inp[n] = ((torch.rand(HN, C, generator=g) * 2 - 1) * bound).bfloat16()
    inp["wo"] = ((torch.rand(C, HN, generator=g) * 2 - 1) * bound).bfloat16()
    inp["f1"], inp["f2"] = rotary_tables(t_max, N, scale=scale, original_context=max(t_max // 4, 16),
                                         dtype=torch.float32)
    return inp


def _gpu_varlen(inp, lens, H, N, table_grad=True):
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32, device="cuda")
    names = ("x",) + WNAMES + ("f1", "f2")
    leaf = {n: inp[n].cuda().clone().requires_grad_(table_grad or n not in ("f1", "f2")) for n in names}
    y = FusedAttentionVarlenFunction.apply(*(leaf[n] for n in names), cu, max(lens), H, N, 1e-6)
    y.backward(inp["dy"].cuda())
    torch.cuda.synchronize()
    out = {"y": y.detach()}
    for n in names:
        out["d" + n] = None if leaf[n].grad is None else leaf[n].grad.detach()
    return out


def _oracle(inp, lens, H, N):
    ys, dxs, acc = [], [], {}
    t0 = 0
    for L in lens:
        if L == 0:
            continue  # an empty sequence contributes nothing
        part = {k: v for k, v in inp.items()}
        part["x"] = inp["x"][t0:t0 + L][None]
        part["dy"] = inp["dy"][t0:t0 + L][None]
        r = ob.block_grads(part, H, N, dtype=torch.float32)
        ys.append(r["y"][0])
        dxs.append(r["dx"][0])
        for k in ("dwq", "dwk", "dwv", "dwg", "dwo", "df1", "df2"):
            acc[k] = r[k] if k not in acc else acc[k] + r[k]
        t0 += L
    acc["y"] = torch.cat(ys)
    acc["dx"] = torch.cat(dxs)
    return acc


@pytest.mark.parametrize(
    "lens,C,H,N",
    [([77, 256, 300, 1, 513], 256, 2, 64), ([130, 64, 200], 512, 4, 128), ([90, 33, 160], 512, 2, 256),
     ([70, 130], 96, 3, 32), ([0, 90, 0, 0, 45], 256, 2, 64), ([100, 57, 130], 1024, 8, 64),
     ([70, 0, 200, 33], 128, 4, 32), ([50, 129], 64, 4, 16)],
    # c1024: dx in two 512-feature groups over the packed tokens (a partial last block).
    ids=["n64-5seq", "n128-3seq", "n256-3seq", "n32-padded-2seq", "n64-empty-seqs", "c1024-3seq", "n32-4seq",
         "n16-2seq"],
)
def test_varlen_forward_backward_matches_oracle_per_sequence(lens, C, H, N):
    inp = _inputs(lens, C, H, N, t_max=max(lens) + 40, seed=21)
    got = _gpu_varlen(inp, lens, H, N)
    ref = _oracle(inp, lens, H, N)
    assert_out_close("y", got["y"], ref["y"])
    for k in ("dx", "dwq", "dwk", "dwv", "dwg", "dwo"):
        assert_grad_close(k, got[k], ref[k], scale=ref["dwv"])
    L = max(lens)
    for k in ("df1", "df2"):
        assert_grad_close(k, got[k][:L], ref[k][:L], scale=ref["dwv"])
        assert float(got[k][L:].abs().max()) == 0.0  # rows past the longest sequence get nothing


def test_varlen_many_short_sequences_forward():
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(1, 97, (40,), generator=g).tolist()
    C, H, N = 256, 2, 64
    inp = _inputs(lens, C, H, N, t_max=128, seed=23)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
    with torch.no_grad():
        y = FusedAttentionVarlenFunction.apply(inp["x"].cuda(), *(inp[n].cuda() for n in WNAMES),
                                               inp["f1"].cuda(), inp["f2"].cuda(), cu, max(lens), H, N, 1e-6)
    t0 = 0
    for i, L in enumerate(lens):
        ref = ob.block_forward(inp["x"][t0:t0 + L][None].float(), *(inp[n].float() for n in WNAMES), inp["f1"],
                               inp["f2"], H, N)[0]
        assert_out_close(f"seq {i} (len {L})", y[t0:t0 + L], ref)
        t0 += L


@pytest.mark.parametrize("N,C,H,B,T", [(64, 512, 8, 3, 700), (128, 256, 2, 2, 257)], ids=["n64", "n128"])
def test_varlen_equal_lengths_is_the_batched_block(N, C, H, B, T):
    inp = _inputs([T] * B, C, H, N, t_max=T, seed=29)
    got = _gpu_varlen(inp, [T] * B, H, N, table_grad=False)
    names = ("x",) + WNAMES + ("f1", "f2")
    leaf = {n: inp[n].cuda().clone() for n in names}
    leaf["x"] = leaf["x"].view(B, T, C)
    for n in ("x",) + WNAMES:
        leaf[n].requires_grad_(True)
    y = FusedAttentionFunction.apply(*(leaf[n] for n in names), H, N, 1e-6)
    y.backward(inp["dy"].cuda().view(B, T, C))
    torch.cuda.synchronize()
    assert torch.equal(got["y"], y.detach().view(B * T, C))
    assert torch.equal(got["dx"], leaf["x"].grad.view(B * T, C))
    for n in WNAMES:
        assert torch.equal(got["d" + n], leaf[n].grad), n
