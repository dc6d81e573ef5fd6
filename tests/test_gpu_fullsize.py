"""Size-independent properties at the full fwd+bwd workload shapes, where the
CPU oracle would be too slow or too large:

  * 50M-pretrain    B=64, T=4096,  C=512,  H=8, N=64
  * long-context    B=8,  T=32768, C=512,  H=8, N=64, YaRN s=4 over 8192
  * wide-head       B=16, T=8192,  C=1024, H=8, N=128

For each:
  * batch independence, bitwise: sequences of the full-batch run equal B=1
    runs on those sequences alone (forward output and input gradient); the
    B=1 shapes are checked against the oracle in test_gpu_parity.py (the
    wide-head one at its full length T=8192 below, the long-context one at
    T=2048 with the same tables);
  * causality, bitwise: changing the last token leaves every earlier output
    unchanged, and the first T/8 tokens equal a run on those tokens alone;
  * all outputs and gradients finite; the weight gradients equal the sum of
    the weight gradients of four batch chunks (linearity of the token
    reduction).
"""
import pytest
import torch

from memory_efficient_attn_layer_amd.attention import FusedAttentionFunction
from memory_efficient_attn_layer_amd.synthetic import WORKLOADS, make_inputs
from tests.parity_util import assert_grad_close, check_block, gpu_block

pytestmark = pytest.mark.gpu

WEIGHTS = ("wq", "wk", "wv", "wg", "wo", "f1", "f2")


@pytest.fixture(scope="module", params=[1, 2, 3], ids=lambda i: WORKLOADS[i].name.split()[0])
def full(request):
    w = WORKLOADS[request.param]
    print(f"\nfull size: {w.name}", flush=True)
    inp = make_inputs(w)
    got = gpu_block(inp, w.H, w.N, table_grad=False)
    yield w, inp, got
    del got
    torch.cuda.empty_cache()


def _slice(inp, b0, b1):
    out = dict(inp)
    out["x"] = inp["x"][b0:b1]
    out["dy"] = inp["dy"][b0:b1]
    return out


def _forward(x, args, w):
    with torch.no_grad():
        y = FusedAttentionFunction.apply(x, *(args[n] for n in WEIGHTS), w.H, w.N, 1e-6)
    torch.cuda.synchronize()
    return y


def test_fullsize_finite(full):
    _, _, got = full
    for k in ("y", "dx", "dwq", "dwk", "dwv", "dwg", "dwo"):
        assert torch.isfinite(got[k].float()).all(), k


def test_fullsize_batch_independence(full):
    w, inp, got = full
    for b in sorted({0, w.B // 2 + 1, w.B - 1}):
        one = gpu_block(_slice(inp, b, b + 1), w.H, w.N, table_grad=False)
        assert torch.equal(got["y"][b:b + 1], one["y"]), f"y of sequence {b}"
        assert torch.equal(got["dx"][b:b + 1], one["dx"]), f"dx of sequence {b}"


def test_fullsize_weight_grads_are_sums_over_sequences(full):
    w, inp, got = full
    acc = {k: torch.zeros_like(got[k], dtype=torch.float32) for k in ("dwq", "dwk", "dwv", "dwg", "dwo")}
    step = w.B // 4
    for b0 in range(0, w.B, step):
        g = gpu_block(_slice(inp, b0, b0 + step), w.H, w.N, table_grad=False)
        for k in acc:
            acc[k] += g[k].float()
    for k in acc:
        assert_grad_close(k, got[k], acc[k], tol=1e-2)


def test_fullsize_causality(full):
    w, inp, got = full
    args = {k: v.cuda() for k, v in inp.items() if k in WEIGHTS}
    x = inp["x"].cuda()
    x2 = x.clone()
    x2[:, -1] = -x2[:, -1] + 0.5
    y2 = _forward(x2, args, w)
    assert torch.equal(y2[:, :-1], got["y"][:, :-1])
    assert not torch.equal(y2[:, -1], got["y"][:, -1])
    del x2, y2
    tp = w.T // 8
    yp = _forward(x[:, :tp].contiguous(), args, w)  # tables keep T rows; the first tp are read
    assert torch.equal(yp, got["y"][:, :tp])


def test_wide_head_full_length_matches_oracle():
    """The wide-head workload's sequence shape at full length (B=1, T=8192,
    C=1024, H=8, N=128) against the fp32 oracle: output, all gradients,
    per-token y and dx."""
    w = WORKLOADS[3]
    print(f"\n{w.name}: B=1 at full length against the oracle", flush=True)
    check_block(w, B=1)
