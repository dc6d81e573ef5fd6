"""GPU parity of the HIP block against the CPU fp32 oracle (and its stages).

Every case prints its shape through the test id. Sizes are chosen so the CPU
oracle finishes in seconds; full-size properties are covered in
test_gpu_fullsize.py.
"""
import math

import pytest
import torch

from memory_efficient_attn_layer_amd import stages
from memory_efficient_attn_layer_amd.synthetic import WORKLOADS, Workload, make_inputs
from oracle import block as ob
from tests.parity_util import assert_grad_close, assert_out_close, check_block, gpu_block

pytestmark = pytest.mark.gpu

W0, W1, W2, W3 = (WORKLOADS[i] for i in range(4))


def _w(name, B, T, C, H, N, scale=1.0, L0=None):
    return Workload(99, name, B, T, C, H, N, scale, L0)


STAGE_CASES = [
    ("cfg0", W0, None),
    ("cfg1-b1-t1024", _w("c1", 1, 1024, 512, 8, 64), None),
    ("cfg3-b1-t512", _w("c3", 1, 512, 1024, 8, 128), None),
    ("ragged-b3-t77", _w("r", 3, 77, 256, 2, 64), None),
    ("yarn4-b1-t300", _w("y", 1, 300, 512, 4, 64, 4.0, 128), None),
    ("n32-yarn4-b2-t300", _w("n32", 2, 300, 256, 8, 32, 4.0, 128), None),
    # Forward-only widths (C > 1024): the output projection in 256- and
    # 512-feature groups.
    ("c1280-h4-b1-t64", _w("c1280", 1, 64, 1280, 4, 64), None),
    ("c2048-h8-n128-b1-t64", _w("c2048", 1, 64, 2048, 8, 128), None),
    ("c16384-h4-n128-b1-t32", _w("c16384", 1, 32, 16384, 4, 128), None),
]


@pytest.mark.parametrize("label,w,B", STAGE_CASES, ids=[c[0] for c in STAGE_CASES])
def test_stage_qkvg_projection(label, w, B):
    inp = make_inputs(w, B=B)
    g = {k: v.cuda() for k, v in inp.items()}
    q, k, v, sig, rx, rq, rk = stages.qkvg_proj(g["x"], g["wq"], g["wk"], g["wv"], g["wg"], g["f1"], g["f2"],
                                                w.H, w.N, stats=True)
    torch.cuda.synchronize()
    it = ob.block_intermediates(*(inp[n].float() for n in ("x", "wq", "wk", "wv", "wg", "wo", "f1", "f2")),
                                w.H, w.N)
    assert_out_close("q", q.transpose(1, 2), it["q"])
    assert_out_close("k", k.transpose(1, 2), it["k"])
    assert_out_close("v", v.transpose(1, 2), it["v"])
    assert_out_close("sig", sig, it["sig"])
    xf = inp["x"].float()
    rx_ref = torch.rsqrt(xf.pow(2).mean(-1) + 1e-6)
    assert_out_close("rx", rx, rx_ref, 1e-4)
    aq = it["a_q"]
    rq_ref = torch.rsqrt(aq.pow(2).mean(-1) + 1e-6).transpose(1, 2)
    assert_out_close("rq", rq, rq_ref, 2e-3)


@pytest.mark.parametrize("label,w,B", STAGE_CASES, ids=[c[0] for c in STAGE_CASES])
def test_stage_attention_forward(label, w, B):
    Bv = w.B if B is None else B
    gen = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(Bv, w.H, w.T, w.N, generator=gen).to(torch.bfloat16) for _ in range(3))
    o, lse = stages.attn_fwd(q.cuda(), k.cuda(), v.cuda(), C=w.C)
    torch.cuda.synchronize()
    qf, kf, vf = (t.float().transpose(1, 2) for t in (q, k, v))
    ref = ob.causal_attention(qf, kf, vf).reshape(Bv, w.T, w.H * w.N)
    assert_out_close("o", o, ref)
    s = torch.einsum("bhtn,bhun->bhtu", q.float(), k.float()) / math.sqrt(w.N)
    s = s.masked_fill(~torch.ones(w.T, w.T, dtype=torch.bool).tril(), float("-inf"))
    lse_ref = torch.logsumexp(s, -1)
    assert float((lse.cpu() - lse_ref).abs().max()) < 1e-3


@pytest.mark.parametrize("label,w,B", STAGE_CASES, ids=[c[0] for c in STAGE_CASES])
def test_stage_gate_oproj(label, w, B):
    Bv = w.B if B is None else B
    gen = torch.Generator().manual_seed(11)
    HN = w.H * w.N
    o = torch.randn(Bv, w.T, HN, generator=gen).to(torch.bfloat16)
    sig = torch.rand(Bv, w.T, HN, generator=gen).to(torch.bfloat16)
    wo = ((torch.rand(w.C, HN, generator=gen) * 2 - 1) * 0.5 / math.sqrt(w.C)).to(torch.bfloat16)
    y = stages.gate_oproj(o.cuda(), sig.cuda(), wo.cuda(), w.H, w.N)
    torch.cuda.synchronize()
    ref = (o.float() * sig.float()) @ wo.float().T
    assert_out_close("y", y, ref)


BLOCK_CASES = [
    ("cfg0-full", W0, None),
    ("cfg1-b1-t4096", W1, 1),
    ("cfg2-yarn4-b1-t2048", _w("c2", 1, 2048, 512, 8, 64, 4.0, 8192), None),
    ("cfg3-b1-t1024", _w("c3", 1, 1024, 1024, 8, 128), None),
    ("ragged-b3-t77", _w("r", 3, 77, 256, 2, 64), None),
    ("ragged-b2-t200-n128", _w("r2", 2, 200, 256, 2, 128), None),
    ("t1-b2", _w("t1", 2, 1, 256, 4, 64), None),
    ("t129-b1", _w("t129", 1, 129, 512, 8, 64), None),
    ("c-ne-hn-b2-t160", _w("chn", 2, 160, 512, 4, 64), None),
    ("c768-b1-t100", _w("c768", 1, 100, 768, 4, 64), None),
    ("yarn8-b2-t300-n128", _w("y8", 2, 300, 256, 2, 128, 8.0, 64), None),
    # H*N not a multiple of 256: the dZ kernel's last feature group is partial.
    ("h5-hn320-b1-t150", _w("h5", 1, 150, 256, 5, 64), None),
    ("h3-hn192-b2-t70", _w("h3", 2, 70, 512, 3, 64), None),
    # C > 1024: dx walks the features in groups of 1024 (the last one partial
    # for C = 1280); the prefill widths (C = H*N = 2048, N = 128, YaRN s = 8).
    ("c1280-h5-b2-t100", _w("c1280", 2, 100, 1280, 5, 64), None),
    ("c2048-h16-n128-yarn8-b1-t256", _w("c2048", 1, 256, 2048, 16, 128, 8.0, 64), None),
    ("c3072-h4-b1-t64", _w("c3072", 1, 64, 3072, 4, 64), None),
    # Wide models: dx walks 4, 5, 8 and 16 feature groups of 1024 (C > H*N
    # and C = H*N), the output projection and dZ take a grid column per
    # feature group; 16384 is the widest model the library accepts.
    ("c4096-h4-n128-b1-t48", _w("c4096", 1, 48, 4096, 4, 128), None),
    ("c5120-h40-n128-b1-t40", _w("c5120", 1, 40, 5120, 40, 128), None),
    ("c8192-h8-n128-yarn4-b2-t24", _w("c8192", 2, 24, 8192, 8, 128, 4.0, 16), None),
    ("c16384-h4-n128-b1-t20", _w("c16384", 1, 20, 16384, 4, 128), None),
    # C a multiple of 64 but not of 256 (any head count H at C = H*N): dx runs
    # the next wider layout with the features past C masked, the output
    # projection and dW end in partial 256-feature tiles.
    ("c384-h6-b2-t130", _w("c384", 2, 130, 384, 6, 64), None),
    ("c640-h5-n128-b1-t200", _w("c640", 1, 200, 640, 5, 128), None),
    ("c192-h3-b2-t90", _w("c192", 2, 90, 192, 3, 64), None),
    ("c64-h1-b2-t100", _w("c64", 2, 100, 64, 1, 64), None),
    ("c320-ne-hn-h2-n128-b1-t64", _w("c320", 1, 64, 320, 2, 128), None),
    ("c1344-h21-b1-t80", _w("c1344", 1, 80, 1344, 21, 64), None),
    # 768 < C <= 1024 with H*N >= 512: dx walks two 512-feature groups over
    # 128 tokens (the second partial here), da_g in dx (H*N <= C) or in its
    # own buffer (H*N > C); 300 tokens end in a partial block.
    ("c800-hn512-b2-t150", _w("c800", 2, 150, 800, 8, 64), None),
    ("c928-hn1024-n128-b1-t300", _w("c928", 1, 300, 928, 8, 128), None),
    # Heads of 32 dimensions with an even H run natively (projection tiles of
    # head pairs, 32-wide attention tiles); heads of 16 run zero-padded to
    # 32 (the head RMSNorm and the attention scale use the true width).
    ("n32-h8-c256-b2-t100", _w("n32", 2, 100, 256, 8, 32), None),
    ("n32-yarn4-h6-c192-b1-t300", _w("n32y", 1, 300, 192, 6, 32, 4.0, 128), None),
    ("n32-h16-c512-b1-t700", _w("n32l", 1, 700, 512, 16, 32), None),
    ("n32-h2-c640-b2-t129", _w("n32c", 2, 129, 640, 2, 32), None),
    ("n32-t1-h4-c128-b3", _w("n32t1", 3, 1, 128, 4, 32), None),
    ("n32-ragged-h2-c64-b3-t77", _w("n32r", 3, 77, 64, 2, 32), None),
    ("n16-h4-c64-b2-t70", _w("n16", 2, 70, 64, 4, 16), None),
    ("n16-yarn4-h8-c128-b1-t333", _w("n16y", 1, 333, 128, 8, 16, 4.0, 64), None),
    # C = H*N a multiple of 32 only (odd H with N = 32 or 16: one zero head
    # added; H = 2 with N = 16; a wide C whose last dx feature group holds 32
    # features).
    ("n32-h3-c96-b2-t90", _w("n32h3", 2, 90, 96, 3, 32), None),
    ("n16-h2-c32-b2-t64", _w("n16h2", 2, 64, 32, 2, 16), None),
    ("n32-h33-c1056-b1-t50", _w("n32w", 1, 50, 1056, 33, 32), None),
    ("n16-h5-c96-b1-t60", _w("n16h5", 1, 60, 96, 5, 16), None),
    # Heads of 256 dimensions: one wave per SIMD in the attention kernels,
    # 32-query tiles in dK/dV, the projection's and dZ's head sums over two
    # waves.
    ("n256-h2-c512-b2-t130", _w("n256", 2, 130, 512, 2, 256), None),
    ("n256-yarn4-h3-c768-b1-t200", _w("n256y", 1, 200, 768, 3, 256, 4.0, 64), None),
    ("n256-h1-c256-b1-t70", _w("n256h1", 1, 70, 256, 1, 256), None),
]


@pytest.mark.parametrize("label,w,B", BLOCK_CASES, ids=[c[0] for c in BLOCK_CASES])
def test_block_forward_backward(label, w, B):
    check_block(w, B=B)


# The same block with tables that take no gradient (df1 = df2 = NULL), the
# case of a module whose tables are buffers: the attention backward then runs
# its other kernel forms (one head per workgroup, three workgroups per CU at
# N = 64, the row tails' operands fetched in one round trip).
BUFFER_TABLE_CASES = [c for c in BLOCK_CASES if c[0] in {
    "cfg0-full", "cfg1-b1-t4096", "cfg2-yarn4-b1-t2048", "cfg3-b1-t1024", "ragged-b3-t77", "ragged-b2-t200-n128",
    "t129-b1", "yarn8-b2-t300-n128", "h5-hn320-b1-t150", "c2048-h16-n128-yarn8-b1-t256", "n32-h8-c256-b2-t100",
    "n16-h4-c64-b2-t70", "n256-h2-c512-b2-t130", "n256-yarn4-h3-c768-b1-t200", "n256-h1-c256-b1-t70",
    "n32-h16-c512-b1-t700", "n32-h3-c96-b2-t90"}]


@pytest.mark.parametrize("label,w,B", BUFFER_TABLE_CASES, ids=[c[0] for c in BUFFER_TABLE_CASES])
def test_block_forward_backward_buffer_tables(label, w, B):
    got, _ = check_block(w, B=B, table_grad=False)
    assert got["df1"] is None and got["df2"] is None


@pytest.mark.parametrize("tscale", [2.0, 2.5], ids=["fixed-offset-wide-range", "online-fallback"])
def test_block_logit_range(tscale):
    """Rotary tables scaled by tscale widen the logit range. The block bounds
    every logit by |q| |k| log2(e)/sqrt(N) (about 11.5 tscale^2 here): 2.0
    (~46) keeps the fixed-offset softmax with probabilities down to 2^-92 of
    the largest, 2.5 (~72) exceeds its limit of 60 and takes the online
    softmax. Both must match the oracle."""
    inp = make_inputs(W0, B=1)
    f1 = (inp["f1"].float() * tscale).to(torch.bfloat16)
    f2 = (inp["f2"].float() * tscale).to(torch.bfloat16)
    check_block(W0, B=1, f1=f1, f2=f2)


def test_block_without_table_grad_matches():
    got, _ = check_block(W0, table_grad=False)
    assert got["df1"] is None and got["df2"] is None


def test_zero_o_proj_known_answer():
    """README.md:35 initialises o_proj to zero: y must be exactly 0 and every
    gradient except dWo exactly 0."""
    inp = make_inputs(W0)
    inp["wo"] = torch.zeros_like(inp["wo"])
    got = gpu_block(inp, W0.H, W0.N)
    assert torch.count_nonzero(got["y"]) == 0
    for k in ("dx", "dwq", "dwk", "dwv", "dwg", "df1", "df2"):
        assert torch.count_nonzero(got[k]) == 0, k
    ref = ob.block_grads(inp, W0.H, W0.N)
    assert_grad_close("dwo", got["dwo"], ref["dwo"])


def test_zero_gate_known_answer():
    """Wg = 0 gives sigmoid = 1/2 exactly: y equals half the projection of o."""
    inp = make_inputs(W0)
    inp["wg"] = torch.zeros_like(inp["wg"])
    g = {k: v.cuda() for k, v in inp.items()}
    q, k, v, sig = stages.qkvg_proj(g["x"], g["wq"], g["wk"], g["wv"], g["wg"], g["f1"], g["f2"], W0.H, W0.N)
    assert torch.all(sig == 0.5)


@pytest.mark.parametrize("table_grad", [False, True], ids=["buffers", "trainable-tables"])
def test_deterministic(table_grad):
    """Two runs are bitwise equal, table gradients included (their sum over
    batch and heads runs in a fixed order)."""
    inp = make_inputs(W0)
    a = gpu_block(inp, W0.H, W0.N, table_grad=table_grad)
    b = gpu_block(inp, W0.H, W0.N, table_grad=table_grad)
    keys = ("y", "dx", "dwq", "dwk", "dwv", "dwg", "dwo") + (("df1", "df2") if table_grad else ())
    for k in keys:
        assert torch.equal(a[k], b[k]), k


def _module_and_tables(C, H, N, T, scale=1.0, L0=None, seed=21):
    from memory_efficient_attn_layer_amd.module import CausalSoftmaxAttention
    from memory_efficient_attn_layer_amd.yarn import Yarn

    torch.manual_seed(seed)
    m = CausalSoftmaxAttention(C, H, N)
    with torch.no_grad():  # README.md:35 zeroes o_proj; give it values so every gradient flows
        m.o_proj.weight.uniform_(-0.5 / math.sqrt(C), 0.5 / math.sqrt(C))
    m = m.bfloat16().cuda()
    yarn = Yarn(N, T, scale=scale, original_context=L0, device="cuda")
    return m, yarn


def test_module_forward_backward_matches_oracle():
    """The drop-in call path: CausalSoftmaxAttention.forward -> fused_attn
    (README.md:37-68, fast_triton_attn.py:681-697) with Parameters and a Yarn
    table module, then loss.backward(); every Parameter .grad and x.grad
    against the oracle."""
    C, H, N, T = 512, 8, 64, 256
    m, yarn = _module_and_tables(C, H, N, T, scale=4.0, L0=64)
    g = torch.Generator().manual_seed(5)
    x0 = torch.randn(2, T, C, generator=g).bfloat16()
    dy = torch.randn(2, T, C, generator=g).bfloat16()
    x = x0.cuda().requires_grad_(True)
    y = m(x, yarn)
    assert y.grad_fn is not None
    (y.float() * dy.cuda().float()).sum().backward()
    torch.cuda.synchronize()
    inp = dict(x=x0, wq=m.q_proj.weight, wk=m.k_proj.weight, wv=m.v_proj.weight, wg=m.g_proj.weight,
               wo=m.o_proj.weight, f1=yarn.factor1, f2=yarn.factor2, dy=dy)
    ref = ob.block_grads(inp, H, N)
    assert_out_close("y", y, ref["y"])
    assert_grad_close("x.grad", x.grad, ref["dx"])
    for name, k in (("q_proj", "dwq"), ("k_proj", "dwk"), ("v_proj", "dwv"), ("g_proj", "dwg"), ("o_proj", "dwo")):
        assert_grad_close(f"{name}.weight.grad", getattr(m, name).weight.grad, ref[k])
    assert yarn.factor1.grad is None  # table buffers receive no gradient


@pytest.mark.parametrize("mode", ["no_grad", "inference_mode"])
def test_module_inference_at_wide_width_saves_nothing(mode):
    """Inference through the module at the prefill widths (C=2048, H=16,
    N=128; C > 1024 has no backward): runs, matches the oracle, keeps no
    graph and allocates no O / lse (the peak stays below what saving them
    would add to y, the workspace and the fp32 tables)."""
    from memory_efficient_attn_layer_amd import _lib

    C, H, N, T = 2048, 16, 128, 256
    m, yarn = _module_and_tables(C, H, N, T, scale=8.0, L0=64)
    x0 = torch.randn(1, T, C, generator=torch.Generator().manual_seed(9)).bfloat16()
    x = x0.cuda()
    ctx = torch.no_grad() if mode == "no_grad" else torch.inference_mode()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    with ctx:
        y = m(x, yarn)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    assert y.grad_fn is None
    M, HN = T, H * N
    d = _lib.desc(1, T, C, H, N, T, 1e-6)
    ws = _lib.load().mea_workspace_bytes(d, _lib.MEA_PASS_FWD)
    no_save = M * C * 2 + ws + 2 * T * N * 4
    saves = M * HN * 2 + H * M * 4
    assert peak < no_save + saves // 2, (peak, no_save, saves)
    inp = dict(x=x0, wq=m.q_proj.weight, wk=m.k_proj.weight, wv=m.v_proj.weight, wg=m.g_proj.weight,
               wo=m.o_proj.weight, f1=yarn.factor1, f2=yarn.factor2)
    ref = ob.block_forward(*(inp[n].detach().float().cpu() for n in ("x", "wq", "wk", "wv", "wg", "wo", "f1", "f2")),
                           H, N)
    assert_out_close("y", y, ref)


def test_inference_forward_matches_training_forward():
    inp = make_inputs(W0)
    g = {k: v.cuda() for k, v in inp.items()}
    args = [g[n] for n in ("x", "wq", "wk", "wv", "wg", "wo", "f1", "f2")]
    from memory_efficient_attn_layer_amd.attention import FusedAttentionFunction

    with torch.no_grad():
        y0 = FusedAttentionFunction.apply(*args, W0.H, W0.N, 1e-6)
    y1 = gpu_block(inp, W0.H, W0.N)["y"]
    assert torch.equal(y0, y1)
