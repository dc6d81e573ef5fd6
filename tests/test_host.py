"""Host-side checks that need no GPU: the C ABI library loads and exports
every function include/mea.h declares, its argument validation returns the
documented status before touching any pointer, and the Python wrapper
rejects unsupported inputs before any launch."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from memory_efficient_attn_layer_amd import _lib
from memory_efficient_attn_layer_amd.attention import FusedAttentionFunction, fused_attn
from memory_efficient_attn_layer_amd.module import CausalSoftmaxAttention
from memory_efficient_attn_layer_amd.yarn import Yarn

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mea.h"


def _header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mea_\w+)\s*\(", text, flags=re.M)))


def _header_enum(name):
    m = re.search(rf"{name}\s*=\s*(-?\d+)", HEADER.read_text())
    return int(m.group(1))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built; run python -m memory_efficient_attn_layer_amd.build")
    return _lib.load()


def test_library_exports_every_declared_function(lib):
    declared = _header_functions()
    assert set(declared) == set(_lib.EXPORTS), (declared, sorted(_lib.EXPORTS))
    for name in declared:
        assert hasattr(lib, name), name


def test_strerror_and_version(lib):
    for code in range(0, -12, -1):
        msg = _lib.strerror(code)
        assert msg and msg != "unknown status", code
    assert _lib.strerror(-1234) == "unknown status"
    assert lib.mea_version().decode().startswith("mea ")


def test_profile_select_bounds(lib):
    """mea_profile_select takes -1 (every kernel) or a kernel id; the
    selection is host state only (no GPU call)."""
    n = 0
    while lib.mea_profile_kernel_name(n) is not None:
        n += 1
    err = _header_enum("MEA_ERR_NULL")
    assert lib.mea_profile_select(-2) == err
    assert lib.mea_profile_select(n) == err
    for k in (-1, 0, n - 1):
        assert lib.mea_profile_select(k) == 0
    lib.mea_profile_select(-1)
    _lib.profile_select("attn_bwd_dkdv")
    _lib.profile_select(None)
    with pytest.raises(ValueError):
        _lib.profile_select("no_such_kernel")


def _d(B=2, T=256, C=256, H=4, N=64, T_max=None, eps=1e-6, N_active=0):
    return _lib.desc(B, T, C, H, N, T if T_max is None else T_max, eps, N_active)


def test_workspace_bytes(lib):
    assert lib.mea_workspace_bytes(None, 0) == 0
    assert lib.mea_workspace_bytes(ctypes.byref(_d()), 7) == 0
    fwd = lib.mea_workspace_bytes(ctypes.byref(_d()), _lib.MEA_PASS_FWD)
    bwd = lib.mea_workspace_bytes(ctypes.byref(_d()), _lib.MEA_PASS_BWD)
    M, HN = 2 * 256, 4 * 64
    assert fwd >= 5 * M * HN * 2
    assert bwd > fwd
    # Table gradients need per-token partials: B * T * 2N fp32 more.
    tab = lib.mea_workspace_bytes(ctypes.byref(_d()), _lib.MEA_PASS_BWD_TABLES)
    assert tab - bwd >= M * 2 * 64 * 4
    # bf16-valued tables: a packed bf16 copy of T rows (8 bytes per row and
    # feature) in every pass's workspace.
    for ps in (_lib.MEA_PASS_FWD, _lib.MEA_PASS_BWD, _lib.MEA_PASS_BWD_TABLES):
        d16 = _lib.desc(2, 256, 256, 4, 64, 256, 1e-6, 0, True)
        plain = lib.mea_workspace_bytes(ctypes.byref(_d()), ps)
        assert lib.mea_workspace_bytes(ctypes.byref(d16), ps) - plain == 256 * 64 * 4
    # Invalid descriptors report 0.
    for bad in (_d(N=96), _d(C=300), _d(T_max=10), _d(eps=0.0), _d(B=0)):
        assert lib.mea_workspace_bytes(ctypes.byref(bad), 0) == 0
    # The backward's head-major gradient offsets limit H * (T + 256) * N to
    # 2^30; the forward has no such limit.
    long_t = _d(B=1, T=1 << 20, T_max=1 << 20, C=1024, H=8, N=128)
    assert lib.mea_workspace_bytes(ctypes.byref(long_t), _lib.MEA_PASS_FWD) > 0
    assert lib.mea_workspace_bytes(ctypes.byref(long_t), _lib.MEA_PASS_BWD) == 0
    ok_t = _d(B=1, T=(1 << 20) - 512, T_max=1 << 20, C=1024, H=8, N=128)
    assert lib.mea_workspace_bytes(ctypes.byref(ok_t), _lib.MEA_PASS_BWD) > 0


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(N=32, H=3), "MEA_ERR_HEAD_DIM"),
        (dict(N=16), "MEA_ERR_HEAD_DIM"),
        (dict(N=32, N_active=8), "MEA_ERR_HEAD_DIM"),
        (dict(N=512), "MEA_ERR_HEAD_DIM"),
        (dict(N_active=48), "MEA_ERR_HEAD_DIM"),
        (dict(N=128, N_active=32), "MEA_ERR_HEAD_DIM"),
        (dict(C=336), "MEA_ERR_MODEL_DIM"),
        (dict(C=16), "MEA_ERR_MODEL_DIM"),
        (dict(T_max=100), "MEA_ERR_SHAPE"),
        (dict(H=0), "MEA_ERR_SHAPE"),
        (dict(eps=-1.0), "MEA_ERR_EPS"),
        (dict(eps=float("nan")), "MEA_ERR_EPS"),
    ],
)
def test_descriptor_validation_before_launch(lib, kw, code):
    d = _d(**kw)
    z = [None] * 32
    assert lib.mea_fwd(ctypes.byref(d), *z[:12], 0, None) == _header_enum(code)
    assert lib.mea_bwd(ctypes.byref(d), *z[:20], 0, None) == _header_enum(code)


def test_pointer_and_workspace_validation(lib):
    d = _d()
    fake = 1 << 20  # aligned, never dereferenced: validation fails first
    args = [fake] * 6 + [fake, fake, fake, fake, fake, fake]
    assert lib.mea_fwd(ctypes.byref(d), None, *args[1:], 10, None) == _header_enum("MEA_ERR_NULL")
    assert lib.mea_fwd(ctypes.byref(d), fake + 2, *args[1:], 10, None) == _header_enum("MEA_ERR_ALIGN")
    # Only one of o_save / lse_save.
    a2 = list(args)
    a2[9] = None
    assert lib.mea_fwd(ctypes.byref(d), fake, *a2[1:], 10, None) == _header_enum("MEA_ERR_NULL")
    # Workspace too small.
    assert lib.mea_fwd(ctypes.byref(d), fake, *args[1:], 10, None) == _header_enum("MEA_ERR_WORKSPACE")
    # mea_bwd pointers: dy x wq wk wv wg wo f1 f2 o lse dx dwq dwk dwv dwg dwo df1 df2 ws
    # (distinct, far apart: dx may overlap nothing else)
    bargs = [(1 << 32) + i * (1 << 28) for i in range(20)]
    b_dwo_null = list(bargs)
    b_dwo_null[16] = None
    assert lib.mea_bwd(ctypes.byref(d), *b_dwo_null, 10, None) == _header_enum("MEA_ERR_NULL")
    b_one_df = list(bargs)
    b_one_df[18] = None
    assert lib.mea_bwd(ctypes.byref(d), *b_one_df, 10, None) == _header_enum("MEA_ERR_NULL")
    assert lib.mea_bwd(ctypes.byref(d), *bargs, 10, None) == _header_enum("MEA_ERR_WORKSPACE")
    # The backward-only workspace is too small once table gradients are asked for.
    wsb = lib.mea_workspace_bytes(ctypes.byref(d), _lib.MEA_PASS_BWD)
    assert lib.mea_bwd(ctypes.byref(d), *bargs, wsb, None) == _header_enum("MEA_ERR_WORKSPACE")
    # dx overlapping another argument (it holds a transient before the
    # result): refused before the workspace is even looked at.
    for other in (0, 1, 9, 19):
        b_alias = list(bargs)
        b_alias[11] = bargs[other] + (4096 if other != 19 else 0)  # the workspace is 10 bytes here
        assert lib.mea_bwd(ctypes.byref(d), *b_alias, 10, None) == _header_enum("MEA_ERR_ALIAS")
    # C above 16384, or H*N*C of 2^29 or more (32-bit weight element
    # indices), is refused in both passes.
    d2 = _d(C=16416)
    assert lib.mea_bwd(ctypes.byref(d2), *bargs, 1 << 40, None) == _header_enum("MEA_ERR_MODEL_DIM")
    d3 = _d(C=16384, H=256, N=128)
    assert lib.mea_bwd(ctypes.byref(d3), *bargs, 1 << 40, None) == _header_enum("MEA_ERR_MODEL_DIM")
    assert lib.mea_workspace_bytes(ctypes.byref(d3), _lib.MEA_PASS_FWD) == 0
    assert lib.mea_workspace_bytes(ctypes.byref(_d(C=2048, H=16, N=128)), _lib.MEA_PASS_BWD) > 0
    assert lib.mea_workspace_bytes(ctypes.byref(_d(C=16384, H=8, N=128)), _lib.MEA_PASS_BWD) > 0


def test_decode_and_prefill_validation(lib):
    fake = 1 << 20  # aligned, never dereferenced: validation fails first
    d = _d(T=512, T_max=512)  # decode: T is the cache capacity
    assert lib.mea_decode_workspace_bytes(None) == 0
    assert lib.mea_decode_workspace_bytes(ctypes.byref(_d(N=96))) == 0
    need = lib.mea_decode_workspace_bytes(ctypes.byref(d))
    # the fp32 products and the bf16 q, sigmoid(g), O of the B new tokens
    assert need >= 2 * (4 * 4 * 64 * 4 + 3 * 4 * 64 * 2)
    # decode pointers: x wq wk wv wg wo f1 f2 pos k_cache v_cache y ws
    dargs = [fake] * 13
    assert lib.mea_decode(ctypes.byref(d), *dargs, 10, None) == _header_enum("MEA_ERR_WORKSPACE")
    no_pos = list(dargs)
    no_pos[8] = None
    assert lib.mea_decode(ctypes.byref(d), *no_pos, need, None) == _header_enum("MEA_ERR_NULL")
    odd_pos = list(dargs)
    odd_pos[8] = fake + 2
    assert lib.mea_decode(ctypes.byref(d), *odd_pos, need, None) == _header_enum("MEA_ERR_ALIGN")
    no_cache = list(dargs)
    no_cache[9] = None
    assert lib.mea_decode(ctypes.byref(d), *no_cache, need, None) == _header_enum("MEA_ERR_NULL")
    # Cache capacity beyond the rotary tables.
    assert lib.mea_decode(ctypes.byref(_d(T=600, T_max=512)), *dargs, need, None) == _header_enum("MEA_ERR_SHAPE")
    # prefill pointers: x wq wk wv wg wo f1 f2 y k_cache v_cache, cache_T, ws
    pd = _d(T=64, T_max=128)
    pargs = [fake] * 11
    assert lib.mea_prefill(ctypes.byref(pd), *pargs, 32, fake, 1 << 40, None) == _header_enum("MEA_ERR_SHAPE")
    assert lib.mea_prefill(ctypes.byref(pd), *pargs, 256, fake, 1 << 40, None) == _header_enum("MEA_ERR_SHAPE")
    assert lib.mea_prefill(ctypes.byref(pd), *pargs, 128, fake, 10, None) == _header_enum("MEA_ERR_WORKSPACE")
    p_no_cache = list(pargs)
    p_no_cache[10] = None
    assert lib.mea_prefill(ctypes.byref(pd), *p_no_cache, 128, fake, 1 << 40, None) == _header_enum("MEA_ERR_NULL")


def test_varlen_validation(lib):
    fake = 1 << 20  # aligned, never dereferenced: validation fails first
    # fwd pointers after (cu, nseq, max_len): x wq wk wv wg wo f1 f2 y o lse ws
    fargs = [fake] * 12
    # T (total tokens) may exceed T_max: the tables need max_len rows only.
    d = _d(B=1, T=1000, T_max=300)
    ok_shape = lib.mea_fwd_varlen(ctypes.byref(d), fake, 4, 300, *fargs, 10, None)
    assert ok_shape == _header_enum("MEA_ERR_WORKSPACE")
    for dd, nseq, max_len, code in [
        (_d(B=2, T=1000, T_max=300), 4, 300, "MEA_ERR_SHAPE"),  # packed batches have B = 1
        (d, 0, 300, "MEA_ERR_SHAPE"),
        (d, 4, 301, "MEA_ERR_SHAPE"),                            # longer than the tables
        (_d(B=1, T=200, T_max=300), 4, 250, "MEA_ERR_SHAPE"),    # longer than the total
        (d, 4, 0, "MEA_ERR_SHAPE"),
    ]:
        assert lib.mea_fwd_varlen(ctypes.byref(dd), fake, nseq, max_len, *fargs, 10, None) == _header_enum(code)
    assert lib.mea_fwd_varlen(ctypes.byref(d), None, 4, 300, *fargs, 10, None) == _header_enum("MEA_ERR_NULL")
    assert lib.mea_fwd_varlen(ctypes.byref(d), fake + 2, 4, 300, *fargs, 10, None) == _header_enum("MEA_ERR_ALIGN")
    # bwd: dy x wq wk wv wg wo f1 f2 o lse dx dwq dwk dwv dwg dwo df1 df2 ws
    bargs = [(1 << 32) + i * (1 << 28) for i in range(20)]
    assert lib.mea_bwd_varlen(ctypes.byref(d), fake, 4, 300, *bargs, 10, None) == _header_enum("MEA_ERR_WORKSPACE")
    assert lib.mea_bwd_varlen(ctypes.byref(_d(B=1, T=1000, T_max=300, C=16416)), fake, 4, 300, *bargs, 1 << 40,
                              None) == _header_enum("MEA_ERR_MODEL_DIM")


def _cpu_args(B=1, T=8, C=256, H=4, N=64, dtype=torch.bfloat16):
    HN = H * N
    x = torch.randn(B, T, C, dtype=dtype)
    ws = [torch.zeros(HN, C, dtype=dtype) for _ in range(4)] + [torch.zeros(C, HN, dtype=dtype)]
    f1 = torch.ones(T, N, dtype=dtype)
    f2 = torch.zeros(T, N, dtype=dtype)
    return x, ws, f1, f2


@pytest.mark.parametrize(
    "mutate,exc",
    [
        (lambda a: a.update(x=a["x"].float()), TypeError),
        (lambda a: a.update(N=32), ValueError),
        (lambda a: a.update(H=0), ValueError),
        (lambda a: a.update(f1=a["f1"][:4], f2=a["f2"][:4]), ValueError),
        (lambda a: a.update(x=a["x"][:, :, :128]), ValueError),
        (lambda a: a.update(eps=0.0), ValueError),
        (lambda a: None, RuntimeError),  # valid shapes but on the CPU: no fallback
    ],
)
def test_python_validation(mutate, exc):
    x, ws, f1, f2 = _cpu_args()
    a = dict(x=x, f1=f1, f2=f2, N=64, H=4, eps=1e-6)
    mutate(a)
    with pytest.raises(exc):
        FusedAttentionFunction.apply(a["x"], *ws, a["f1"], a["f2"], a["H"], a["N"], a["eps"])


def test_module_and_tables_construct_on_cpu():
    m = CausalSoftmaxAttention(256, 4, 64)
    assert torch.all(m.o_proj.weight == 0)
    bound = 0.5 / 256 ** 0.5
    assert m.q_proj.weight.abs().max() <= bound and m.q_proj.bias is None
    y = Yarn(64, 128)
    assert y.factor1.shape == (128, 64) and y.factor1.dtype == torch.bfloat16
    x = torch.randn(1, 8, 256, dtype=torch.bfloat16)
    with pytest.raises(TypeError):  # fp32 weights of a fresh nn.Linear are rejected like the reference would
        fused_attn(x, m.q_proj, m.k_proj, m.v_proj, m.g_proj, m.o_proj, y, 4, 64)


def test_save_decision_follows_grad_mode(monkeypatch):
    """Whether the forward saves activations is decided from grad mode and
    requires_grad before Function.forward runs (inside it grad mode is always
    off, and ctx.needs_input_grad reports True for a Parameter even under
    no_grad): no_grad / inference_mode and parameters that need no grad all
    give need_backward=False."""
    import memory_efficient_attn_layer_amd.attention as att

    seen = []

    def record(x, weights, f1, f2, H, N, eps, need_backward):
        seen.append(need_backward)
        raise RuntimeError("validation reached")

    monkeypatch.setattr(att, "_validate", record)
    m = CausalSoftmaxAttention(256, 4, 64).bfloat16()
    y = Yarn(64, 16)
    x = torch.randn(1, 16, 256, dtype=torch.bfloat16)
    for ctx in (torch.no_grad, torch.inference_mode):
        with ctx(), pytest.raises(RuntimeError, match="validation reached"):
            m(x, y)
        assert seen[-1] is False
    with pytest.raises(RuntimeError, match="validation reached"):
        m(x, y)
    assert seen[-1] is True
    for p in m.parameters():
        p.requires_grad_(False)
    with pytest.raises(RuntimeError, match="validation reached"):
        m(x, y)
    assert seen[-1] is False
    with pytest.raises(RuntimeError, match="validation reached"):
        m(x.requires_grad_(True), y)  # an input that needs grad is enough
    assert seen[-1] is True


def test_static_decode_validation(lib):
    """mea_decode_static checks its arguments, then refuses a shape whose
    scratch exceeds the static buffer, before touching the device."""
    fake = 1 << 20  # aligned, never dereferenced: validation fails first
    dargs = [fake] * 12  # x wq wk wv wg wo f1 f2 pos k_cache v_cache y
    d = _d(T=512, T_max=512)
    no_pos = list(dargs)
    no_pos[8] = None
    assert lib.mea_decode_static(ctypes.byref(d), *no_pos, None) == _header_enum("MEA_ERR_NULL")
    assert lib.mea_decode_static(ctypes.byref(_d(N=96)), *dargs, None) == _header_enum("MEA_ERR_HEAD_DIM")
    assert lib.mea_workspace_bytes(ctypes.byref(_d(N=256, C=512, H=2)), _lib.MEA_PASS_BWD) > 0
    assert lib.mea_decode_workspace_bytes(ctypes.byref(_d(N=256, C=512, H=2))) > 0
    big = _d(B=4096, T=512, T_max=512, C=2048, H=16, N=128)
    assert lib.mea_decode_workspace_bytes(ctypes.byref(big)) > _lib.MEA_STATIC_SCRATCH_BYTES
    assert lib.mea_decode_static(ctypes.byref(big), *dargs, None) == _header_enum("MEA_ERR_SCRATCH")
    m = re.search(r"#define MEA_STATIC_SCRATCH_BYTES \((\d+)u << (\d+)\)", HEADER.read_text())
    assert int(m.group(1)) << int(m.group(2)) == _lib.MEA_STATIC_SCRATCH_BYTES


def test_descriptor_accepts_narrow_heads(lib):
    """32-wide heads run natively with an even H; heads of 16 dimensions are
    described as N = 32 (or 64) with N_active; 32 with an odd H as N = 64
    (the Python API adds a zero head instead)."""
    for n_act in (0, 16, 32, 64):
        assert lib.mea_workspace_bytes(ctypes.byref(_d(N_active=n_act)), _lib.MEA_PASS_FWD) > 0
    for n_act in (0, 16, 32):
        assert lib.mea_workspace_bytes(ctypes.byref(_d(N=32, N_active=n_act)), _lib.MEA_PASS_BWD) > 0
    assert lib.mea_workspace_bytes(ctypes.byref(_d(N=128, N_active=128)), _lib.MEA_PASS_BWD) > 0


def test_storage_width_of_narrow_heads():
    """storage_shape: the (heads, head width) the library runs for each (H, N)."""
    from memory_efficient_attn_layer_amd.attention import storage_shape
    from memory_efficient_attn_layer_amd.decode import cache_heads, cache_width

    assert [storage_shape(4, n) for n in (16, 32, 64, 128, 256)] == [(4, 32), (4, 32), (4, 64), (4, 128), (4, 256)]
    assert [storage_shape(3, n) for n in (16, 32, 64, 128, 256)] == [(4, 32), (4, 32), (3, 64), (3, 128), (3, 256)]
    assert cache_width(32, 8) == 32 and cache_width(16, 8) == 32 and cache_width(32, 5) == 32
    assert cache_heads(32, 5) == 6 and cache_heads(16, 1) == 2 and cache_heads(64, 5) == 5


def test_pad_heads_layout_and_gradients():
    """The padding is differentiable and exact: every head keeps its N rows
    (columns of Wo, table columns) in place, the padding is zero (identity
    rotary pairs in the tables), and gradients of the padded tensors reach
    the caller's tensors as their slices."""
    from memory_efficient_attn_layer_amd.attention import _pad_heads

    PAD_N, PAD_H = 64, 4
    torch.manual_seed(0)
    H, N, C, T = 3, 32, 96, 10
    ws = [torch.randn(H * N, C, requires_grad=True) for _ in range(4)] + [torch.randn(C, H * N, requires_grad=True)]
    f1 = torch.randn(T, N, requires_grad=True)
    f2 = torch.randn(T, N, requires_grad=True)
    (wq, wk, wv, wg, wo), p1, p2 = _pad_heads(H, N, ws, f1, f2, PAD_N, PAD_H)
    assert wq.shape == (PAD_H * PAD_N, C) and wo.shape == (C, PAD_H * PAD_N) and p1.shape == (T, PAD_N)
    for h in range(H):
        assert torch.equal(wq[h * PAD_N:h * PAD_N + N], ws[0][h * N:(h + 1) * N])
        assert torch.count_nonzero(wq[h * PAD_N + N:(h + 1) * PAD_N]) == 0
        assert torch.equal(wo[:, h * PAD_N:h * PAD_N + N], ws[4][:, h * N:(h + 1) * N])
        assert torch.count_nonzero(wo[:, h * PAD_N + N:(h + 1) * PAD_N]) == 0
    # The added head is zero throughout.
    assert torch.count_nonzero(wq[H * PAD_N:]) == 0 and torch.count_nonzero(wo[:, H * PAD_N:]) == 0
    assert torch.equal(p1[:, :N], f1) and torch.all(p1[:, N:] == 1)
    assert torch.equal(p2[:, :N], f2) and torch.all(p2[:, N:] == 0)
    gq = torch.randn_like(wq)
    go = torch.randn_like(wo)
    g1 = torch.randn_like(p1)
    (wq * gq).sum().backward()
    (wo * go).sum().backward()
    (p1 * g1).sum().backward()
    assert torch.equal(ws[0].grad, gq.reshape(PAD_H, PAD_N, C)[:H, :N].reshape(H * N, C))
    assert torch.equal(ws[4].grad, go.reshape(C, PAD_H, PAD_N)[:, :H, :N].reshape(C, H * N))
    assert torch.equal(f1.grad, g1[:, :N])


def test_bf16_table_flag_follows_table_dtype():
    """The descriptor's tables_bf16 (packed bf16 table copy in the projection)
    is set only when both tables are bf16, whose values the fp32 copies hold
    exactly; fp16 and fp32 tables keep the fp32 reads."""
    from memory_efficient_attn_layer_amd.attention import _bf16_tables

    t = torch.zeros(8, 64)
    assert _bf16_tables(t.bfloat16(), t.bfloat16())
    for a, b in ((t, t), (t.half(), t.half()), (t.bfloat16(), t), (t.half(), t.bfloat16())):
        assert not _bf16_tables(a, b)
    d = _lib.desc(1, 8, 64, 1, 64, 8, 1e-6, 0, True)
    assert d.tables_bf16 == 1 and _lib.desc(1, 8, 64, 1, 64, 8, 1e-6).tables_bf16 == 0
    # Every bf16 number survives the round trip bf16 -> fp32 -> bf16 unchanged.
    vals = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    finite = vals[torch.isfinite(vals)]
    assert torch.equal(finite.float().bfloat16().view(torch.int16), finite.view(torch.int16))


def test_varlen_host_offsets_are_checked():
    """fused_attn_varlen checks offsets it holds on the host (a list or a CPU
    tensor) before any launch: a max_len below the longest sequence would
    leave that sequence's last rows unwritten, so it is an error."""
    from memory_efficient_attn_layer_amd.attention import check_offsets, fused_attn_varlen

    m = CausalSoftmaxAttention(256, 4, 64)
    yarn = Yarn(64, 512)
    x = torch.randn(300, 256).bfloat16()
    args = (x, m.q_proj, m.k_proj, m.v_proj, m.g_proj, m.o_proj, yarn, 4, 64)
    with pytest.raises(ValueError, match="below the longest"):
        fused_attn_varlen(*args, [0, 100, 300], max_len=150)
    with pytest.raises(ValueError, match="below the longest"):
        fused_attn_varlen(*args, torch.tensor([0, 100, 300], dtype=torch.int32), max_len=199)
    with pytest.raises(ValueError, match="nondecreasing"):
        fused_attn_varlen(*args, [0, 200, 100, 300])
    with pytest.raises(ValueError, match="from 0 to 300"):
        fused_attn_varlen(*args, [0, 100, 250])
    with pytest.raises(ValueError, match="nseq"):
        fused_attn_varlen(*args, [300])
    assert check_offsets([0, 100, 100, 300], 300) == 200  # empty sequences are fine


def test_attention_work_order_is_a_permutation(tmp_path):
    """The attention kernels' workgroup -> (b, h, block) order (attn_item in
    csrc/common.cuh: per-XCD ranges, the slot rotation, the heaviest-first
    tail) is a permutation for every grid size, blocks per head and slot
    count: compiled for the host from the kernels' own header and
    enumerated on the CPU (tests/work_order.cpp)."""
    import shutil
    import subprocess

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not found")
    exe = tmp_path / "work_order"
    src = Path(__file__).resolve().parent / "work_order.cpp"
    subprocess.run([hipcc, "--cuda-host-only", "-x", "hip", "-O2", "-std=c++17", str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.startswith("ok ")
