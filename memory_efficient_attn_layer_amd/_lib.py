"""ctypes binding of libmea.so (the C ABI declared in include/mea.h).

The library is loaded only after ``import torch`` so that its HIP runtime
dependency (soname libamdhip64.so.7) resolves to the runtime torch already
mapped; device pointers and streams handed over by torch are then valid in
the library. There is no fallback: if the library is missing the block
cannot run and every entry point raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see above)

LIB_PATH = Path(__file__).resolve().with_name("libmea.so")

MEA_PASS_FWD = 0
MEA_PASS_BWD = 1
MEA_PASS_BWD_TABLES = 2  # backward that also writes the table gradients
MEA_STATIC_SCRATCH_BYTES = 16 << 20  # include/mea.h


class MeaDesc(ctypes.Structure):
    """Mirror of ``struct mea_desc``."""

    _fields_ = [
        ("B", ctypes.c_int64),
        ("T", ctypes.c_int64),
        ("C", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("T_max", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("N_active", ctypes.c_int64),
        ("tables_bf16", ctypes.c_int64),
    ]


_vp = ctypes.c_void_p
_fp = ctypes.c_void_p  # float* passed as an address
_desc = ctypes.POINTER(MeaDesc)

# name -> (restype, argtypes); exactly the symbols include/mea.h declares.
EXPORTS = {
    "mea_workspace_bytes": (ctypes.c_size_t, [_desc, ctypes.c_int]),
    "mea_fwd": (ctypes.c_int, [_desc] + [_vp] * 6 + [_fp, _fp, _vp, _vp, _fp, _vp, ctypes.c_size_t, _vp]),
    "mea_bwd": (
        ctypes.c_int,
        [_desc] + [_vp] * 7 + [_fp, _fp, _vp, _fp] + [_vp] * 6 + [_fp, _fp, _vp, ctypes.c_size_t, _vp],
    ),
    "mea_fwd_varlen": (
        ctypes.c_int,
        [_desc, _vp, ctypes.c_int32, ctypes.c_int32] + [_vp] * 6 + [_fp, _fp, _vp, _vp, _fp, _vp, ctypes.c_size_t, _vp],
    ),
    "mea_bwd_varlen": (
        ctypes.c_int,
        [_desc, _vp, ctypes.c_int32, ctypes.c_int32] + [_vp] * 7 + [_fp, _fp, _vp, _fp] + [_vp] * 6
        + [_fp, _fp, _vp, ctypes.c_size_t, _vp],
    ),
    "mea_prefill": (ctypes.c_int, [_desc] + [_vp] * 6 + [_fp, _fp, _vp, _vp, _vp, ctypes.c_int64, _vp, ctypes.c_size_t, _vp]),
    "mea_decode_workspace_bytes": (ctypes.c_size_t, [_desc]),
    "mea_decode": (ctypes.c_int, [_desc] + [_vp] * 6 + [_fp, _fp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "mea_decode_static": (ctypes.c_int, [_desc] + [_vp] * 6 + [_fp, _fp, _vp, _vp, _vp, _vp, _vp]),
    "mea_qkvg_proj": (ctypes.c_int, [_desc] + [_vp] * 5 + [_fp, _fp] + [_vp] * 4 + [_fp, _fp, _fp, _vp]),
    "mea_attn_fwd": (ctypes.c_int, [_desc, _vp, _vp, _vp, _vp, _fp, _vp]),
    "mea_gate_oproj": (ctypes.c_int, [_desc, _vp, _vp, _vp, _vp, _vp]),
    "mea_bwd_stage_grads": (
        ctypes.c_int,
        [_desc] + [_vp] * 7 + [_fp, _fp, _vp, _fp] + [_vp] * 5 + [_fp, _fp, _fp, _vp, ctypes.c_size_t, _vp],
    ),
    "mea_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "mea_version": (ctypes.c_char_p, []),
    "mea_profile_enable": (ctypes.c_int, [ctypes.c_int]),
    "mea_profile_read": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_double)]),
    "mea_profile_kernel_name": (ctypes.c_char_p, [ctypes.c_int]),
    "mea_profile_select": (ctypes.c_int, [ctypes.c_int]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def _check_single_hip_runtime() -> None:
    """Refuses to run if two different HIP runtimes ended up mapped."""
    try:
        maps = Path("/proc/self/maps").read_text()
    except OSError:
        return
    paths = {ln.split()[-1] for ln in maps.splitlines() if "libamdhip64.so" in ln and "/" in ln}
    real = {str(Path(p).resolve()) for p in paths}
    if len(real) > 1:
        raise RuntimeError(f"two HIP runtimes are mapped in this process: {sorted(real)}")


def load() -> ctypes.CDLL:
    """Loads (once) and returns the library; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m memory_efficient_attn_layer_amd.build` "
                "(the block has no CPU or eager fallback)"
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _check_single_hip_runtime()
        _lib = lib
        return lib


def strerror(code: int) -> str:
    return load().mea_strerror(int(code)).decode()


def check(code: int, what: str) -> None:
    if code != 0:
        raise RuntimeError(f"{what} failed: {strerror(code)} (status {code})")


def desc(B: int, T: int, C: int, H: int, N: int, T_max: int, eps: float, N_active: int = 0,
         tables_bf16: bool = False) -> MeaDesc:
    """A descriptor; N_active > 0: heads of N_active dimensions carried zero-padded to N;
    tables_bf16: the fp32 tables passed hold bf16 values (the caller's tables were bf16)."""
    return MeaDesc(int(B), int(T), int(C), int(H), int(N), int(T_max), float(eps), int(N_active),
                   int(bool(tables_bf16)))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def profile_enable(on: bool) -> None:
    check(load().mea_profile_enable(1 if on else 0), "mea_profile_enable")


def profile_select(name: str | None) -> None:
    """Limits the recording to the named kernel (None: every kernel)."""
    lib = load()
    k = -1
    if name is not None:
        k = 0
        while True:
            n = lib.mea_profile_kernel_name(k)
            if n is None:
                raise ValueError(f"no kernel named {name!r}")
            if n.decode() == name:
                break
            k += 1
    check(lib.mea_profile_select(k), "mea_profile_select")


def profile_read() -> dict:
    """{kernel name: (launch count, total ms)} of the launches recorded while
    profiling was enabled (waits for their completion events)."""
    lib = load()
    out = {}
    k = 0
    while True:
        name = lib.mea_profile_kernel_name(k)
        if name is None:
            break
        cnt, ms = ctypes.c_int(0), ctypes.c_double(0.0)
        check(lib.mea_profile_read(k, ctypes.byref(cnt), ctypes.byref(ms)), "mea_profile_read")
        if cnt.value:
            out[name.decode()] = (cnt.value, ms.value)
        k += 1
    return out
