"""ctypes binding of ``include/fjx_tri.h`` (``foldjax_amd/lib/libfjx_tri.so``).

The library is loaded on first use. A missing library raises ``RuntimeError``
naming the build command -- there is no fallback path, mirroring the
reference's refusal to fall back when its fused kernel library is absent
(``src/foldjax/models/_cueq.py:46-63``).
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("FJX_LIB", Path(__file__).resolve().parent / "lib" / "libfjx_tri.so"))

FJX_DTYPE_F32 = 0
FJX_DTYPE_BF16 = 1
FJX_OUTGOING = 0
FJX_INCOMING = 1
FJX_OK = 0
FJX_ERR_INVALID = 1
FJX_ERR_UNSUPPORTED = 2
FJX_ERR_WORKSPACE = 3
FJX_ERR_HIP = 4

ABI_VERSION = 6
NOALLOC_SCRATCH_BYTES = 256 << 20

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t


class TriMulArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("n", _i64), ("c_z", _i64), ("c_h", _i64),
        ("direction", _i32), ("dtype", _i32), ("eps", _f32),
        ("x", _vp), ("mask", _vp),
        ("norm_in_weight", _vp), ("norm_in_bias", _vp),
        ("p_in_weight", _vp), ("g_in_weight", _vp),
        ("norm_out_weight", _vp), ("norm_out_bias", _vp),
        ("p_out_weight", _vp), ("g_out_weight", _vp),
        ("residual", _vp), ("out", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("out_mask", _vp),
    ]


class TriAttnArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("n", _i64), ("c_z", _i64), ("heads", _i64), ("head_dim", _i64),
        ("starting", _i32), ("dtype", _i32), ("eps", _f32), ("inf", _f32),
        ("x", _vp), ("mask", _vp),
        ("norm_weight", _vp), ("norm_bias", _vp), ("bias_weight", _vp),
        ("q_weight", _vp), ("k_weight", _vp), ("v_weight", _vp), ("g_weight", _vp), ("o_weight", _vp),
        ("residual", _vp), ("out", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("out_mask", _vp),
    ]


class TriAttnCoreArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("rows", _i64), ("heads", _i64), ("n", _i64), ("head_dim", _i64),
        ("dtype", _i32), ("scale", _f32),
        ("q", _vp), ("k", _vp), ("v", _vp), ("tri_bias", _vp), ("mask_bias", _vp),
        ("out", _vp), ("workspace", _vp), ("workspace_bytes", _sz),
    ]


class TransitionArgs(ctypes.Structure):
    _fields_ = [
        ("rows", _i64), ("c", _i64), ("dtype", _i32), ("eps", _f32),
        ("x", _vp), ("norm_weight", _vp), ("norm_bias", _vp),
        ("w_a", _vp), ("w_b", _vp), ("w_o", _vp),
        ("row_mask", _vp), ("residual", _vp), ("out", _vp),
        ("hidden", _i64), ("workspace", _vp), ("workspace_bytes", _sz),
        ("pb_n", _i64), ("pb_heads", _i64), ("pb_eps", _f32),
        ("pb_norm_weight", _vp), ("pb_norm_bias", _vp), ("pb_weight", _vp), ("pb_out", _vp),
        ("out_mask", _vp), ("pb_f32", _i32),
    ]


class SingleAttentionArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("n", _i64), ("c_s", _i64), ("c_z", _i64), ("heads", _i64),
        ("dtype", _i32), ("eps", _f32), ("inf", _f32),
        ("s", _vp), ("z", _vp), ("mask", _vp),
        ("pre_norm_weight", _vp), ("pre_norm_bias", _vp),
        ("z_norm_weight", _vp), ("z_norm_bias", _vp), ("z_weight", _vp),
        ("q_weight", _vp), ("q_bias", _vp), ("k_weight", _vp), ("v_weight", _vp),
        ("g_weight", _vp), ("o_weight", _vp),
        ("residual", _vp), ("out", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("pair_bias", _vp),
        ("z_dtype", _i32), ("out_mask", _vp),
        ("extra_bias", _vp), ("extra_bias_stride_b", _i64), ("extra_bias_stride_h", _i64),
    ]


# every symbol the header declares, with its ctypes signature
SYMBOLS = {
    "fjx_trimul_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i32]),
    "fjx_trimul_fwd": (ctypes.c_int, [ctypes.POINTER(TriMulArgs), _vp]),
    "fjx_trimul_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(TriMulArgs), _vp]),
    "fjx_triattn_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "fjx_triattn_fwd": (ctypes.c_int, [ctypes.POINTER(TriAttnArgs), _vp]),
    "fjx_triattn_core_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "fjx_triattn_core": (ctypes.c_int, [ctypes.POINTER(TriAttnCoreArgs), _vp]),
    "fjx_transition_workspace_size": (_sz, [_i64, _i64, _i64, _i32]),
    "fjx_transition_fwd": (ctypes.c_int, [ctypes.POINTER(TransitionArgs), _vp]),
    "fjx_pair_bias_size": (_sz, [_i64, _i64, _i64, _i32]),
    "fjx_single_attention_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i32]),
    "fjx_single_attention_fwd": (ctypes.c_int, [ctypes.POINTER(SingleAttentionArgs), _vp]),
    "fjx_last_error": (ctypes.c_char_p, []),
    "fjx_abi_version": (ctypes.c_int, []),
    "fjx_prof_enable": (ctypes.c_int, [ctypes.c_int]),
    "fjx_prof_reset": (ctypes.c_int, []),
    "fjx_prof_collect": (ctypes.c_int, []),
    "fjx_prof_num_kernels": (ctypes.c_int, []),
    "fjx_prof_kernel_name": (ctypes.c_char_p, [ctypes.c_int]),
    "fjx_prof_read": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64)]),
    "fjx_probe_issue_mix": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_float),
                                           _vp]),
    "fjx_probe_hbm_stream": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _i64, ctypes.POINTER(ctypes.c_float), _vp]),
}

_lock = threading.Lock()
_lib = None


class FjxError(RuntimeError):
    """A non-zero return code from the HIP library, with its message."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def load() -> ctypes.CDLL:
    """Load the library once; raise ``RuntimeError`` if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.is_file():
            raise RuntimeError(
                f"the gfx950 HIP library is not built ({LIB_PATH} is missing); run "
                "`python -m foldjax_amd.build` (needs hipcc) before using the 'hip' backend"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SYMBOLS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.fjx_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {lib.fjx_abi_version()}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def check(rc: int) -> None:
    if rc != FJX_OK:
        msg = load().fjx_last_error().decode()
        if rc in (FJX_ERR_INVALID, FJX_ERR_UNSUPPORTED):
            raise ValueError(msg)
        raise FjxError(rc, msg)


def prof_enable(on: bool = True) -> None:
    load().fjx_prof_enable(1 if on else 0)


def prof_reset() -> None:
    load().fjx_prof_reset()


def prof_read() -> dict[str, tuple[float, int]]:
    """Collect pending events and return ``{kernel: (total_ms, launches)}``."""
    lib = load()
    check(lib.fjx_prof_collect())
    out = {}
    for i in range(lib.fjx_prof_num_kernels()):
        ms = ctypes.c_double()
        cnt = _i64()
        check(lib.fjx_prof_read(i, ctypes.byref(ms), ctypes.byref(cnt)))
        out[lib.fjx_prof_kernel_name(i).decode()] = (ms.value, cnt.value)
    return out


def probe_issue_mix(mix: int, waves_per_simd: int, iters: int, stream: int = 0) -> float:
    """Kernel milliseconds of ``fjx_probe_issue_mix`` (the flash tile's
    instruction mix alone; see the header)."""
    ms = ctypes.c_float()
    check(load().fjx_probe_issue_mix(mix, waves_per_simd, iters, ctypes.byref(ms), stream))
    return ms.value


def probe_hbm_stream(mode: int, wgs_per_cu: int, nbytes: int, stream: int = 0) -> float:
    """Kernel milliseconds of ``fjx_probe_hbm_stream`` (a plain HBM streaming
    kernel; see the header)."""
    ms = ctypes.c_float()
    check(load().fjx_probe_hbm_stream(mode, wgs_per_cu, nbytes, ctypes.byref(ms), stream))
    return ms.value
