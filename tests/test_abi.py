"""CPU checks of the C ABI: the library loads, exports every declared symbol,
its struct layouts match the ctypes mirrors, and argument errors come back as
codes and messages -- all without launching a kernel."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import tempfile
from pathlib import Path

import pytest

from foldjax_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "fjx_tri.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fjx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.is_file():
        pytest.fail(f"{_lib.LIB_PATH} is not built; run `python -m foldjax_amd.build`")
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    declared = _declared_functions()
    assert declared, "no declarations parsed from the header"
    assert set(declared) == set(_lib.SYMBOLS), "ctypes bindings and header disagree"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (fjx_[a-z0-9_]+)$", nm.stdout, flags=re.M))
    missing = set(declared) - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    for name in declared:
        assert hasattr(lib, name)


def test_abi_version(lib):
    assert lib.fjx_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_c(tmp_path):
    """Compile a C probe against the header and compare sizeof/offsetof with
    the ctypes mirrors, field by field."""
    structs = {
        "fjx_trimul_args": _lib.TriMulArgs,
        "fjx_triattn_args": _lib.TriAttnArgs,
        "fjx_triattn_core_args": _lib.TriAttnCoreArgs,
        "fjx_transition_args": _lib.TransitionArgs,
        "fjx_single_attention_args": _lib.SingleAttentionArgs,
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "fjx_tri.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", "-I/opt/rocm/include",
                    str(src), "-o", str(exe)], check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, out):
        cname, field, value = line.split()
        cls = structs[cname]
        got = ctypes.sizeof(cls) if field == "size" else getattr(cls, field).offset
        assert got == int(value), f"{cname}.{field}: ctypes {got} != C {value}"


def test_workspace_sizes_are_host_only(lib):
    assert lib.fjx_trimul_workspace_size(1, 1024, 128, 128, _lib.FJX_DTYPE_BF16) >= 3 * 1024 * 1024 * 128 * 2
    assert lib.fjx_trimul_workspace_size(0, 8, 128, 128, 0) == 0
    assert lib.fjx_triattn_workspace_size(1, 384, 128, 4, 32, _lib.FJX_DTYPE_BF16) > 0
    assert lib.fjx_triattn_core_workspace_size(1, 3, 4, 70, 32, _lib.FJX_DTYPE_F32) > 0
    # the narrow fused forms (c_z 32, 64, 96 with c_h = 128: the template
    # stack's 64) take the c = 128 workspace; the general-width paths (c_z
    # not a multiple of 32, c_h != 128) their own, larger one
    fused = lib.fjx_trimul_workspace_size(1, 64, 128, 128, _lib.FJX_DTYPE_BF16)
    assert lib.fjx_trimul_workspace_size(1, 64, 64, 128, _lib.FJX_DTYPE_BF16) == fused
    assert lib.fjx_trimul_workspace_size(1, 64, 48, 128, _lib.FJX_DTYPE_BF16) > fused
    assert lib.fjx_trimul_workspace_size(1, 64, 64, 64, _lib.FJX_DTYPE_BF16) > 0
    fused_a = lib.fjx_triattn_workspace_size(1, 64, 128, 4, 32, _lib.FJX_DTYPE_BF16)
    assert lib.fjx_triattn_workspace_size(1, 64, 64, 4, 32, _lib.FJX_DTYPE_BF16) == fused_a
    assert lib.fjx_triattn_workspace_size(1, 64, 64, 2, 32, _lib.FJX_DTYPE_BF16) > 0
    assert lib.fjx_transition_workspace_size(100, 128, 0, _lib.FJX_DTYPE_BF16) == 0  # fused: none
    assert lib.fjx_transition_workspace_size(100, 64, 0, _lib.FJX_DTYPE_BF16) == 0  # narrow fused: none
    assert lib.fjx_transition_workspace_size(100, 384, 1536, _lib.FJX_DTYPE_BF16) > 0  # single track: general path
    assert lib.fjx_transition_workspace_size(100, 48, 0, _lib.FJX_DTYPE_BF16) >= 100 * (48 + 192 + 48) * 2
    # the prepared pair bias: [batch, heads, Np, Np], Np = n rounded up to 64
    assert lib.fjx_pair_bias_size(2, 1000, 16, _lib.FJX_DTYPE_BF16) == 2 * 16 * 1024 * 1024 * 2
    assert lib.fjx_pair_bias_size(1, 64, 4, _lib.FJX_DTYPE_F32) == 4 * 64 * 64 * 4
    assert lib.fjx_pair_bias_size(1, 0, 4, _lib.FJX_DTYPE_F32) == 0


def test_invalid_arguments_return_codes_without_launching(lib):
    a = _lib.TriMulArgs(batch=1, n=8, c_z=128, c_h=128, direction=7, dtype=0, eps=1e-5)
    rc = lib.fjx_trimul_fwd(ctypes.byref(a), None)
    assert rc == _lib.FJX_ERR_INVALID
    assert "Unsupported triangle multiplication direction" in lib.fjx_last_error().decode()

    a = _lib.TriMulArgs(batch=1, n=8, c_z=60, c_h=128, direction=0, dtype=0, eps=1e-5)
    assert lib.fjx_trimul_fwd(ctypes.byref(a), None) == _lib.FJX_ERR_UNSUPPORTED
    assert "multiples of 8" in lib.fjx_last_error().decode()

    a = _lib.TriMulArgs(batch=1, n=8, c_z=128, c_h=128, direction=0, dtype=0, eps=1e-5)
    assert lib.fjx_trimul_fwd(ctypes.byref(a), None) == _lib.FJX_ERR_INVALID  # null pointers

    fake = 0x1000  # never dereferenced: the workspace check fails first
    a = _lib.TriMulArgs(batch=1, n=8, c_z=128, c_h=128, direction=0, dtype=1, eps=1e-5,
                        x=fake, norm_in_weight=fake, norm_in_bias=fake, p_in_weight=fake, g_in_weight=fake,
                        norm_out_weight=fake, norm_out_bias=fake, p_out_weight=fake, g_out_weight=fake,
                        out=fake, workspace=fake, workspace_bytes=16)
    assert lib.fjx_trimul_fwd(ctypes.byref(a), None) == _lib.FJX_ERR_WORKSPACE
    assert "workspace" in lib.fjx_last_error().decode()

    a = _lib.TriMulArgs(batch=1, n=8, c_z=128, c_h=128, direction=0, dtype=1, eps=1e-5,
                        x=fake + 8, norm_in_weight=fake, norm_in_bias=fake, p_in_weight=fake, g_in_weight=fake,
                        norm_out_weight=fake, norm_out_bias=fake, p_out_weight=fake, g_out_weight=fake,
                        out=fake, workspace=fake, workspace_bytes=16)
    assert lib.fjx_trimul_fwd(ctypes.byref(a), None) == _lib.FJX_ERR_INVALID  # misaligned x
    assert "16-byte aligned" in lib.fjx_last_error().decode()

    t = _lib.TriAttnArgs(batch=1, n=8, c_z=128, heads=8, head_dim=16, starting=1, dtype=0)
    assert lib.fjx_triattn_fwd(ctypes.byref(t), None) == _lib.FJX_ERR_UNSUPPORTED
    c = _lib.TriAttnCoreArgs(batch=1, rows=1, heads=1, n=4, head_dim=64, dtype=0)
    assert lib.fjx_triattn_core(ctypes.byref(c), None) == _lib.FJX_ERR_UNSUPPORTED
    assert lib.fjx_trimul_fwd(None, None) == _lib.FJX_ERR_INVALID
    tr = _lib.TransitionArgs(rows=4, c=100, dtype=1)
    assert lib.fjx_transition_fwd(ctypes.byref(tr), None) == _lib.FJX_ERR_UNSUPPORTED
    tr = _lib.TransitionArgs(rows=4, c=64, dtype=1, hidden=-1)
    assert lib.fjx_transition_fwd(ctypes.byref(tr), None) == _lib.FJX_ERR_INVALID
    sa = _lib.SingleAttentionArgs(batch=1, n=4, c_s=384, c_z=128, heads=8, dtype=1)  # head_dim 48 > 32
    assert lib.fjx_single_attention_fwd(ctypes.byref(sa), None) == _lib.FJX_ERR_UNSUPPORTED


def test_pair_bias_arguments_are_checked_before_launch(lib):
    """The transition's pair-bias output and the single attention's prepared
    pair bias are validated on the host (fake, never dereferenced pointers)."""
    fake = 0x1000
    base = dict(dtype=1, eps=1e-5, x=fake, norm_weight=fake, norm_bias=fake, w_a=fake, w_b=fake, w_o=fake,
                out=fake, pb_out=fake, pb_norm_weight=fake, pb_norm_bias=fake, pb_weight=fake)
    tr = _lib.TransitionArgs(rows=18, c=64, pb_n=3, pb_heads=16, workspace=fake, workspace_bytes=1 << 40, **base)
    assert lib.fjx_transition_fwd(ctypes.byref(tr), None) == _lib.FJX_ERR_UNSUPPORTED
    assert "c == 128" in lib.fjx_last_error().decode()
    tr = _lib.TransitionArgs(rows=10, c=128, pb_n=3, pb_heads=16, **base)  # 10 is not a multiple of 3^2
    assert lib.fjx_transition_fwd(ctypes.byref(tr), None) == _lib.FJX_ERR_INVALID
    assert "multiple of pb_n^2" in lib.fjx_last_error().decode()
    tr = _lib.TransitionArgs(rows=18, c=128, pb_n=3, pb_heads=0, **base)
    assert lib.fjx_transition_fwd(ctypes.byref(tr), None) == _lib.FJX_ERR_INVALID
    tr = _lib.TransitionArgs(rows=18, c=128, pb_n=3, pb_heads=16, **dict(base, pb_weight=None))
    assert lib.fjx_transition_fwd(ctypes.byref(tr), None) == _lib.FJX_ERR_INVALID
    assert "pair-bias weight" in lib.fjx_last_error().decode()
    tr = _lib.TransitionArgs(rows=18, c=128, pb_n=3, pb_heads=16, **dict(base, pb_out=fake + 4))
    assert lib.fjx_transition_fwd(ctypes.byref(tr), None) == _lib.FJX_ERR_INVALID
    assert "16-byte aligned" in lib.fjx_last_error().decode()

    # with a prepared pair bias, z and its weights are not required: the call
    # gets as far as the workspace check
    sa = _lib.SingleAttentionArgs(batch=1, n=4, c_s=384, c_z=0, heads=16, dtype=1, s=fake, out=fake,
                                  q_weight=fake, k_weight=fake, v_weight=fake, g_weight=fake, o_weight=fake,
                                  pair_bias=fake, workspace=fake, workspace_bytes=16)
    assert lib.fjx_single_attention_fwd(ctypes.byref(sa), None) == _lib.FJX_ERR_WORKSPACE
    sa.pair_bias = None  # then z is required again
    assert lib.fjx_single_attention_fwd(ctypes.byref(sa), None) == _lib.FJX_ERR_UNSUPPORTED  # c_z == 0


def test_check_maps_codes_to_exceptions(lib):
    a = _lib.TriMulArgs(batch=1, n=8, c_z=128, c_h=128, direction=9, dtype=0)
    with pytest.raises(ValueError, match="direction"):
        _lib.check(lib.fjx_trimul_fwd(ctypes.byref(a), None))


def test_profiling_counters_start_empty(lib):
    _lib.prof_reset()
    stats = _lib.prof_read()
    assert "triattn_flash" in stats and "trimul_contract" in stats
    assert all(v == (0.0, 0) for v in stats.values())


def test_missing_library_raises_runtime_error(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="foldjax_amd.build"):
        _lib.load()
