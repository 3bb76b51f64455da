"""The C-ABI library loads and exports every entry point include/vybdq.h declares; host-side
precondition checks return their error codes before any launch. CPU only: no call here
reaches the GPU."""

import os
import re

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "vybdq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vybdq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "vybdq_gemv_q4_0" in names and "vybdq_last_error" in names
    assert len(names) >= 8


def test_library_exports_every_declared_symbol():
    from vybforge_amd import _lib
    for name in declared_functions():
        assert hasattr(_lib.lib, name), f"{name} not exported"
    # and the ctypes table covers exactly the header
    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_abi_version():
    from vybforge_amd import _lib
    assert _lib.lib.vybdq_abi_version() == 1


@pytest.mark.parametrize("args,code,text", [
    # (W, X, Y, M, N, K, x_dt, y_dt, RS, order, stream)
    ((1, 16, 1, 1, 16, 48, 0, 0, 0, 0, 0), -2, "K must be"),        # K % 32 != 0
    ((1, 16, 1, 9, 16, 64, 0, 0, 0, 0, 0), -2, "M must be"),        # M > 8
    ((0, 16, 1, 1, 16, 64, 0, 0, 0, 0, 0), -1, "null W"),
    ((1, 16, 1, 1, 16, 64, 7, 0, 0, 0, 0), -1, "x_dt"),
    ((1, 16, 1, 1, 16, 64, 0, 0, 0, 5, 0), -1, "order"),
    ((2, 16, 1, 1, 16, 64, 0, 0, 0, 0, 0), -3, "W must be"),        # W not 4-byte aligned
    ((4, 8, 1, 1, 16, 64, 0, 0, 0, 0, 0), -3, "X must be"),         # X not 16-byte aligned
    ((4, 16, 1, 1, 0, 64, 0, 0, 0, 0, 0), -2, "N must be"),
])
def test_gemv_preconditions(args, code, text):
    from vybforge_amd import _lib
    rc = _lib.lib.vybdq_gemv_q4_0(*args)
    assert rc == code
    assert text in _lib.last_error()


@pytest.mark.parametrize("args,code,text", [
    # (wtype, W, Xq, Xs, Y, N, K, y_dt, RS, stream)
    ((14, 4, 16, 4, 4, 16, 256, 0, 0, 0), -1, "wtype must be"),     # Q6_K has no xq8 GEMV
    ((12, 4, 16, 4, 4, 16, 320, 0, 0, 0), -2, "K must be"),         # K % 256 != 0
    ((12, 4, 16, 4, 4, 16, 65792, 0, 0, 0), -2, "at most 65536"),
    ((22, 4, 8, 4, 4, 16, 256, 0, 0, 0), -3, "Xq must be"),         # Xq not 16-byte aligned
    ((22, 4, 16, 2, 4, 16, 256, 0, 0, 0), -3, "Xs must be"),        # Xs not 4-byte aligned
    ((13, 2, 16, 4, 4, 16, 256, 0, 0, 0), -3, "W must be"),         # W not 4-byte aligned
    ((13, 0, 16, 4, 4, 16, 256, 0, 0, 0), -1, "null W"),
    ((13, 4, 16, 4, 4, 0, 256, 0, 0, 0), -2, "N must be"),
    ((13, 4, 16, 4, 4, 16, 256, 9, 0, 0), -1, "y_dt"),
])
def test_gemv_xq8_preconditions(args, code, text):
    from vybforge_amd import _lib
    rc = _lib.lib.vybdq_gemv_xq8(*args)
    assert rc == code
    assert text in _lib.last_error()


def test_dequant_preconditions():
    from vybforge_amd import _lib
    assert _lib.lib.vybdq_dequant_q4_0(0, 1, 1, 0, 0, 0) == _lib.ERR_ARG
    assert _lib.lib.vybdq_dequant_q4_0(1, 1, 1, 0, 2, 0) == _lib.ERR_ARG   # BF16 out not offered
    assert _lib.lib.vybdq_dequant_q8_0(1, 1, -1, 0, 0) == _lib.ERR_SHAPE
    assert _lib.lib.vybdq_dequant_q8_0(1, 1, 0, 0, 0) == _lib.OK          # empty: no launch


def test_quant_preconditions():
    from vybforge_amd import _lib
    assert _lib.lib.vybdq_quant_q8_act(1, 1, 1, 2, 33, 0, 0) == _lib.ERR_SHAPE
    assert _lib.lib.vybdq_quant_q8_act(1, 1, 2, 2, 32, 0, 0) == _lib.ERR_ALIGN


def test_moe_noalloc_size_limit_on_host():
    """The allocation-free MoE entry rejects a shape whose workspace exceeds its scratch before it
    touches the device (GLM-5 shapes at 4096 tokens)."""
    from vybforge_amd import _lib
    assert _lib.lib.vybdq_moe_workspace_size(4096, 6144, 2048, 256, 8) > _lib.MOE_NOALLOC_MAX_BYTES
    assert _lib.lib.vybdq_moe_workspace_size(233, 6144, 2048, 256, 8) <= _lib.MOE_NOALLOC_MAX_BYTES
    assert _lib.lib.vybdq_moe_workspace_size(234, 6144, 2048, 256, 8) > _lib.MOE_NOALLOC_MAX_BYTES
    rc = _lib.lib.vybdq_moe_forward_noalloc(2, 16, 2, 16, 0, 0, 16, 16, 16, 0, 0, 0, 16, 0, 0, 0, 4096, 6144, 2048,
                                            256, 8, 2.5, 10.0, 0)
    assert rc == _lib.ERR_WORKSPACE
    assert "scratch" in _lib.last_error()


def test_pblock_preconditions_on_host():
    """vybdq_launch_pblock / _grid reject a null or misaligned block, an unknown kind and an EXL3DQ
    block without its grid before they touch the device."""
    from vybforge_amd import _lib
    L = _lib.lib
    assert L.vybdq_launch_pblock(_lib.PB_MOE, 0, 0) == _lib.ERR_ARG
    assert L.vybdq_launch_pblock(_lib.PB_MOE, 4100, 0) == _lib.ERR_ALIGN
    assert L.vybdq_launch_pblock(_lib.PB_GEMV + 3, 4096, 0) == _lib.ERR_ARG
    assert L.vybdq_launch_pblock(0xB00, 4096, 0) == _lib.ERR_ARG
    assert L.vybdq_launch_pblock(0x702, 4096, 0) == _lib.ERR_ARG
    assert L.vybdq_launch_pblock(_lib.PB_EXL3DQ, 4096, 0) == _lib.ERR_ARG
    assert "grid" in _lib.last_error()
    assert L.vybdq_launch_pblock_grid(_lib.PB_EXL3DQ, 4096, 0, 256, 0) == _lib.ERR_SHAPE
    assert L.vybdq_launch_pblock_grid(_lib.PB_EXL3DQ, 0, 1, 256, 0) == _lib.ERR_ARG
    for kind in (_lib.PB_EXL3HGEN, _lib.PB_EXL3HAD132, _lib.PB_EXL3HAD232, _lib.PB_EXL3CVT32):
        assert L.vybdq_launch_pblock(kind, 0, 0) == _lib.ERR_ARG
        assert L.vybdq_launch_pblock(kind, 4100, 0) == _lib.ERR_ALIGN


def test_exl3_deq_map_preconditions_on_host():
    """The map-driven decode (exl3deq / exl3deq32) rejects null pointers, an output type other than
    float32 / float64 and a misaligned map or output before it touches the device."""
    from vybforge_amd import _lib
    L = _lib.lib
    assert L.vybdq_exl3_deq_map(0, 4096, 4096, _lib.F32, 0) == _lib.ERR_ARG
    assert L.vybdq_exl3_deq_map(4096, 4096, 0, _lib.F64, 0) == _lib.ERR_ARG
    assert L.vybdq_exl3_deq_map(4096, 4096, 4096, _lib.F16, 0) == _lib.ERR_ARG
    assert L.vybdq_exl3_deq_map(4096, 4100, 4096, _lib.F32, 0) == _lib.ERR_ALIGN
    assert L.vybdq_exl3_deq_map(4096, 4096, 4100, _lib.F64, 0) == _lib.ERR_ALIGN
    assert L.vybdq_exl3_deq_map(4096, 4096, 4098, _lib.F32, 0) == _lib.ERR_ALIGN


@pytest.mark.parametrize("cb", [0, 2, -1])
def test_exl3_rejects_codebooks_other_than_mcg(cb):
    """Only the mcg codebook (1) exists in the reference; every EXL3 entry point refuses any other
    id on the host, before it touches the device."""
    from vybforge_amd import _lib
    L = _lib.lib
    assert L.vybdq_exl3_decode_tiles(4096, 4096, 128, 128, cb, 0, 0) == _lib.ERR_ARG
    assert "codebook" in _lib.last_error()
    assert L.vybdq_dequant_exl3(4096, 4096, 4096, 4096, 128, 128, cb, 0, 0) == _lib.ERR_ARG
    assert L.vybdq_exl3_gemm(4096, 4096, 4096, 4096, 4096, 1, 128, 128, cb, 1, 0, 4096, 1 << 20, 0) == _lib.ERR_ARG
    assert "codebook" in _lib.last_error()
