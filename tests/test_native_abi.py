"""CPU checks of the C ABI: the library loads, exports every declared symbol, and the
ctypes mirrors of the ABI structs have the C layout.  No GPU work is launched."""
import ctypes as C
import os
import re

import pytest

from polar_pack_amd import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "polar_pack.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\**\s+\**(pp_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("pp_quad_gemm", "pp_quad_dequant", "pp_quad_stream", "pp_dual_gemm", "pp_dual_dequant",
                 "pp_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = nat.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding table covers them all
    assert set(declared_functions()) <= set(nat.EXPORTS)


def test_struct_layouts_match():
    out = (C.c_int64 * 4)()
    assert nat.lib().pp_abi_sizes(out, 4) == 4
    assert out[0] == C.sizeof(nat.QuadProj)
    assert out[1] == C.sizeof(nat.QuadItem)
    assert out[2] == C.sizeof(nat.QuadSeg)
    assert out[3] == C.sizeof(nat.DualProj)


def test_version_and_error_string():
    lib = nat.lib()
    assert b"gfx950" in lib.pp_version()
    assert isinstance(lib.pp_last_error(), bytes)


def test_invalid_arguments_are_rejected_without_a_gpu():
    lib = nat.lib()
    # null LUT array -> PP_EINVAL before any device call
    rc = lib.pp_quad_gemm(None, 0, 0, None, 0, 0, None, 0, None, None, None, 0, 0, None, 0, 0, 1, 1, 1,
                          None, 0, None)
    assert rc == nat.PP_EINVAL
    assert b"luts" in lib.pp_last_error()
    rc = lib.pp_dual_gemm(None, 0, 0, None, 7, 0, 0, None, 32, 0, None, 64, None, None, 1024, 0, None, None, 0, 0,
                          None, None, 0, 0, 1, 1, 1, None, 0, None)
    assert rc == nat.PP_EINVAL
    assert b"code_layout" in lib.pp_last_error()
    with pytest.raises(RuntimeError):
        nat.check(rc, "pp_dual_gemm")


def test_stream_rows_query():
    assert nat.lib().pp_quad_stream_rows(1) >= 1
    assert nat.lib().pp_quad_stream_rows(9) == 0
    assert b"1..8" in nat.lib().pp_last_error()
