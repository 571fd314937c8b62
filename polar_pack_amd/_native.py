"""ctypes binding of ``lib/libpolar_pack.so`` (declarations in include/polar_pack.h).

The product path has no fallback: if the library is missing or cannot load,
:func:`lib` raises, and every operator fails loudly.
"""
from __future__ import annotations

import collections
import ctypes as C
import os
import threading

from .build import LIB

PP_OK, PP_EINVAL, PP_EHIP, PP_ENOSUPPORT = 0, 1, 2, 3
PP_F16, PP_F32 = 0, 1
PP_DUAL_I16_OFFSET, PP_DUAL_U16_BE = 0, 1
PP_QUAD_NK, PP_QUAD_KN = 0, 1
PP_GEMM_ROWS, PP_GEMM_KN, PP_GEMM_GENERIC = 1, 2, 3
PP_ITEM_TAIL = 1
PP_ITEM_FP16 = 2

vp = C.c_void_p
i64 = C.c_int64
i32 = C.c_int


class QuadProj(C.Structure):
    """``pp_quad_proj`` (include/polar_pack.h)."""
    _fields_ = [("codes", vp), ("ldc", i64), ("pos0", i64), ("x", vp), ("x_sm", i64),
                ("out", vp * 4), ("o_sm", i64), ("N", C.c_int32), ("K", C.c_int32)]


class QuadItem(C.Structure):
    """``pp_quad_item`` (include/polar_pack.h)."""
    _fields_ = [("proj", C.c_int32), ("row0", C.c_int32), ("nrows", C.c_int32), ("flags", C.c_int32),
                ("plug_lo", i64), ("plug_hi", i64)]


class QuadSeg(C.Structure):
    """``pp_quad_seg`` (include/polar_pack.h)."""
    _fields_ = [("proj", C.c_int32), ("row0", C.c_int32), ("row1", C.c_int32), ("task0", C.c_int32),
                ("plug_lo", i64), ("k0", C.c_int32), ("k1", C.c_int32), ("parts", C.c_int32),
                ("reserved", C.c_int32), ("acc_off", i64)]


class DualProj(C.Structure):
    """``pp_dual_proj`` (include/polar_pack.h)."""
    _fields_ = [("codes", vp), ("ldc", i64), ("pos0", i64), ("x", vp), ("x_sm", i64),
                ("out", vp * 2), ("o_sm", i64), ("N", C.c_int32), ("K", C.c_int32)]


EXPORTS = {
    "pp_last_error": (C.c_char_p, []),
    "pp_version": (C.c_char_p, []),
    "pp_abi_sizes": (i32, [C.POINTER(i64), i32]),
    "pp_quad_gemm": (i32, [vp, i64, i64, vp, i64, i64, vp, i32, vp, vp, vp, i64, i64, vp, i64, i64,
                           i64, i64, i64, vp, i64, vp]),
    "pp_quad_gemm_workspace_size": (i64, [vp, i64, i64, vp, i64, i64, i64, i64, i64, i64]),
    "pp_quad_gemm_kernel": (i32, [vp, i64, i64, vp, i64, i64, i64, i64, i64]),
    "pp_quad_rows_plan_size": (i64, [i64]),
    "pp_quad_rows_workspace_size": (i64, [i64, i64, i64]),
    "pp_quad_rows_parts": (i32, [i64, i64, i64]),
    "pp_quad_rows_plan": (i32, [vp, i64, i64, i64, i64, i64, i64, vp, vp]),
    "pp_quad_rows": (i32, [vp, i64, vp, i64, vp, i32, vp, vp, vp, vp, i64, vp, i64, vp, i64, i64, i64, i64, i64,
                           vp, i64, vp]),
    "pp_dual_gemm_kernel": (i32, [vp, i64, i64, vp, i64, i64, i64, i64, i64, i64, i64, i64]),
    "pp_quad_gemm_noalloc": (i32, [vp, i64, i64, vp, i64, i64, vp, i32, vp, vp, vp, i64, i64, vp, i64, i64,
                                   i64, i64, i64, vp]),
    "pp_quad_dequant": (i32, [vp, i64, i64, vp, i32, vp, vp, vp, i64, i64, vp, i64, i64, vp]),
    "pp_quad_dequant_f16": (i32, [vp, i64, i64, vp, i32, vp, vp, vp, i64, i64, vp, i64, i64, vp]),
    "pp_quad_dequant_f16_t": (i32, [vp, i64, vp, i32, vp, vp, vp, i64, i64, vp, i64, i64, vp]),
    "pp_quad_mfma": (i32, [vp, i64, i64, vp, i64, vp, i32, vp, vp, vp, i64, vp, i64, i64, vp, i64, i64, i64, i64,
                           vp, i64, vp]),
    "pp_quad_mfma_workspace_size": (i64, [i64, i64, i64]),
    "pp_quad_mfma_waves": (i64, [i64]),
    "pp_quad_big": (i32, [vp, i32, i64, vp, i64, vp, i32, vp, vp, vp, i64, vp, i64, i64, i64, i64, vp, i64, i64, i64,
                          i64, vp, i64, vp]),
    "pp_quad_big_plan": (i32, [i64, i64, i64, i32, vp, vp]),
    "pp_quad_big_workspace_size": (i64, [i64, i64, i64]),
    "pp_dual_mfma": (i32, [vp, i64, vp, i64, vp, i64, vp, i32, vp, vp, i32, i32, vp, vp, i64, vp, i64, i64, i64,
                           i64, vp, vp, i64, i64, i64, i64, vp, i64, vp]),
    "pp_dual_mfma_plan": (i32, [i64, i64, i64, vp, vp]),
    "pp_dual_nk_mfma": (i32, [vp, i32, i64, i64, vp, i64, vp, i64, i64, i64, vp, i32, vp, vp, i32, i32, vp, vp, i64,
                              vp, i64, i64, vp, vp, i64, i64, i64, i64, vp, i64, vp]),
    "pp_dual_mfma_workspace_size": (i64, [i64, i64, i64]),
    "pp_quad_stream_rows": (i32, [i64]),
    "pp_quad_stream_chunk": (i32, [i64]),
    "pp_quad_stream_waves": (i64, [i64]),
    "pp_quad_stream": (i32, [vp, i64, vp, i64, vp, i64, vp, vp, i64, vp, vp, vp, vp, vp, i64, i64, vp, vp, i64, vp]),
    "pp_quad_plug_codes": (i32, [vp, i64, vp, i64, vp, vp]),
    "pp_plug_search": (i32, [vp, i64, i64, i64, i64, i64, i64, vp, vp]),
    "pp_quad_codes_nk": (i32, [vp, i64, i64, i64, vp, vp]),
    "pp_dual_stream_rows": (i32, [i64]),
    "pp_dual_stream_chunk": (i32, [i64]),
    "pp_dual_stream_waves": (i64, [i64]),
    "pp_dual_stream": (i32, [vp, i64, vp, i64, vp, i64, vp, vp, i64, i32, vp, i64, i32, vp, i64, i64, i64, vp, i64,
                             vp, vp, vp, vp, vp, vp, i64, i64, vp, vp, i64, vp]),
    "pp_dual_scale_table": (i32, [vp, i64, i64, vp, vp, vp, i64, i64, vp, i64, vp]),
    "pp_dual_rows_workspace_size": (i64, [i64, i64, i64]),
    "pp_dual_rows_parts": (i32, [i64, i64, i64]),
    "pp_dual_rows": (i32, [vp, vp, i64, i32, i32, vp, i64, i64, i64, vp, i64, vp, vp, vp, vp, vp, vp, i64, i64, vp,
                           i64, vp]),
    "pp_dual_task_entries": (i32, [vp, i64, vp, i64, i64, vp, vp]),
    "pp_dual_plug_table": (i32, [vp, i64, i32, vp, i64, i64, i64, vp, vp, vp, i64, vp, vp, i64, i64, vp, vp]),
    "pp_dual_gemm": (i32, [vp, i64, i64, vp, i32, i64, i64, vp, i64, i64, vp, i32, vp, vp, i32, i32,
                           vp, vp, i64, i64, vp, vp, i64, i64, i64, i64, i64, vp, i64, vp]),
    "pp_dual_gemm_workspace_size": (i64, [vp, i64, i64, vp, i64, i64, i64, i64, i64, i64, i64, i64, i64]),
    "pp_dual_dequant": (i32, [vp, i32, i64, i64, vp, i64, i64, vp, i32, vp, vp, i32, i32, vp, vp, i64, i64,
                              vp, vp, i64, i64, vp]),
    "pp_dual_dequant_f16": (i32, [vp, i32, i64, i64, vp, i64, i64, vp, i32, vp, vp, i32, i32, vp, vp, i64, i64,
                                  vp, vp, i64, i64, vp]),
    "pp_dual_dequant_f16_t": (i32, [vp, i32, i64, vp, i64, vp, i32, vp, vp, i32, i32, vp, vp, i64, i64, vp, vp,
                                    i64, i64, vp]),
}

_lock = threading.Lock()
_lib = None


def lib_path() -> str:
    return os.environ.get("POLAR_PACK_LIB", LIB)


def lib() -> C.CDLL:
    """Load the HIP library once; raise if it is absent (no fallback path exists)."""
    global _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not os.path.exists(path):
                raise RuntimeError(f"polar_pack_amd: native library {path} is missing; build it with "
                                   "`python -m polar_pack_amd.build`")
            h = C.CDLL(path)
            for name, (res, args) in EXPORTS.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _lib = h
    return _lib


def check(rc: int, what: str) -> None:
    if rc != PP_OK:
        msg = lib().pp_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def ptr_array(ptrs, ctype=vp):
    arr = (ctype * len(ptrs))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr


def float_array(vals):
    arr = (C.c_float * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = float(v)
    return arr


def raw_stream(dev) -> int:
    """The HIP stream handle of ``dev``'s current torch stream (what
    ``torch.cuda.current_stream(dev).cuda_stream`` returns, without building the stream
    object: 0.2 against 1.9 us per call)."""
    import torch
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def plug_search(idx, n: int, pos0: int, pld: int, rows: int, slices: int, cols: int, dev):
    """int64 device tensor of rows*slices + 1 plug ranges (pp_plug_search): entry
    r*slices + s is the first j with idx[j] >= pos0 + r*pld + s*cols, the last one the first
    j with idx[j] >= pos0 + rows*pld; ``idx`` the ascending uint32 positions (int32 or
    uint32 tensor), one launch."""
    import torch
    row_plug = torch.empty(rows * slices + 1, dtype=torch.int64, device=dev)
    check(lib().pp_plug_search(idx.data_ptr(), n, pos0, pld, rows, slices, cols, row_plug.data_ptr(),
                               raw_stream(dev)), "pp_plug_search")
    return row_plug


# Zeroed workspaces of the kernels that take one zero on entry and leave it zero (the K-slice
# accumulators of pp_quad_mfma, pp_quad_big, pp_dual_mfma): one per (device, stream), grown
# on demand and reused by every call on that stream, since calls on one stream run in order.
# At most ZERO_WS_STREAMS streams per device keep one (least recently used dropped first), so
# callers that cycle through many streams do not pile up device memory; release_workspaces()
# drops them all.  A call that fails drops its stream's buffer (it may not have been left
# zero).  Under stream capture every call gets a fresh zeroed buffer, as the graph records it.
ZERO_WS_STREAMS = 4
_zero_ws = collections.OrderedDict()


def zero_workspace(dev, nbytes: int):
    """(buffer, key): a zeroed uint8 device tensor of at least ``nbytes`` bytes for the current
    stream of ``dev`` (None when nbytes is 0); pass ``key`` to :func:`drop_workspace` if the
    call using it fails."""
    import torch
    if nbytes <= 0:
        return None, None
    dev = torch.device(dev)
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(nbytes, dtype=torch.uint8, device=dev), None
    key = (dev.index, raw_stream(dev))
    with _lock:
        ws = _zero_ws.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=dev)
            _zero_ws[key] = ws
        _zero_ws.move_to_end(key)
        mine = [k for k in _zero_ws if k[0] == key[0]]
        for k in mine[:max(0, len(mine) - ZERO_WS_STREAMS)]:
            del _zero_ws[k]
    return ws, key


def drop_workspace(key) -> None:
    if key is not None:
        with _lock:
            _zero_ws.pop(key, None)


def release_workspaces() -> None:
    """Drop every cached K-slice workspace (their memory returns to torch's caching
    allocator once the calls that used them have completed on their streams)."""
    with _lock:
        _zero_ws.clear()
