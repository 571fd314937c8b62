"""Dual-pack operators: drop-in for the reference's ``polar_kernels.py``.

Same names, arguments, return values and error behaviour as the reference
(polar_kernels.py:9-11, 98-151), computed by the gfx950 HIP library:

* :func:`pack_amp_phase` -- int16 ``((amp & 63) << 10 | (phase & 1023)) - 32768``.
* :func:`quantize_polar_bitpacked` -- per-layer packer (torch on the weights' device).
* :func:`polar_dual_bitpacked` -- one packed pass -> 2 fp16 GEMM outputs.
  Keyword-only extensions: ``plug=(idx, amp)`` (``.dualpack`` plug table,
  polar_bitpack.py:240-243), ``elem_base``, ``layout`` (``"i16"`` kernel layout
  or ``"u16be"`` file layout) and ``chunk_size`` (0 = the kernel's (k*N + n)
  group rule, > 0 = the container's stream-position rule).
* :func:`dual_dequant` -- float32 (or fp16) weights of a code view.

The kernel of a call comes from one table, :data:`polar_pack_amd.routes.DUAL_ROUTES`:
batches of 1-4 tokens (1-8 on the (K,N) kernel layout) run on the fused decode kernels;
2-64 tokens on the int16 (K,N) kernel layout on the matrix-core decode (pp_dual_mfma; to 128
without a plug table on rows it loads 8 codes at a time, its producer/consumer form from 65),
5-64 on container (N,K) rows on its (N,K) form (pp_dual_nk_mfma); larger ones decode once
into fp16 weights (the values the reference's kernel rounds its
weights to, polar_kernels.py:78-82) and run a library fp16 GEMM (hipBLASLt through
torch.matmul).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _native as nat
from . import plugs, routes
from .quad_kernels import _check_device

_LAYOUTS = {"i16": nat.PP_DUAL_I16_OFFSET, "u16be": nat.PP_DUAL_U16_BE}


def pack_amp_phase(amp_q, phase_q):
    """polar_kernels.py:9-11."""
    packed = ((amp_q.to(torch.int32) & 0x3F) << 10) | (phase_q.to(torch.int32) & 0x3FF)
    return (packed - 32768).to(torch.int16)


def quantize_polar_bitpacked(w1, w2, amp_bits=6, num_phases=1024, mu=255, group_size=32):
    """Per-layer dual packer (polar_kernels.py:118-151).

    Returns ``(packed int16 (K,N), bmax fp16 flat, amp_lut fp16[2^amp_bits],
    cos_lut fp16[num_phases], sin_lut fp16[num_phases])`` on w1's device.
    """
    K, N = w1.shape
    amplitude = torch.sqrt(w1 ** 2 + w2 ** 2)
    phase = torch.atan2(w2, w1)
    phase_q = (torch.round((phase + math.pi) / (2 * math.pi) * num_phases).long() % num_phases).to(torch.int16)
    total = K * N
    flat = amplitude.flatten()
    pad = (group_size - total % group_size) % group_size
    if pad:
        flat = torch.nn.functional.pad(flat, (0, pad))
    grouped = flat.reshape(-1, group_size)
    bmax = grouped.abs().max(dim=1, keepdim=True).values
    bmax = torch.where(bmax > 1e-10, bmax, torch.ones_like(bmax))
    norm = grouped / bmax
    log_mu = math.log(1 + mu)
    compressed = torch.sign(norm) * torch.log1p(mu * norm.abs()) / log_mu
    levels = (1 << amp_bits) - 1
    amp_q = torch.round(compressed * levels).clamp(0, levels).to(torch.int8).flatten()[:total].reshape(K, N)
    bmax = bmax.flatten().to(torch.float16)
    packed = pack_amp_phase(amp_q, phase_q)
    phases = torch.linspace(-math.pi, math.pi, num_phases + 1)[:-1]
    cos_lut = torch.cos(phases).to(torch.float16).to(w1.device)
    sin_lut = torch.sin(phases).to(torch.float16).to(w1.device)
    i = torch.arange(levels + 1, dtype=torch.float32)
    amp_lut = ((torch.exp(i / levels * log_mu) - 1.0) / mu).to(torch.float16).to(w1.device)
    return packed, bmax, amp_lut, cos_lut, sin_lut


def _lut_dtype(*ts):
    dt = ts[0].dtype
    for t in ts:
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError("dual LUTs must be contiguous tensors of one dtype")
    if dt == torch.float16:
        return nat.PP_F16
    if dt == torch.float32:
        return nat.PP_F32
    raise TypeError(f"dual LUT dtype must be float16 or float32, got {dt}")


def _codes_view(packed, layout):
    if layout not in _LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}")
    if packed.element_size() != 2:
        raise TypeError("dual codes are 16-bit (int16 kernel layout or uint16 big-endian file layout)")
    return _LAYOUTS[layout]


def _dual_plug(plug, device):
    if plug is None:
        return None, None, 0, ()
    idx, amp = plug
    if idx.dtype not in (torch.uint32, torch.int32) or amp.dtype != torch.float16 or amp.numel() != idx.numel():
        raise TypeError("plug must be (uint32 idx (P,), float16 amplitude (P,))")
    if idx.device != device or amp.device != device:
        raise ValueError("plug tensors must be on the codes' device")
    idx, amp = plugs.ascending(idx.contiguous(), amp.contiguous())
    return idx.data_ptr(), amp.data_ptr(), idx.numel(), (idx, amp)


def polar_dual_bitpacked(a_fp16, packed, bmax, amp_lut, cos_lut, sin_lut, num_phases=1024, group_size=32, *,
                         plug=None, elem_base=0, layout="i16", chunk_size=0, fused=None):
    """2 GEMMs from one packed pass (polar_kernels.py:98-115); returns ``(out1, out2)`` fp16 (M,N).

    ``plug=(idx uint32 (P,), amp fp16 (P,))`` replaces the amplitude of the pair at storage
    offset ``idx - elem_base`` (polar_bitpack.py:240-243); entries in any order (sorted once
    per table on the device, :mod:`polar_pack_amd.plugs`).  The kernel is chosen by
    :data:`polar_pack_amd.routes.DUAL_ROUTES` from the storage of ``packed``, M, the plug table
    and ``fused`` (the int16 (K,N) layout or container rows, K % 32 == 0): True runs the
    matrix-core decode at any size, False never (the fused row kernels up to 4 or 8 tokens,
    then the fp16 decode + library GEMM), None (default) picks by size."""
    M, K = a_fp16.shape
    K_b, N = packed.shape
    assert K == K_b
    dev = _check_device(a_fp16, packed, bmax, amp_lut, cos_lut, sin_lut)
    if a_fp16.dtype != torch.float16 or bmax.dtype != torch.float16:
        raise TypeError("a and bmax must be float16")
    out1, out2 = torch.empty((2, M, N), dtype=torch.float16, device=dev).unbind(0)
    if M == 0 or N == 0:
        return out1, out2
    if K == 0:
        out1.zero_()
        out2.zero_()
        return out1, out2
    lay = _codes_view(packed, layout)
    lut_dt = _lut_dtype(amp_lut, cos_lut, sin_lut)
    if cos_lut.numel() != num_phases or sin_lut.numel() != num_phases:
        raise ValueError("cos_lut / sin_lut must have num_phases entries")
    a = a_fp16
    if a.stride(1) != 1 or a.data_ptr() % 16 or (M > 1 and a.stride(0) % 8):
        a = a.contiguous()
    bmax = bmax.contiguous()
    pi, pa, pn, keep = _dual_plug(plug, dev)
    L = nat.lib()
    route = dual_call_route(packed, M, layout=layout, group_size=group_size, chunk_size=chunk_size,
                            elem_base=elem_base, plug_n=pn, fused=fused)
    if route == "dual_mfma":
        _dual_mfma(a, packed, bmax, amp_lut, cos_lut, sin_lut, num_phases, group_size, lut_dt, keep, pn,
                   int(elem_base), out1, out2, L, dev)
        del keep
        return out1, out2
    if route == "dual_nk_mfma":
        _dual_nk_mfma(a, packed, lay, bmax, amp_lut, cos_lut, sin_lut, num_phases, group_size, chunk_size, lut_dt,
                      keep, pn, int(elem_base), out1, out2, L, dev)
        del keep
        return out1, out2
    if route == "prefill":
        # fp16 weights laid out (N,K), the GEMM's fastest right operand, then one batched GEMM
        # over the two models: K-contiguous codes (container rows) decode along their storage
        # into it (the kernel rule's groups need the (K,N) indices); (K,N) codes with unit
        # column stride through the transposing decode; other strides into (K,N) weights
        kn = "dual_kn" in routes.dual_storage(packed.stride(0), packed.stride(1), packed.data_ptr(), K, N, layout,
                                              group_size, chunk_size, int(elem_base))
        nk = packed.stride(0) == 1 and packed.stride(1) != 1 and chunk_size > 0
        if kn:
            w = torch.empty((2, N, K), dtype=torch.float16, device=dev)
            _dequant_t_into(packed, bmax, amp_lut, cos_lut, sin_lut, num_phases, group_size, plug,
                            elem_base, layout, w[0], w[1])
        else:
            view = packed.t() if nk else packed
            w = torch.empty((2,) + tuple(view.shape), dtype=torch.float16, device=dev)
            _dequant_into(view, bmax, amp_lut, cos_lut, sin_lut, num_phases, group_size, plug, elem_base,
                          layout, chunk_size, w[0], w[1])
            if not nk:
                out = torch.matmul(a_fp16, w)       # (2, M, N)
                return out[0], out[1]
        out = torch.matmul(a_fp16, w.transpose(1, 2))
        return out[0], out[1]
    # dual_kn, dual_rows, generic: pp_dual_gemm picks among them alike
    ws_bytes = L.pp_dual_gemm_workspace_size(a.data_ptr(), a.stride(0), a.stride(1), packed.data_ptr(),
                                             packed.stride(0), packed.stride(1), group_size, chunk_size,
                                             int(elem_base), pn, M, N, K)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    stream = nat.raw_stream(dev)
    rc = L.pp_dual_gemm(a.data_ptr(), a.stride(0), a.stride(1), packed.data_ptr(), lay, packed.stride(0),
                        packed.stride(1), bmax.data_ptr(), group_size, chunk_size, amp_lut.data_ptr(),
                        amp_lut.numel(), cos_lut.data_ptr(), sin_lut.data_ptr(), num_phases, lut_dt, pi, pa, pn,
                        int(elem_base), out1.data_ptr(), out2.data_ptr(), out1.stride(0), out1.stride(1), M, N, K,
                        ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    nat.check(rc, "pp_dual_gemm")
    del keep
    return out1, out2


def dual_call_route(packed, M, *, layout="i16", group_size=32, chunk_size=0, elem_base=0, plug_n=0, fused=None):
    """The route (:data:`polar_pack_amd.routes.DUAL_ROUTES`) of a ``polar_dual_bitpacked`` call
    with these codes, M tokens and ``plug_n`` plug entries."""
    K, N = packed.shape
    caps = routes.dual_storage(packed.stride(0), packed.stride(1), packed.data_ptr(), K, N, layout, group_size,
                               chunk_size, int(elem_base), plug_n)
    return routes.dual_route(M, K, N, caps, plug_n > 0, fused)


def _dual_mfma(a, packed, bmax, amp_lut, cos_lut, sin_lut, num_phases, group_size, lut_dt, keep, pn, elem_base,
               out1, out2, L, dev):
    """More than 8 tokens on the int16 (K,N) layout: the matrix-core decode (pp_dual_mfma).
    Plug positions (k*ldk + n of the storage, relative to elem_base) move to the kernel's
    (N,K) frame n*K + k and are located per (column, K slice) (pp_plug_search)."""
    M, K = a.shape
    N = packed.shape[1]
    ldk = packed.stride(0)
    plan = (ctypes.c_int64 * 2)()
    nat.check(L.pp_dual_mfma_plan(M, N, K, ctypes.byref(plan, 0), ctypes.byref(plan, 8)), "pp_dual_mfma_plan")
    slices, cols = int(plan[0]), int(plan[1])
    row_plug = None
    if pn:
        p = (keep[0].view(torch.int32).to(torch.int64) & 0xFFFFFFFF) - elem_base
        k, n = p // ldk, p % ldk
        ok = (p >= 0) & (k < K) & (n < N)
        # entries outside the K x N block go to position N*K, past every column's search
        # range: the entry count stays static (no wait on the device; graph-capturable)
        pos, order = torch.sort(torch.where(ok, n * K + k, N * K))
        amps = keep[1][order].contiguous()
        keep = (torch.where(pos >= 2 ** 31, pos - 2 ** 32, pos).to(torch.int32).contiguous(), amps)
        row_plug = nat.plug_search(keep[0], pn, 0, K, N, slices, cols, dev)
    ws_bytes = L.pp_dual_mfma_workspace_size(M, N, slices)
    ws, wkey = nat.zero_workspace(dev, ws_bytes)
    stream = nat.raw_stream(dev)
    rc = L.pp_dual_mfma(packed.data_ptr(), ldk, a.data_ptr(), a.stride(0), bmax.data_ptr(), group_size,
                        amp_lut.data_ptr(), amp_lut.numel(), cos_lut.data_ptr(), sin_lut.data_ptr(), num_phases,
                        lut_dt, keep[0].data_ptr() if pn else None, keep[1].data_ptr() if pn else None, pn,
                        row_plug.data_ptr() if row_plug is not None else None, 0, K, slices, cols,
                        out1.data_ptr(), out2.data_ptr(), out1.stride(0), M, N, K,
                        ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    if rc:
        nat.drop_workspace(wkey)
    nat.check(rc, "pp_dual_mfma")
    del keep, row_plug, ws


def _dual_nk_mfma(a, packed, lay, scales, amp_lut, cos_lut, sin_lut, num_phases, group_size, chunk_size, lut_dt,
                  keep, pn, elem_base, out1, out2, L, dev):
    """5-64 tokens on (N,K) container rows: the matrix-core decode (pp_dual_nk_mfma), plug
    starts per (row, K slice) found on the device (pp_plug_search; polar_bitpack.py:240-243)."""
    M, K = a.shape
    N = packed.shape[1]
    ldc = packed.stride(1)
    plan = (ctypes.c_int64 * 2)()
    nat.check(L.pp_dual_mfma_plan(M, N, K, ctypes.byref(plan, 0), ctypes.byref(plan, 8)), "pp_dual_mfma_plan")
    slices, cols = int(plan[0]), int(plan[1])
    row_plug = nat.plug_search(keep[0], pn, elem_base, ldc, N, slices, cols, dev) if pn else None
    ws_bytes = L.pp_dual_mfma_workspace_size(M, N, slices)
    ws, wkey = nat.zero_workspace(dev, ws_bytes)
    stream = nat.raw_stream(dev)
    rc = L.pp_dual_nk_mfma(packed.data_ptr(), lay, ldc, elem_base, a.data_ptr(), a.stride(0), scales.data_ptr(),
                           scales.numel(), group_size, chunk_size, amp_lut.data_ptr(), amp_lut.numel(),
                           cos_lut.data_ptr(), sin_lut.data_ptr(), num_phases, lut_dt,
                           keep[0].data_ptr() if pn else None, keep[1].data_ptr() if pn else None, pn,
                           row_plug.data_ptr() if row_plug is not None else None, slices, cols, out1.data_ptr(),
                           out2.data_ptr(), out1.stride(0), M, N, K, ws.data_ptr() if ws is not None else None,
                           ws_bytes, stream)
    if rc:
        nat.drop_workspace(wkey)
    nat.check(rc, "pp_dual_nk_mfma")
    del keep, row_plug, ws


def dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut, num_phases=1024, group_size=32, *, plug=None,
                 elem_base=0, layout="i16", chunk_size=0, dtype=torch.float32):
    """(K,N) weight pair ``(w1, w2)`` of a code view, plug applied, float32 or float16
    (``dtype``)."""
    K, N = packed.shape
    dev = _check_device(packed, bmax, amp_lut, cos_lut, sin_lut)
    if dtype not in (torch.float32, torch.float16):
        raise TypeError("dtype must be torch.float32 or torch.float16")
    w1 = torch.empty((K, N), dtype=dtype, device=dev)
    w2 = torch.empty_like(w1)
    if K * N == 0:
        return w1, w2
    _dequant_into(packed, bmax, amp_lut, cos_lut, sin_lut, num_phases, group_size, plug, elem_base, layout,
                  chunk_size, w1, w2)
    return w1, w2


def _dequant_into(packed, bmax, amp_lut, cos_lut, sin_lut, num_phases, group_size, plug, elem_base, layout,
                  chunk_size, w1, w2):
    """Decode a (K,N) code view into the contiguous (K,N) tensors w1, w2 (float32 or fp16)."""
    K, N = packed.shape
    dev = packed.device
    lay = _codes_view(packed, layout)
    lut_dt = _lut_dtype(amp_lut, cos_lut, sin_lut)
    pi, pa, pn, keep = _dual_plug(plug, dev)
    stream = nat.raw_stream(dev)
    fn = nat.lib().pp_dual_dequant if w1.dtype == torch.float32 else nat.lib().pp_dual_dequant_f16
    rc = fn(packed.data_ptr(), lay, packed.stride(0), packed.stride(1), bmax.contiguous().data_ptr(), group_size,
            chunk_size, amp_lut.data_ptr(), amp_lut.numel(), cos_lut.data_ptr(), sin_lut.data_ptr(), num_phases,
            lut_dt, pi, pa, pn, int(elem_base), w1.data_ptr(), w2.data_ptr(), N, K, stream)
    nat.check(rc, "pp_dual_dequant")
    del keep


def _dequant_t_into(packed, bmax, amp_lut, cos_lut, sin_lut, num_phases, group_size, plug, elem_base, layout, w1, w2):
    """Decode (K,N) codes with unit column stride (the kernel's group rule) into the
    contiguous fp16 (N,K) tensors w1, w2: the weights transposed (pp_dual_dequant_f16_t)."""
    K, N = packed.shape
    dev = packed.device
    lay = _codes_view(packed, layout)
    lut_dt = _lut_dtype(amp_lut, cos_lut, sin_lut)
    pi, pa, pn, keep = _dual_plug(plug, dev)
    stream = nat.raw_stream(dev)
    rc = nat.lib().pp_dual_dequant_f16_t(packed.data_ptr(), lay, packed.stride(0), bmax.contiguous().data_ptr(),
                                         group_size, amp_lut.data_ptr(), amp_lut.numel(), cos_lut.data_ptr(),
                                         sin_lut.data_ptr(), num_phases, lut_dt, pi, pa, pn, int(elem_base),
                                         w1.data_ptr(), w2.data_ptr(), N, K, stream)
    nat.check(rc, "pp_dual_dequant_f16_t")
    del keep


def header_luts(amp_bits=6, phase_bits=10, mu=255.0, device=None):
    """float32 LUTs of a ``.dualpack`` header, computed in float64 and rounded once:
    amp_lut[i] = expm1(i/levels * ln(1+mu)) / mu and the phase tables of
    ang = i / 2^phase_bits * 2 pi - pi (polar_bitpack.py:213-215, 237, 245)."""
    levels = 2 ** amp_bits - 1
    i = torch.arange(levels + 1, dtype=torch.float64)
    amp = torch.expm1(i / levels * math.log1p(mu)) / mu
    nph = 1 << phase_bits
    j = torch.arange(nph, dtype=torch.float64)
    ang = j / nph * 2 * math.pi - math.pi
    return [t.to(torch.float32).to(device) for t in (amp, torch.cos(ang), torch.sin(ang))]
