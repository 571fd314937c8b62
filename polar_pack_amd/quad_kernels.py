"""Quad-pack operators: drop-in for the reference's ``quad_kernels.py``.

Same names, arguments, return values and error behaviour as the reference
(quad_kernels.py:16-50, 146-159), computed by the gfx950 HIP library:

* :func:`pack_quad_layer` -- 4 (K,N) weight matrices -> uint32 codes (K,N),
  7 fp16 LUTs, 4 RMS scales (torch on the weights' device; the uint32 words
  are assembled on the device instead of the reference's numpy round trip).
* :func:`quad_bitpacked` -- one packed pass -> 4 fp16 GEMM outputs.
  Keyword-only extensions: ``plug=(idx, vals)`` (the ``.quadpack`` plug table,
  quaternion_packer.py:187-193) and ``elem_base``.
* :func:`quad_dequant` -- float32 (or fp16) weights of a code view.

The kernel of a call comes from one table, :data:`polar_pack_amd.routes.QUAD_ROUTES`
(K % 32 == 0 for the matrix cores): on an (N,K) block seen as (K,N) (the container layout)
the row kernel to 4 tokens, the matrix-core batch decode at 5-64 and the fused matrix-core
kernel at 65-128; on (K,N) storage the fused (K,N) row kernel at 1 token (and with plug
entries up to 8) and the fused matrix-core kernel on the codes as stored from 2 tokens (3
when N > K) to 256 (two 8-token row passes up to 16 tokens when K % 32 != 0); larger
batches, and more tokens on other layouts, decode once into fp16 weights (the values the
reference's kernel rounds its weights to, quad_kernels.py:117-126) and run a library fp16
GEMM (hipBLASLt through torch.matmul), where the matmul's compute, not the weight stream,
bounds the time.
"""
from __future__ import annotations

import collections
import ctypes
import math
import threading
import weakref

import torch

from . import _native as nat
from . import plugs, routes

MU = 255.0   # quad_kernels.py:13
_plans_lock = threading.Lock()


def _u32_words(nq, q1, q2, q3):
    """Assemble [nq|q1|q2|q3] words on the device as a torch.uint32 tensor."""
    w = (nq.to(torch.int64) << 24) | (q1.to(torch.int64) << 16) | (q2.to(torch.int64) << 8) | q3.to(torch.int64)
    w = torch.where(w >= 2 ** 31, w - 2 ** 32, w).to(torch.int32)
    return w.view(torch.uint32)


def pack_quad_layer(w1, w2, w3, w4, mu=MU):
    """Pack 4 weight matrices (K,N) into uint32 codes + LUTs (quad_kernels.py:16-50).

    Returns ``(codes uint32 (K,N) on w1.device, luts [norm, cos1, sin1, cos2,
    sin2, cos3, sin3] fp16[256] on w1.device, scales [4 floats])``.
    """
    ws = [w1, w2, w3, w4]
    s = [torch.sqrt((w.float() ** 2).mean()) for w in ws]
    wn = [w.float() / sk for w, sk in zip(ws, s)]
    r = torch.sqrt(wn[0] ** 2 + wn[1] ** 2 + wn[2] ** 2 + wn[3] ** 2)
    r_max = float(r.max()) * 1.001
    log_mu = math.log1p(mu)
    t1 = torch.atan2(torch.sqrt(wn[1] ** 2 + wn[2] ** 2 + wn[3] ** 2), wn[0])
    t2 = torch.atan2(torch.sqrt(wn[2] ** 2 + wn[3] ** 2), wn[1])
    t3 = torch.atan2(wn[3], wn[2]) % (2 * math.pi)
    nq = torch.round(torch.log1p(mu * r / r_max) / log_mu * 255).clip(0, 255)
    q1 = torch.round(t1 / math.pi * 255).clip(0, 255)
    q2 = torch.round(t2 / math.pi * 255).clip(0, 255)
    q3 = torch.round(t3 / (2 * math.pi) * 255).clip(0, 255)
    codes = _u32_words(nq, q1, q2, q3)
    i = torch.arange(256, dtype=torch.float32)
    half_turn = i / 255 * math.pi
    full_turn = i / 255 * 2 * math.pi
    tables = [(torch.exp(i / 255 * log_mu) - 1) * r_max / mu,
              torch.cos(half_turn), torch.sin(half_turn), torch.cos(half_turn), torch.sin(half_turn),
              torch.cos(full_turn), torch.sin(full_turn)]
    luts = [t.to(torch.float16).to(w1.device) for t in tables]
    return codes, luts, [float(sk) for sk in s]


def _lut_args(luts):
    if len(luts) != 7:
        raise ValueError("quad LUTs: expected 7 tables [norm, cos1, sin1, cos2, sin2, cos3, sin3]")
    dt = luts[0].dtype
    for t in luts:
        if t.dtype != dt or t.numel() < 256 or not t.is_contiguous():
            raise ValueError("quad LUTs must be 7 contiguous tensors of one dtype with 256 entries")
    if dt == torch.float16:
        code = nat.PP_F16
    elif dt == torch.float32:
        code = nat.PP_F32
    else:
        raise TypeError(f"quad LUT dtype must be float16 or float32, got {dt}")
    return nat.ptr_array([t.data_ptr() for t in luts]), code


def _plug_args(plug, device):
    if plug is None:
        return None, None, 0, ()
    idx, vals = plug
    if idx.dtype not in (torch.uint32, torch.int32):
        raise TypeError("plug index must be uint32 (or int32 holding uint32 bits)")
    if vals.dtype != torch.float16 or vals.numel() != 4 * idx.numel():
        raise TypeError("plug values must be float16 (P, 4)")
    if idx.device != device or vals.device != device:
        raise ValueError("plug tensors must be on the codes' device")
    idx, vals = plugs.ascending(idx.contiguous(), vals.contiguous())
    return idx.data_ptr(), vals.data_ptr(), idx.numel(), (idx, vals)


def _check_device(*ts):
    dev = ts[0].device
    if dev.type != "cuda":
        raise ValueError("polar_pack_amd operators run on a ROCm device (tensor.device.type == 'cuda')")
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError("all operands must be on one device")
    return dev


def quad_bitpacked(a, codes, luts, scales, *, plug=None, elem_base=0, fused=None):
    """4 GEMMs from one packed pass (quad_kernels.py:146-159).

    ``a`` fp16 (M,K); ``codes`` uint32 (K,N) view (any strides); ``luts`` the
    7 tables of :func:`pack_quad_layer` (fp16 or fp32); ``scales`` 4 floats.
    Returns a list of 4 fp16 (M,N) tensors ``out_k = fp16(s_k * a @ W_k)``.
    ``plug=(idx uint32 (P,), vals fp16 (P,4))`` replaces the normalised tuple
    of the element at storage offset ``idx - elem_base`` of ``codes``, as a ``.quadpack``
    file's table does (quaternion_packer.py:187-193); entries in any order (sorted once per
    table on the device, :mod:`polar_pack_amd.plugs`).
    The kernel is chosen by :data:`polar_pack_amd.routes.QUAD_ROUTES` from the storage of
    ``codes``, M, the plug table and ``fused``: None (default) picks by size, True runs the
    fused matrix-core kernel wherever it can (K % 32 == 0), False never runs it (the fp16
    decode + library GEMM instead above 64 tokens, which needs 8 bytes of scratch per code
    word).
    """
    M, K = a.shape
    K_b, N = codes.shape
    assert K == K_b
    dev = _check_device(a, codes, *luts)
    if a.dtype != torch.float16:
        raise TypeError("a must be float16")
    if codes.dtype not in (torch.uint32, torch.int32):
        raise TypeError("codes must be uint32")
    # the 4 outputs as slices of one allocation (one allocator call instead of 4)
    outs = list(torch.empty((4, M, N), dtype=torch.float16, device=dev).unbind(0))
    if M == 0 or N == 0:
        return outs
    if K == 0:
        for o in outs:
            o.zero_()
        return outs
    lut_ptrs, lut_dtype = _lut_args(luts)
    sc = nat.float_array(scales)
    pi, pv, pn, keep = _plug_args(plug, dev)
    route = quad_call_route(codes, M, pn, fused)
    L = nat.lib()
    if route in ("big_nk", "big_kn"):
        lay = nat.PP_QUAD_NK if route == "big_nk" else nat.PP_QUAD_KN
        _quad_big(a, codes, lay, lut_ptrs, lut_dtype, sc, keep, pn, int(elem_base), outs, L, dev)
    elif route == "kn_mfma":
        _quad_kn_mfma(a, codes, lut_ptrs, lut_dtype, sc, keep, pn, int(elem_base), outs, L, dev)
    elif route == "mfma":
        for i0 in range(0, M, 64):        # the matrix-core decode takes up to 64 tokens per launch
            i1 = min(M, i0 + 64)
            _quad_mfma(a[i0:i1], codes, lut_ptrs, lut_dtype, sc, keep, pn, int(elem_base),
                       [o[i0:i1] for o in outs], L, dev)
    elif route == "prefill":
        _quad_prefill(a, codes, lut_ptrs, lut_dtype, sc, pi, pv, pn, int(elem_base), outs, L, dev)
    elif route == "rows":
        _quad_rows(a, codes, lut_ptrs, lut_dtype, sc, keep, pn, int(elem_base), outs, L, dev)
    else:                                 # kn, generic: pp_quad_gemm picks among them alike
        _quad_gemm(a, codes, lut_ptrs, lut_dtype, sc, pi, pv, pn, int(elem_base), outs, L, dev)
    del keep
    return outs


def quad_call_route(codes, M, plug_n=0, fused=None):
    """The route (:data:`polar_pack_amd.routes.QUAD_ROUTES`) of a ``quad_bitpacked`` call with
    these codes, M tokens and ``plug_n`` plug entries."""
    K, N = codes.shape
    caps = routes.quad_storage(codes.stride(0), codes.stride(1), codes.data_ptr(), K, N, plug_n)
    return routes.quad_route(M, K, N, caps, plug_n > 0, fused)


# Plans of the row kernel's one-Linear launches (pp_quad_rows): per plug table (the sorted
# copy plugs.ascending returns, checked by identity and version), position, shape and token
# count, the range [lo, hi) of the table's entries inside the Linear's rows and each
# wavefront's first entry (pp_quad_rows_plan over that range).  Made once, on the first call
# outside stream capture (finding the range reads two numbers back from the device).
_ROWS_PLANS = collections.OrderedDict()
_ROWS_PLANS_MAX = 2048


def _rows_plan(idx, pn, elem_base, ldc, M, N, K, L, dev):
    """(lo, hi, wave_plug) for the plug entries of an (N,K) Linear at ``elem_base``."""
    key = (id(idx), elem_base, ldc, M, N, K)
    with _plans_lock:
        hit = _ROWS_PLANS.get(key)
        if hit is not None:
            ref, ver, plan = hit
            if ref() is idx and idx._version == ver:
                _ROWS_PLANS.move_to_end(key)
                return plan
    capturing = torch.cuda.is_current_stream_capturing()
    if capturing:
        lo, hi = 0, pn                    # no host read-back under capture: the whole table
    else:
        pos = idx.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
        bounds = torch.tensor([elem_base, elem_base + (N - 1) * ldc + K], dtype=torch.int64, device=dev)
        lo, hi = (int(v) for v in torch.searchsorted(pos, bounds).tolist())
    wave_plug = torch.empty(int(L.pp_quad_rows_plan_size(M)), dtype=torch.int64, device=dev)
    if hi > lo:
        nat.check(L.pp_quad_rows_plan(idx.data_ptr() + 4 * lo, hi - lo, elem_base, ldc, M, N, K, wave_plug.data_ptr(),
                                      nat.raw_stream(dev)), "pp_quad_rows_plan")
    plan = (lo, hi, wave_plug)
    if not capturing:
        with _plans_lock:
            _ROWS_PLANS[key] = (weakref.ref(idx), idx._version, plan)
            while len(_ROWS_PLANS) > _ROWS_PLANS_MAX:
                _ROWS_PLANS.popitem(last=False)
    return plan


def _quad_rows(a, codes, lut_ptrs, lut_dtype, sc, keep, pn, elem_base, outs, L, dev):
    """(N,K) rows at 1-8 tokens: the row kernel's one-Linear launch (pp_quad_rows), with its
    plan (the Linear's slice of the plug table and each wavefront's first entry) cached per
    plug table, and column slices meeting in the stream's zeroed workspace."""
    M, K = a.shape
    N = codes.shape[1]
    ldc = codes.stride(1)
    if a.stride(1) != 1 or a.data_ptr() % 16 or (M > 1 and a.stride(0) % 8):
        a = a.contiguous()
    lo = hi = 0
    wave_plug = None
    if pn:
        lo, hi, wave_plug = _rows_plan(keep[0], pn, elem_base, ldc, M, N, K, L, dev)
    ws_bytes = L.pp_quad_rows_workspace_size(M, N, K)
    ws, wkey = nat.zero_workspace(dev, ws_bytes)
    n = hi - lo
    rc = L.pp_quad_rows(a.data_ptr(), a.stride(0), codes.data_ptr(), ldc, lut_ptrs, lut_dtype, sc,
                        keep[0].data_ptr() + 4 * lo if n else None, keep[1].data_ptr() + 8 * lo if n else None,
                        None, n, wave_plug.data_ptr() if n else None, elem_base,
                        nat.ptr_array([o.data_ptr() for o in outs]), outs[0].stride(0), outs[0].stride(1),
                        M, N, K, ws.data_ptr() if ws is not None else None, ws_bytes, nat.raw_stream(dev))
    if rc:
        nat.drop_workspace(wkey)
    nat.check(rc, "pp_quad_rows")


def _quad_gemm(a, codes, lut_ptrs, lut_dtype, sc, pi, pv, pn, elem_base, outs, L, dev):
    """pp_quad_gemm: the row kernel on (N,K) rows, the (K,N) row kernel on (K,N) codes (8 tokens
    per pass), the generic decode + GEMV otherwise."""
    M, K = a.shape
    N = codes.shape[1]
    if a.stride(1) != 1 or a.data_ptr() % 16 or (M > 1 and a.stride(0) % 8):
        a = a.contiguous()
    ws_bytes = L.pp_quad_gemm_workspace_size(a.data_ptr(), a.stride(0), a.stride(1), codes.data_ptr(),
                                             codes.stride(0), codes.stride(1), pn, M, N, K)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    stream = nat.raw_stream(dev)
    rc = L.pp_quad_gemm(a.data_ptr(), a.stride(0), a.stride(1), codes.data_ptr(), codes.stride(0),
                        codes.stride(1), lut_ptrs, lut_dtype, sc, pi, pv, pn, elem_base,
                        nat.ptr_array([o.data_ptr() for o in outs]), outs[0].stride(0), outs[0].stride(1),
                        M, N, K, ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    nat.check(rc, "pp_quad_gemm")


def transposed_plug(idx, vals, elem_base, ldk, K, N):
    """Plug entries of a (K,N) code tensor (row stride ``ldk``, positions relative to
    ``elem_base``) moved to its (N,K) transpose: position k*ldk + n becomes n*K + k, entries
    outside the K x N block to N*K (past every row's search range, so the entry count stays
    that of the input: no wait on the device, and the call can be captured in a graph),
    re-sorted (the matrix-core path searches them).
    Returns (int32 tensor holding the uint32 positions, (P, 4) fp16 values)."""
    p = (idx.view(torch.int32).to(torch.int64) & 0xFFFFFFFF) - elem_base
    k, n = p // ldk, p % ldk
    ok = (p >= 0) & (k < K) & (n < N)
    pos, order = torch.sort(torch.where(ok, n * K + k, N * K))
    return (torch.where(pos >= 2 ** 31, pos - 2 ** 32, pos).to(torch.int32).contiguous(),
            vals.reshape(-1, 4)[order].contiguous())


def _quad_kn_mfma(a, codes, lut_ptrs, lut_dtype, sc, keep, pn, elem_base, outs, L, dev):
    """9-64 tokens on (K,N) storage: transpose the codes to (N,K) rows (pp_quad_codes_nk,
    one read and one write of the codes) and run the matrix-core decode on them; plug
    positions are moved to the transposed storage and re-sorted."""
    K, N = codes.shape
    ldk = codes.stride(0)
    cnk = torch.empty((N, K), dtype=torch.int32, device=dev)
    stream = nat.raw_stream(dev)
    nat.check(L.pp_quad_codes_nk(codes.data_ptr(), ldk, K, N, cnk.data_ptr(), stream), "pp_quad_codes_nk")
    view = cnk.view(torch.uint32).t()
    keep2, pn2 = (), 0
    if pn:
        keep2 = transposed_plug(keep[0], keep[1], elem_base, ldk, K, N)
        pn2 = int(keep2[0].numel())
    for i0 in range(0, a.shape[0], 64):
        i1 = min(a.shape[0], i0 + 64)
        _quad_mfma(a[i0:i1], view, lut_ptrs, lut_dtype, sc, keep2, pn2, 0, [o[i0:i1] for o in outs], L, dev)


def _quad_big(a, codes, layout, lut_ptrs, lut_dtype, sc, keep, pn, elem_base, outs, L, dev):
    """More than 64 tokens on (N,K) or (K,N) storage, or 9-64 on (K,N): the fused decode
    on the matrix cores (pp_quad_big).  Plug entries are located per (row, K slice) (pp_plug_search)
    (quaternion_packer.py:188-189); on (K,N) storage they are first moved to the (N,K)
    frame the kernel reads them in."""
    M, K = a.shape
    N = codes.shape[1]
    if a.stride(1) != 1 or a.data_ptr() % 16 or (M > 1 and a.stride(0) % 8):
        a = a.contiguous()
    plan = (ctypes.c_int64 * 2)()
    nat.check(L.pp_quad_big_plan(M, N, K, layout, ctypes.byref(plan, 0), ctypes.byref(plan, 8)), "pp_quad_big_plan")
    slices, cols = int(plan[0]), int(plan[1])
    if layout == nat.PP_QUAD_NK:
        ldc = codes.stride(1)
        pos0, pld = elem_base, ldc
    else:
        ldc = codes.stride(0)
        pos0, pld = 0, K
        if pn:
            keep = transposed_plug(keep[0], keep[1], elem_base, ldc, K, N)
            pn = int(keep[0].numel())
    row_plug = None
    if pn:
        row_plug = nat.plug_search(keep[0], pn, pos0, pld, N, slices, cols, dev)
    ws_bytes = L.pp_quad_big_workspace_size(M, N, slices)
    ws, wkey = nat.zero_workspace(dev, ws_bytes)
    stream = nat.raw_stream(dev)
    rc = L.pp_quad_big(codes.data_ptr(), layout, ldc, a.data_ptr(), a.stride(0), lut_ptrs, lut_dtype, sc,
                       keep[0].data_ptr() if pn else None, keep[1].data_ptr() if pn else None, pn,
                       row_plug.data_ptr() if row_plug is not None else None, pos0, pld, slices, cols,
                       nat.ptr_array([o.data_ptr() for o in outs]), outs[0].stride(0), M, N, K,
                       ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    if rc:
        nat.drop_workspace(wkey)
    nat.check(rc, "pp_quad_big")
    del keep, row_plug, ws
    return outs


def _quad_prefill(a, codes, lut_ptrs, lut_dtype, sc, pi, pv, pn, elem_base, outs, L, dev):
    """Decode into fp16 weights s_m * W_m (plug applied), then one batched fp16 GEMM over the
    4 models with the activations broadcast (one library call instead of 4: 101-113 against
    152-177 us for four 1024 x 4096 x 4096 products, measured).  The weights are laid out
    (N,K), the GEMM's fastest right operand (x @ W as x @ (W^T)^T: 101 against 113 us for
    the 4 products above, 28 against 37 us at 128 tokens): codes with K contiguous (an (N,K)
    buffer seen as (K,N)) decode along their storage into it; (K,N) codes with unit column
    stride through the transposing decode (pp_quad_dequant_f16_t); other strides into (K,N)
    weights."""
    M, K = a.shape
    N = codes.shape[1]
    nk = codes.stride(0) == 1 and codes.stride(1) != 1
    stream = nat.raw_stream(dev)
    if not nk and codes.stride(1) == 1 and codes.stride(0) >= N and codes.stride(0) % 4 == 0 and N % 8 == 0 \
            and K % 8 == 0 and codes.data_ptr() % 16 == 0:
        w = torch.empty((4, N, K), dtype=torch.float16, device=dev)
        rc = L.pp_quad_dequant_f16_t(codes.data_ptr(), codes.stride(0), lut_ptrs, lut_dtype, sc, pi, pv, pn,
                                     elem_base, nat.ptr_array([w[m].data_ptr() for m in range(4)]), N, K, stream)
        nat.check(rc, "pp_quad_dequant_f16_t")
    else:
        view = codes.t() if nk else codes
        R, C = view.shape
        w = torch.empty((4, R, C), dtype=torch.float16, device=dev)
        rc = L.pp_quad_dequant_f16(view.data_ptr(), view.stride(0), view.stride(1), lut_ptrs, lut_dtype, sc, pi, pv,
                                   pn, elem_base, nat.ptr_array([w[m].data_ptr() for m in range(4)]), C, R, stream)
        nat.check(rc, "pp_quad_dequant_f16")
        if not nk:
            out = torch.matmul(a, w)      # (4, M, N): the outputs are its 4 contiguous slices
            outs[:] = [out[m] for m in range(4)]
            return
    out = torch.matmul(a, w.transpose(1, 2))
    outs[:] = [out[m] for m in range(4)]


def _quad_mfma(a, codes, lut_ptrs, lut_dtype, sc, keep, pn, elem_base, outs, L, dev):
    """5-64 tokens on (N,K) rows: the matrix-core batch decode (pp_quad_mfma), plug starts per
    (row, K slice) found on the device (pp_plug_search; quaternion_packer.py:188-189)."""
    M, K = a.shape
    N = codes.shape[1]
    ldc = codes.stride(1)
    if a.stride(1) != 1 or a.data_ptr() % 16 or (M > 1 and a.stride(0) % 8):
        a = a.contiguous()
    from .stream import mfma_slices
    slices, cols = mfma_slices(N, K, int(L.pp_quad_mfma_waves(M)))
    row_plug = None
    if pn:
        row_plug = nat.plug_search(keep[0], pn, elem_base, ldc, N, slices, cols, dev)
    ws_bytes = L.pp_quad_mfma_workspace_size(M, N, slices)
    ws, wkey = nat.zero_workspace(dev, ws_bytes)
    stream = nat.raw_stream(dev)
    rc = L.pp_quad_mfma(codes.data_ptr(), ldc, elem_base, a.data_ptr(), a.stride(0), lut_ptrs, lut_dtype, sc,
                        keep[0].data_ptr() if pn else None, keep[1].data_ptr() if pn else None, pn,
                        row_plug.data_ptr() if row_plug is not None else None, slices, cols,
                        nat.ptr_array([o.data_ptr() for o in outs]), outs[0].stride(0), M, N, K,
                        ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    if rc:
        nat.drop_workspace(wkey)
    nat.check(rc, "pp_quad_mfma")
    del keep, row_plug, ws
    return outs


def quad_dequant(codes, luts, scales, *, plug=None, elem_base=0, dtype=torch.float32):
    """(K,N) weights ``s_k * W_k`` of a code view, plug applied (4 tensors), float32 or
    float16 (``dtype``)."""
    K, N = codes.shape
    dev = _check_device(codes, *luts)
    if dtype not in (torch.float32, torch.float16):
        raise TypeError("dtype must be torch.float32 or torch.float16")
    outs = [torch.empty((K, N), dtype=dtype, device=dev) for _ in range(4)]
    if K * N == 0:
        return outs
    lut_ptrs, lut_dtype = _lut_args(luts)
    pi, pv, pn, keep = _plug_args(plug, dev)
    stream = nat.raw_stream(dev)
    fn = nat.lib().pp_quad_dequant if dtype == torch.float32 else nat.lib().pp_quad_dequant_f16
    rc = fn(codes.data_ptr(), codes.stride(0), codes.stride(1), lut_ptrs, lut_dtype, nat.float_array(scales), pi, pv,
            pn, int(elem_base), nat.ptr_array([o.data_ptr() for o in outs]), N, K, stream)
    nat.check(rc, "pp_quad_dequant")
    del keep
    return outs


def header_luts(r_max, device=None):
    """float32 LUTs of a ``.quadpack`` header (quaternion_packer.py:178-181), computed
    in float64 and rounded once; cos1/sin1 and cos2/sin2 are the same half-turn table.
    Like the reference unpacker, the module constant mu = 255 is used, not the
    header's mu field (quaternion_packer.py:153, 178)."""
    i = torch.arange(256, dtype=torch.float64)
    log_mu = math.log1p(MU)
    half = i / 255 * math.pi
    full = i / 255 * 2 * math.pi
    t = [(torch.exp(i / 255 * log_mu) - 1) * float(r_max) / MU,
         torch.cos(half), torch.sin(half), torch.cos(half), torch.sin(half), torch.cos(full), torch.sin(full)]
    return [x.to(torch.float32).to(device) for x in t]
