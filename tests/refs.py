"""Oracle references shared by the GPU parity tests (test infrastructure).

* :func:`quad_rows_pack` -- an oracle ``QuadPack`` over chosen rows of one projection of
  a device-resident quad stream (codes and plug entries gathered from the device), so the
  float64 container decode (``oracle.quadpack.unpack_quad_f64``) runs on a row sample of
  a multi-GB stream;
* :func:`quad_rows_ref` -- float64 outputs of those rows;
* :func:`mfma_reference` / :func:`check_mfma` -- the reference of the matrix-core route:
  weights decoded in float32 on the header LUTs and rounded once to fp16 operands (as the
  reference's ``tl.dot`` takes them, quad_kernels.py:116-126), the float32 dot-product
  bound, and a normwise check against the exact decode; :func:`kn_mfma_reference` the same
  for a (K,N) code array with any LUTs;
* :func:`dual_pack_host` / :func:`dual_rows_ref` -- the same for a dual stream, tails
  included.
"""
import numpy as np
import torch

from oracle import dualpack as odp
from oracle import layer as olay
from oracle import quadpack as oqp
from parity import assert_gemv_close, normwise
from polar_pack_amd import quad_kernels as qk


def _u32(t):
    return t.view(torch.int32).cpu().numpy().view(np.uint32)


def quad_rows_pack(pack, plug_host, pos0, K, rows):
    """Oracle QuadPack whose codes are the given rows (each K tuples, all below ``pack.n``)
    of the projection at stream position ``pos0``, concatenated, with their plug entries
    moved to the concatenated positions."""
    rows = np.asarray(rows, np.int64)
    starts = int(pos0) + rows * int(K)
    assert np.all(starts + K <= pack.n)
    idx = (starts[:, None] + np.arange(K, dtype=np.int64)[None, :]).reshape(-1)
    dev = pack.codes.device
    codes = _u32(pack.codes.view(torch.int32)[torch.from_numpy(idx).to(dev)])
    lo = np.searchsorted(plug_host, starts, side="left")
    hi = np.searchsorted(plug_host, starts + K, side="left")
    sel = np.concatenate([np.arange(a, b, dtype=np.int64) for a, b in zip(lo, hi)] + [np.zeros(0, np.int64)])
    new = np.concatenate([plug_host[a:b].astype(np.int64) - starts[i] + i * int(K)
                          for i, (a, b) in enumerate(zip(lo, hi))] + [np.zeros(0, np.int64)])
    vals = pack.plug_vals[torch.from_numpy(sel).to(dev)].cpu().numpy() if sel.size else np.zeros((0, 4), np.float16)
    return oqp.QuadPack(n=int(idx.size), s=tuple(pack.s), r_max=float(pack.r_max), codes=codes,
                        plug_idx=new.astype(np.uint32), plug_vals=vals), int(sel.size)


def quad_rows_ref(pack, plug_host, pos0, K, rows, x):
    """float64 outputs (4 arrays (M, len(rows))) of the given rows for activations x (M, K),
    and the number of plug entries in those rows."""
    qp, n_plug = quad_rows_pack(pack, plug_host, pos0, K, rows)
    W = oqp.unpack_quad_f64(qp)
    xd = np.asarray(x, np.float64)
    return [xd @ W[m].reshape(len(rows), K).T for m in range(4)], n_plug


def mfma_reference(qp, pos0, N, K, x):
    """float64 GEMM of the exact decode, of the fp16 operands the matrix-core route feeds
    to its dot products (float32 decode on the header LUTs, plug tuples substituted, each
    normalised weight rounded once to fp16), and the float32 dot-product bound."""
    W = oqp.unpack_quad_f64(qp, pos0, pos0 + N * K)
    luts = [l.numpy() for l in qk.header_luts(qp.r_max)]
    wn = olay.quad_dequant(qp.codes[pos0:pos0 + N * K].reshape(1, -1), luts, dtype=np.float32)
    lo, hi = np.searchsorted(qp.plug_idx, [pos0, pos0 + N * K])
    at = qp.plug_idx[lo:hi].astype(np.int64) - pos0
    exact, w16, bound = [], [], []
    xd = np.asarray(x, np.float64)
    for m in range(4):
        s = float(np.float32(qp.s[m]))
        h = wn[m][0].astype(np.float16)
        h[at] = qp.plug_vals[lo:hi, m]
        wh = h.astype(np.float64).reshape(N, K) * s
        exact.append(xd @ W[m].reshape(N, K).T)
        w16.append(xd @ wh.T)
        bound.append(2.0 ** -18 * (np.abs(xd) @ np.abs(wh).T))
    return exact, w16, bound


def kn_mfma_reference(a, codes_kn, luts, scales, plug_at=None, plug_vals=None, cols=None):
    """The matrix-core reference for codes given as a (K,N) array with arbitrary 7-table
    LUTs: float64 products of the exact decode and of the fp16 operands (float32 decode
    on the LUTs rounded once, plug tuples substituted at (k, n) = plug_at), with the
    float32 dot-product bound; only output columns ``cols`` when given (row sample)."""
    codes = np.asarray(codes_kn, np.uint32)
    if cols is not None:
        cols = np.asarray(cols, np.int64)
        codes = codes[:, cols]
        if plug_at is not None:
            pos = {int(n): i for i, n in enumerate(cols)}
            keep = np.array([int(n) in pos for n in plug_at[1]], bool)
            plug_at = (plug_at[0][keep], np.array([pos[int(n)] for n in plug_at[1][keep]], np.int64))
            plug_vals = plug_vals[keep]
    lf = [l.float().cpu().numpy() if torch.is_tensor(l) else np.asarray(l, np.float32) for l in luts]
    W = olay.quad_dequant(codes, lf, scales)
    W32 = olay.quad_dequant(codes, lf, dtype=np.float32)
    ad = np.asarray(a, np.float64)
    exact, w16, bound = [], [], []
    for m in range(4):
        h = W32[m].astype(np.float16)
        we = W[m].copy()
        if plug_at is not None:
            h[plug_at] = plug_vals[:, m]
            we[plug_at] = plug_vals[:, m].astype(np.float64) * scales[m]
        w = h.astype(np.float64) * float(np.float32(scales[m]))
        exact.append(ad @ we)
        w16.append(ad @ w)
        bound.append(2.0 ** -18 * (np.abs(ad) @ np.abs(w)))
    return exact, w16, bound


def check_mfma(got, ref, what):
    """Matrix-core outputs: within rel 1e-3 (+ the float32 dot-product bound) of the fp16
    operand product, and normwise within 1e-3 of the exact float64 decode."""
    exact, w16, bound = ref
    for m in range(4):
        g = got[m].float().cpu().numpy() if torch.is_tensor(got[m]) else np.asarray(got[m])
        assert_gemv_close(g, w16[m], f"{what} model {m}", bound=bound[m])
        assert normwise(g, exact[m]) <= 1e-3, f"{what} model {m}: normwise {normwise(g, exact[m]):.2e}"


def quad_pack_host(pack):
    """Oracle QuadPack of a whole device pack (host copy of every array)."""
    return oqp.QuadPack(n=pack.n, s=tuple(pack.s), r_max=float(pack.r_max), codes=_u32(pack.codes),
                        plug_idx=pack.plug_host().copy(), plug_vals=pack.plug_vals.cpu().numpy(),
                        tails=[t.cpu().numpy() for t in pack.tails])


def dual_pack_host(pack):
    """Oracle DualPack of a device dual pack (either code layout; host copies)."""
    raw = pack.codes.cpu().numpy().view(np.uint16)
    be = raw if pack.layout == "u16be" else (raw ^ np.uint16(0x8000)).byteswap()
    return odp.DualPack(n_pairs=pack.n_codes, n1=pack.n1, n2=pack.n2, codes_be=be.view(np.uint8),
                        scales=pack.scales.cpu().numpy(), plug_idx=pack.plug_host().copy(),
                        plug_val=pack.plug_val.cpu().numpy(), amp_bits=pack.amp_bits, phase_bits=pack.phase_bits,
                        mu=pack.mu, group_size=pack.group_size, chunk_size=pack.chunk_size)


def dual_weights_f64(dp, tails, lo, hi):
    """float64 (w1, w2) at stream positions [lo, hi): the oracle decode below ``n_pairs``,
    each model's fp16 tail after it, 0 where a model has no weight."""
    out = [np.zeros(hi - lo), np.zeros(hi - lo)]
    n = dp.n_pairs
    if lo < n:
        w = odp.decode_pairs_f64(dp, lo, min(hi, n))
        for m in range(2):
            out[m][:min(hi, n) - lo] = w[m]
    for m in range(2):
        t = tails[m] if m < len(tails) else np.zeros(0, np.float16)
        a, b = max(lo, n), min(hi, n + t.size)
        if b > a:
            out[m][a - lo:b - lo] = t[a - n:b - n].astype(np.float64)
    return out


def dual_rows_ref(dp, tails, pos0, K, rows, x):
    """float64 outputs (2 arrays (M, len(rows))) of the given rows of the projection at
    ``pos0``."""
    xd = np.asarray(x, np.float64)
    res = [np.zeros((xd.shape[0], len(rows))), np.zeros((xd.shape[0], len(rows)))]
    for i, r in enumerate(rows):
        lo = int(pos0) + int(r) * int(K)
        w = dual_weights_f64(dp, tails, lo, lo + int(K))
        for m in range(2):
            res[m][:, i] = xd @ w[m]
    return res


def route_class(route):
    """How a route's products are held to the oracle: ``fused`` (the row kernels and the
    generic decode: float32 decode, rel 1e-3 against the exact products), ``mfma`` (the matrix
    cores: fp16 operands, the float32 dot-product bound), ``prefill`` (fp16 decode + library
    GEMM: the fp16-weight bound)."""
    if route in ("rows", "kn", "generic", "dual_kn", "dual_rows"):
        return "fused"
    if route in ("mfma", "big_nk", "big_kn", "kn_mfma", "dual_mfma", "dual_nk_mfma"):
        return "mfma"
    assert route == "prefill", route
    return "prefill"
