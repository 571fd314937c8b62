"""GPU parity of the matrix-core batch decode (pp_quad_mfma) against the float64 oracle."""
import functools

import numpy as np
import pytest
import torch

import gen
from oracle import layer as olay
from oracle import quadpack as oqp
from parity import assert_gemv_close, fp16_weight_bound, normwise
from polar_pack_amd import quad_kernels as qk
from refs import route_class
from polar_pack_amd.container import QuadPackFile
from polar_pack_amd.stream import QuadBatch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@functools.lru_cache(maxsize=None)
def _packed(shapes, seed, threshold):
    n = sum(a * b for a, b in shapes)
    qp = oqp.pack_quad(gen.correlated_models(seed, [n] * 4), threshold=threshold)
    dev = QuadPackFile(n=qp.n, s=qp.s, r_max=qp.r_max, codes=qp.codes, plug_idx=qp.plug_idx,
                       plug_vals=qp.plug_vals).to_device(DEV)
    return qp, dev


def packed(shapes, seed, threshold):
    return _packed(tuple(shapes), seed, threshold)


def oracle(qp, pos0, N, K, x):
    """float64 GEMM of the float64 decode (``exact``), and of the fp16 operands the
    matrix-core path feeds to the dot product, as the reference's tl.dot does
    (quad_kernels.py:116-126): the decode evaluated in float32 on the header LUTs
    (oracle.layer.quad_dequant, float32 mode), plug tuples substituted, each normalised
    weight rounded once to fp16 (``w16``), with the float32 dot-product bound."""
    W = oqp.unpack_quad_f64(qp, pos0, pos0 + N * K)
    luts = [l.numpy() for l in qk.header_luts(qp.r_max)]
    wn = olay.quad_dequant(qp.codes[pos0:pos0 + N * K].reshape(1, -1), luts, dtype=np.float32)
    lo, hi = np.searchsorted(qp.plug_idx, [pos0, pos0 + N * K])
    at = qp.plug_idx[lo:hi].astype(np.int64) - pos0
    exact, w16, bound = [], [], []
    xd = x.astype(np.float64)
    for m in range(4):
        s = float(np.float32(qp.s[m]))
        h = wn[m][0].astype(np.float16)
        h[at] = qp.plug_vals[lo:hi, m]
        wh = h.astype(np.float64).reshape(N, K) * s
        exact.append(xd @ W[m].reshape(N, K).T)
        w16.append(xd @ wh.T)
        bound.append(2.0 ** -18 * (np.abs(xd) @ np.abs(wh).T))
    return exact, w16, bound


def check(got, ref, what):
    exact, w16, bound = ref
    for m in range(4):
        g = got[m].float().cpu().numpy()
        assert_gemv_close(g, w16[m], f"{what} model {m}", bound=bound[m])
        assert normwise(g, exact[m]) <= 1e-3, f"{what} model {m}: normwise {normwise(g, exact[m]):.2e}"


# two projections in one stream: the second starts mid-stream (plug positions relative)
SHAPES = [(48, 2048), (100, 1024)]


@pytest.mark.parametrize("M", [1, 9, 16, 17, 33, 64])
@pytest.mark.parametrize("slices", [None, 1, 3])
def test_batch_decode_matches_oracle(M, slices):
    qp, pack = packed(SHAPES, 31, threshold=0.015)   # ~1.5% of tuples plugged
    assert qp.plug_idx.size > 100
    pos = 0
    for p, (N, K) in enumerate(SHAPES):
        qb = QuadBatch(pack, N, K, pos0=pos, M=M, slices=slices)
        x, outs = qb.make_buffers()
        x_np = np.random.default_rng(40 + p).standard_normal((M, K)).astype(np.float16)
        x.copy_(torch.from_numpy(x_np))
        for o in outs:
            o.fill_(float("nan"))
        qb.bind(x, outs)
        ref = oracle(qp, pos, N, K, x_np)
        for rep in range(2):
            qb()
            torch.cuda.synchronize()
            check(outs, ref, f"proj {p} rep {rep}")
            if qb.workspace is not None:
                assert int(torch.count_nonzero(qb.workspace)) == 0
        pos += N * K


def test_dense_plug_rows_refill_the_window():
    """Rows with many entries in one 32-column step (window refills inside a step)."""
    qp, pack = packed([(32, 512)], 33, threshold=0.0005)      # every tuple plugged
    counts = np.bincount(qp.plug_idx.astype(np.int64) // 32, minlength=32 * 512 // 32)
    assert counts.max() > 4
    qb = QuadBatch(pack, 32, 512, M=16, slices=1)
    x, outs = qb.make_buffers()
    x_np = np.random.default_rng(2).standard_normal((16, 512)).astype(np.float16)
    x.copy_(torch.from_numpy(x_np))
    qb.bind(x, outs)
    qb()
    torch.cuda.synchronize()
    check(outs, oracle(qp, 0, 32, 512, x_np), "dense")


@pytest.mark.parametrize("M", [12, 64, 100, 130, 300])
def test_drop_in_operator_takes_the_matrix_cores_for_large_batches(M):
    """9..64 tokens in one launch of the batch decode, 65..128 on the fused large-batch
    kernel (both multiply the fp16-rounded decode on the matrix cores); more (the
    reference's prefill sizes) as an fp16 decode of the (N,K) storage and a library GEMM."""
    qp, pack = packed(SHAPES, 35, threshold=0.015)
    N, K = SHAPES[1]
    pos = SHAPES[0][0] * SHAPES[0][1]
    codes = pack.codes[pos:pos + N * K].reshape(N, K).t()        # the reference's (K, N) view
    luts = qk.header_luts(pack.r_max, device=DEV)
    x_np = np.random.default_rng(9).standard_normal((M, K)).astype(np.float16)
    outs = qk.quad_bitpacked(torch.from_numpy(x_np).to(DEV), codes, luts, list(pack.s),
                             plug=(pack.plug_idx, pack.plug_vals), elem_base=pos)
    for m in range(4):
        assert outs[m].shape == (M, N) and outs[m].dtype == torch.float16
    if route_class(qk.quad_call_route(codes, M, pack.plug_idx.numel())) == "mfma":
        check(outs, oracle(qp, pos, N, K, x_np), "drop-in")
        return
    # above: fp16 decode (s_m folded in) + library GEMM, held to the fp16-weight bound
    W = oqp.unpack_quad_f64(qp, pos, pos + N * K)
    for m in range(4):
        w = W[m].reshape(N, K).T
        got = outs[m].float().cpu().numpy()
        assert_gemv_close(got, x_np.astype(np.float64) @ w, f"prefill model {m}", bound=fp16_weight_bound(x_np, w))
        assert normwise(got, x_np.astype(np.float64) @ w) <= 1e-3
