"""Prefill sizes (128, 333 and 1,024 tokens) through both drop-in operators, with plug
entries, on the default route and with ``fused=True`` (the matrix-core kernels at any size),
against the float64 oracle: the matrix cores held to the fp16 operands they multiply (the
float32 decode rounded once, plug values substituted) with the float32 dot-product bound;
the fp16 decode + library GEMM to the fp16-weight bound; both normwise within 1e-3 of the
exact decode (quad_kernels.py:53-67, 123-134; polar_kernels.py:60-86)."""
import numpy as np
import pytest
import torch

from oracle import dualpack as odp
from oracle import layer as olay
from oracle import quadpack as oqp
from parity import assert_gemv_close, fp16_weight_bound, normwise
from polar_pack_amd import polar_kernels as pk
from polar_pack_amd import quad_kernels as qk
from refs import check_mfma, mfma_reference, route_class
from test_gpu_big import SHAPES, stream_pack as quad_stream_pack
from test_gpu_dual import be_codes_tensor, kernel_layout_layer, prefill_bound, stream_pack as dual_stream_pack
from test_gpu_quad import check_route, fp16_luts, random_codes, u32

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PREFILL_M = [128, 333, 1024]


@pytest.mark.parametrize("fused", [None, True])
@pytest.mark.parametrize("M", PREFILL_M)
def test_quad_container_rows(M, fused):
    """(N,K) rows of a quad stream (~1.5 % of tuples plugged), two projections, the second
    starting mid-stream (plug positions relative to its stream position)."""
    qp, pack = quad_stream_pack()
    pos = 0
    for p, (N, K) in enumerate(SHAPES):
        codes = pack.codes[pos:pos + N * K].reshape(N, K).t()
        route = qk.quad_call_route(codes, M, pack.plug_idx.numel(), fused)
        luts = qk.header_luts(pack.r_max, device=DEV)
        x = np.random.default_rng(10 * M + p).standard_normal((M, K)).astype(np.float16)
        outs = qk.quad_bitpacked(torch.from_numpy(x).to(DEV), codes, luts, list(pack.s),
                                 plug=(pack.plug_idx, pack.plug_vals), elem_base=pos, fused=fused)
        what = f"proj {p} M={M} route={route}"
        if route_class(route) == "mfma":
            check_mfma(outs, mfma_reference(qp, pos, N, K, x), what)
        else:
            assert route_class(route) == "prefill", what
            W = oqp.unpack_quad_f64(qp, pos, pos + N * K)
            for m in range(4):
                w = W[m].reshape(N, K).T
                exact = olay.gemm_f64(x, w)
                got = outs[m].float().cpu().numpy()
                assert_gemv_close(got, exact, f"{what} model {m}", bound=fp16_weight_bound(x, w))
                assert normwise(got, exact) <= 1e-3, what
        pos += N * K


@pytest.mark.parametrize("fused", [None, True])
@pytest.mark.parametrize("M", PREFILL_M)
def test_quad_kn_layer(M, fused):
    """pack_quad_layer's (K,N) codes with a plug table at random positions."""
    K, N = 512, 300
    seed = 4000 + M + (fused is True)
    codes = random_codes((K, N), seed)
    luts, scales = fp16_luts(seed)
    rng = np.random.default_rng(seed)
    flat = rng.choice(K * N, 400, replace=False).astype(np.uint32)
    vals = (rng.standard_normal((400, 4)) * 0.5).astype(np.float16)
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    route = qk.quad_call_route(u32(codes), M, flat.size, fused)
    outs = qk.quad_bitpacked(a.to(DEV), u32(codes).to(DEV), [l.to(DEV) for l in luts], scales, fused=fused,
                             plug=(u32(flat).to(DEV), torch.from_numpy(vals).to(DEV)))
    check_route(outs, a, codes, luts, scales, route_class(route), (flat // N, flat % N), vals,
                f"kn M={M} route={route}")


@pytest.mark.parametrize("fused", [None, True])
@pytest.mark.parametrize("M", PREFILL_M)
def test_dual_kernel_layout(M, fused):
    """quantize_polar_bitpacked's int16 (K,N) codes with plug amplitudes."""
    K, N, plug = 1024, 500, 300
    seed = 5000 + M + (fused is True)
    packed, bmax, amp_lut, cos_lut, sin_lut = kernel_layout_layer(K, N, seed)
    rng = np.random.default_rng(seed)
    flat = rng.choice(K * N, plug, replace=False).astype(np.uint32)
    amps = np.abs(rng.standard_normal(plug) * 0.05).astype(np.float16)
    dv = [torch.from_numpy(np.ascontiguousarray(t)).to(DEV) for t in (packed, bmax, amp_lut, cos_lut, sin_lut)]
    route = pk.dual_call_route(dv[0], M, plug_n=plug, fused=fused)
    a = rng.standard_normal((M, K)).astype(np.float16)
    o1, o2 = pk.polar_dual_bitpacked(torch.from_numpy(a).to(DEV), *dv, fused=fused,
                                     plug=(u32(flat).to(DEV), torch.from_numpy(amps).to(DEV)))
    W = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    ph = (packed.astype(np.int32) + 32768) & 1023
    kk, nn = flat // N, flat % N
    for w, lut in ((W[0], cos_lut), (W[1], sin_lut)):
        w[kk, nn] = amps.astype(np.float64) * np.asarray(lut, np.float64)[ph[kk, nn]]
    for o, w in ((o1, W[0]), (o2, W[1])):
        exact = olay.gemm_f64(a, w)
        got = o.float().cpu().numpy()
        assert_gemv_close(got, exact, f"M={M} route={route}", bound=prefill_bound(a, w, route))
        assert normwise(got, exact) <= 1e-3


@pytest.mark.parametrize("M", PREFILL_M)
def test_dual_container_rows(M):
    """(N,K) rows of a .dualpack stream (big-endian codes, chunked group scales, 2 % of pairs
    in the plug table)."""
    N, K = 96, 512
    dp = dual_stream_pack(N * K + 700, N * K, 13, 0.02, 4096)
    amp, cs, sn = pk.header_luts(mu=dp.mu, device=DEV)
    view = be_codes_tensor(dp)[:N * K].reshape(N, K).t()
    scales = torch.from_numpy(dp.scales).to(DEV)
    plug = (u32(dp.plug_idx).to(DEV), torch.from_numpy(dp.plug_val).to(DEV))
    route = pk.dual_call_route(view, M, layout="u16be", chunk_size=dp.chunk_size, plug_n=dp.plug_idx.size)
    a = np.random.default_rng(M).standard_normal((M, K)).astype(np.float16)
    o1, o2 = pk.polar_dual_bitpacked(torch.from_numpy(a).to(DEV), view, scales, amp, cs, sn, layout="u16be",
                                     chunk_size=dp.chunk_size, plug=plug)
    d1, d2 = odp.decode_pairs_f64(dp, 0, N * K)
    for o, d in ((o1, d1), (o2, d2)):
        w = d.reshape(N, K).T
        exact = olay.gemm_f64(a, w)
        got = o.float().cpu().numpy()
        assert_gemv_close(got, exact, f"M={M} route={route}", bound=prefill_bound(a, w, route))
        assert normwise(got, exact) <= 1e-3
