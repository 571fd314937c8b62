"""Every route of the drop-in operators' routing tables (polar_pack_amd/routes.py) on both
sides of each of its token boundaries, against the float64 oracle, with the plug tables passed
in shuffled order (the operators sort them on the device); duplicate plug positions resolve as
the reference's unpackers resolve them (the last entry wins)."""
import numpy as np
import pytest
import torch

from oracle import dualpack as odp
from oracle import layer as olay
from parity import assert_gemv_close
from polar_pack_amd import polar_kernels as pk
from polar_pack_amd import quad_kernels as qk
from refs import route_class
from test_gpu_dual import be_codes_tensor, kernel_layout_layer, prefill_bound, stream_pack
from test_gpu_quad import check_route, fp16_luts, random_codes, u32

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SCAN = range(1, 300)


def boundary_ms(route_of):
    """1, then M - 1 and M at every token count M where the route changes (up to 299)."""
    ms = {1}
    prev = route_of(1)
    for M in SCAN:
        r = route_of(M)
        if r != prev:
            ms |= {M - 1, M}
        prev = r
    return sorted(ms)


QUAD_CASES = [
    # layout, K, N
    ("nk", 256, 96),       # container rows, K % 32 == 0: rows | mfma | big_nk | prefill
    ("nk", 264, 96),       # K % 32 != 0: rows | prefill
    ("kn", 256, 96),       # pack_quad_layer codes, N <= K
    ("kn", 128, 256),      # N > K
    ("kn", 264, 96),       # K % 32 != 0
]


@pytest.mark.parametrize("fused", [None, True, False])
@pytest.mark.parametrize("plug", [0, 160])
@pytest.mark.parametrize("layout,K,N", QUAD_CASES)
def test_quad_route_boundaries(layout, K, N, plug, fused):
    seed = K * 3 + N + plug + (0 if fused is None else 1 + int(fused))
    codes = random_codes((K, N), seed)
    luts, scales = fp16_luts(seed)
    L = [l.to(DEV) for l in luts]
    rng = np.random.default_rng(seed)
    flat = rng.choice(K * N, plug, replace=False).astype(np.uint32)      # shuffled: not ascending
    vals = (rng.standard_normal((plug, 4)) * 0.5).astype(np.float16)
    if layout == "kn":
        view = u32(codes).to(DEV)
        at = (flat // N, flat % N)
    else:
        view = u32(np.ascontiguousarray(codes.T)).to(DEV).t()
        at = (flat % K, flat // K)                                       # storage offset n*K + k
    kw = {}
    if plug:
        kw = dict(plug=(u32(flat).to(DEV), torch.from_numpy(vals).to(DEV)))
    for M in boundary_ms(lambda m: qk.quad_call_route(view, m, plug, fused)):
        route = qk.quad_call_route(view, M, plug, fused)
        a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
        outs = qk.quad_bitpacked(a.to(DEV), view, L, scales, fused=fused, **kw)
        check_route(outs, a, codes, luts, scales, route_class(route), at if plug else None, vals if plug else None,
                    f"{layout} {K}x{N} plug={plug} fused={fused} M={M} route={route}")


def test_quad_duplicate_plug_positions_last_wins():
    """A plug table with repeated positions: every route applies the last entry of each
    position (numpy's fancy-indexed store in the reference's unpacker keeps the last)."""
    K, N = 256, 96
    codes = random_codes((K, N), 5)
    luts, scales = fp16_luts(5)
    L = [l.to(DEV) for l in luts]
    rng = np.random.default_rng(5)
    base = rng.choice(K * N, 60, replace=False).astype(np.uint32)
    flat = np.concatenate([base, base[:25], base[:10]])               # 25 positions twice, 10 three times
    vals = (rng.standard_normal((flat.size, 4)) * 0.5).astype(np.float16)
    last = {}
    for i, p in enumerate(flat):
        last[int(p)] = i
    keep = np.array(sorted(last.values()))
    for layout in ("nk", "kn"):
        if layout == "kn":
            view = u32(codes).to(DEV)
            at = (flat[keep] // N, flat[keep] % N)
        else:
            view = u32(np.ascontiguousarray(codes.T)).to(DEV).t()
            at = (flat[keep] % K, flat[keep] // K)
        for M in (1, 8, 40, 100, 200):
            route = qk.quad_call_route(view, M, flat.size)
            a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
            outs = qk.quad_bitpacked(a.to(DEV), view, L, scales,
                                     plug=(u32(flat).to(DEV), torch.from_numpy(vals).to(DEV)))
            check_route(outs, a, codes, luts, scales, route_class(route), at, vals[keep],
                        f"{layout} M={M} route={route}")


DUAL_KN_CASES = [(256, 96), (128, 256), (264, 96)]


@pytest.mark.parametrize("fused", [None, True, False])
@pytest.mark.parametrize("plug", [0, 120])
@pytest.mark.parametrize("K,N", DUAL_KN_CASES)
def test_dual_kn_route_boundaries(K, N, plug, fused):
    seed = 11 * K + N + plug + (0 if fused is None else 1 + int(fused))
    packed, bmax, amp_lut, cos_lut, sin_lut = kernel_layout_layer(K, N, seed)
    rng = np.random.default_rng(seed)
    flat = rng.choice(K * N, plug, replace=False).astype(np.uint32)
    amps = np.abs(rng.standard_normal(plug) * 0.05).astype(np.float16)
    dv = [torch.from_numpy(np.ascontiguousarray(t)).to(DEV) for t in (packed, bmax, amp_lut, cos_lut, sin_lut)]
    W = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    if plug:
        ph = (packed.astype(np.int32) + 32768) & 1023
        kk, nn = flat // N, flat % N
        for w, lut in ((W[0], cos_lut), (W[1], sin_lut)):
            w[kk, nn] = amps.astype(np.float64) * np.asarray(lut, np.float64)[ph[kk, nn]]
    kw = dict(plug=(u32(flat).to(DEV), torch.from_numpy(amps).to(DEV))) if plug else {}
    for M in boundary_ms(lambda m: pk.dual_call_route(dv[0], m, plug_n=plug, fused=fused)):
        route = pk.dual_call_route(dv[0], M, plug_n=plug, fused=fused)
        a = rng.standard_normal((M, K)).astype(np.float16)
        o1, o2 = pk.polar_dual_bitpacked(torch.from_numpy(a).to(DEV), *dv, fused=fused, **kw)
        for o, w in ((o1, W[0]), (o2, W[1])):
            assert_gemv_close(o.float().cpu().numpy(), olay.gemm_f64(a, w), f"M={M} route={route}",
                              bound=prefill_bound(a, w, route))


@pytest.mark.parametrize("plug_shuffled", [False, True])
def test_dual_container_route_boundaries(plug_shuffled):
    """(N,K) rows of a .dualpack stream (big-endian codes, chunked groups): the fused row
    kernel to 4 tokens, then the fp16 decode + GEMM; plug table as stored or shuffled."""
    N, K = 64, 512
    dp = stream_pack(N * K + 500, N * K, 9, 0.02, 4096)
    amp, cs, sn = pk.header_luts(mu=dp.mu, device=DEV)
    view = be_codes_tensor(dp)[:N * K].reshape(N, K).t()
    scales = torch.from_numpy(dp.scales).to(DEV)
    order = np.random.default_rng(1).permutation(dp.plug_idx.size) if plug_shuffled else np.arange(dp.plug_idx.size)
    plug = (u32(dp.plug_idx[order]).to(DEV), torch.from_numpy(dp.plug_val[order]).to(DEV))
    d1, d2 = odp.decode_pairs_f64(dp, 0, N * K)
    rng = np.random.default_rng(2)
    route_of = lambda m: pk.dual_call_route(view, m, layout="u16be", chunk_size=dp.chunk_size,
                                            plug_n=dp.plug_idx.size)
    for M in boundary_ms(route_of):
        route = route_of(M)
        a = rng.standard_normal((M, K)).astype(np.float16)
        o1, o2 = pk.polar_dual_bitpacked(torch.from_numpy(a).to(DEV), view, scales, amp, cs, sn, layout="u16be",
                                         chunk_size=dp.chunk_size, plug=plug)
        for o, d in ((o1, d1), (o2, d2)):
            w = d.reshape(N, K).T
            assert_gemv_close(o.float().cpu().numpy(), olay.gemm_f64(a, w), f"M={M} route={route}",
                              bound=prefill_bound(a, w, route))
