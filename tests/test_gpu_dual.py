"""GPU parity of the dual decode against the float64 oracle (same seeded inputs)."""
import numpy as np
import pytest
import torch

import gen
from oracle import dualpack as odp
from oracle import layer as olay
from parity import fp16_ulp_distance, assert_dequant_close, assert_gemv_close, fp16_weight_bound
from polar_pack_amd import polar_kernels as pk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


def kernel_layout_layer(K, N, seed, dtype=torch.float16):
    w1, w2 = [torch.from_numpy(w.reshape(K, N)).to(dtype) for w in gen.correlated_models(seed, [K * N] * 2)]
    return olay.quantize_polar_bitpacked(w1, w2)


def prefill_bound(a, w, route):
    """The matrix-core decodes and the fp16 decode + library GEMM (routes ``dual_mfma``,
    ``dual_nk_mfma`` and ``prefill``) multiply weights rounded to fp16, as the reference's
    kernel rounds them (polar_kernels.py:78-82): held to the fp16-weight bound; the fused row
    kernels to rel 1e-3."""
    return fp16_weight_bound(a, w) if route in ("dual_mfma", "dual_nk_mfma", "prefill") else None


def to_dev(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in arrs]


@pytest.mark.parametrize("K,N", [(64, 96), (33, 40), (256, 512)])
def test_dual_dequant_kernel_layout(K, N):
    packed, bmax, amp_lut, cos_lut, sin_lut = kernel_layout_layer(K, N, K + N)
    got = pk.dual_dequant(*to_dev(packed, bmax, amp_lut, cos_lut, sin_lut))
    ref = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    for g, r in zip(got, ref):
        assert_dequant_close(g.cpu().numpy(), r)


def stream_pack(n1, n2, seed, cap, chunk):
    w1, w2 = gen.correlated_models(seed, [n1, n2], delta_growth=False)
    return odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=cap, chunk_size=chunk))


def be_codes_tensor(dp):
    """File-layout codes (big-endian u16 bytes) as a device int16 tensor of n_pairs elements."""
    return torch.from_numpy(dp.codes_be.view(np.int16).copy()).to(DEV)


@pytest.mark.parametrize("chunk", [1000, 10_001, 50_000_000])
def test_dual_dequant_container_layout_with_plug(chunk):
    dp = stream_pack(30_000, 27_000, 3, 0.03, chunk)
    N, K = 120, 250                                      # 30,000 pairs viewed as a (N,K) Linear
    codes = be_codes_tensor(dp)[:N * K].reshape(N, K).t()
    amp, cs, sn = pk.header_luts(mu=dp.mu, device=DEV)
    got = pk.dual_dequant(codes, torch.from_numpy(dp.scales).to(DEV), amp, cs, sn, layout="u16be",
                          chunk_size=dp.chunk_size,
                          plug=(u32(dp.plug_idx).to(DEV), torch.from_numpy(dp.plug_val).to(DEV)))
    d1, d2 = odp.decode_pairs_f64(dp, 0, N * K)
    for g, r in zip(got, (d1, d2)):
        assert_dequant_close(g.cpu().numpy(), r.reshape(N, K).T)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("K,N", [(256, 512), (64, 96), (2048, 200)])
def test_polar_dual_bitpacked_kernel_layout(K, N, M):
    packed, bmax, amp_lut, cos_lut, sin_lut = kernel_layout_layer(K, N, 11 * K + N)
    a = np.random.default_rng(M).standard_normal((M, K)).astype(np.float16)
    dv = to_dev(a, packed, bmax, amp_lut, cos_lut, sin_lut)
    o1, o2 = pk.polar_dual_bitpacked(*dv)
    route = pk.dual_call_route(dv[1], M)
    W = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    for o, w in ((o1, W[0]), (o2, W[1])):
        assert o.shape == (M, N) and o.dtype == torch.float16
        assert_gemv_close(o.float().cpu().numpy(), olay.gemm_f64(a, w), bound=prefill_bound(a, w, route))


@pytest.mark.parametrize("M", [1, 2, 4, 6])
@pytest.mark.parametrize("chunk", [4096, 10_001, 50_000_000])
def test_polar_dual_bitpacked_container_stream(chunk, M):
    """(N,K) Linears cut from a .dualpack stream, big-endian codes, chunked groups, plug."""
    n1 = 3 * 2048 * 64 + 1000
    dp = stream_pack(n1, n1 - 777, 7, 0.01, chunk)
    amp, cs, sn = pk.header_luts(mu=dp.mu, device=DEV)
    codes_all = be_codes_tensor(dp)
    scales = torch.from_numpy(dp.scales).to(DEV)
    plug = (u32(dp.plug_idx).to(DEV), torch.from_numpy(dp.plug_val).to(DEV))
    rng = np.random.default_rng(M)
    for base, N, K in ((0, 64, 2048), (64 * 2048, 128, 1024), (2 * 64 * 2048, 16, 8192)):
        a = rng.standard_normal((M, K)).astype(np.float16)
        view = codes_all[base:base + N * K].reshape(N, K).t()
        o1, o2 = pk.polar_dual_bitpacked(torch.from_numpy(a).to(DEV), view, scales, amp, cs, sn, layout="u16be",
                                         chunk_size=dp.chunk_size, plug=plug, elem_base=base)
        route = pk.dual_call_route(view, M, layout="u16be", chunk_size=dp.chunk_size, elem_base=base,
                                   plug_n=plug[0].numel())
        d1, d2 = odp.decode_pairs_f64(dp, base, base + N * K)
        for o, d in ((o1, d1), (o2, d2)):
            w = d.reshape(N, K).T
            assert_gemv_close(o.float().cpu().numpy(), olay.gemm_f64(a, w), f"base {base}",
                              bound=prefill_bound(a, w, route))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_quantize_polar_bitpacked_on_gpu_matches_oracle(dtype):
    """The packer computes in the weights' dtype, as the reference does (polar_kernels.py:120-124),
    with torch's GPU rule for Python scalars (kept in float32, division through the
    reciprocal; the oracle's ``gpu_scalars`` mode): codes equal but for rare one-step flips
    where device and host transcendentals round apart."""
    K, N = 128, 64
    w1, w2 = [torch.from_numpy(w.reshape(K, N)).to(dtype) for w in gen.correlated_models(5, [K * N] * 2)]
    got = pk.quantize_polar_bitpacked(w1.to(DEV), w2.to(DEV))
    ref = olay.quantize_polar_bitpacked(w1, w2, gpu_scalars=True)
    p_got = got[0].cpu().numpy().astype(np.int32) + 32768
    p_ref = ref[0].astype(np.int32) + 32768
    dph = np.abs(((p_got & 1023) - (p_ref & 1023) + 512) % 1024 - 512)
    assert (dph > 0).mean() < 0.01 and dph.max() <= 1, ((dph > 0).mean(), dph.max())
    assert np.abs((p_got >> 10) - (p_ref >> 10)).max() <= 1
    db = np.abs(got[1].cpu().numpy().view(np.int16).astype(np.int32) - ref[1].view(np.int16).astype(np.int32))
    assert db.max() <= 1                                 # group max of device sqrt: within one fp16 ulp
    for i in (2, 3, 4):
        np.testing.assert_array_equal(got[i].cpu().numpy().view(np.uint16), ref[i].view(np.uint16))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 8, 11])
@pytest.mark.parametrize("K,N,plug", [(2048, 1000 - 1000 % 8, 0), (2048, 1000 - 1000 % 8, 700), (64, 96, 0),
                                      (520, 4096, 300), (4096, 4096, 0)])
def test_polar_dual_bitpacked_kn_fast_path(K, N, plug, M):
    """Contiguous (K,N) codes, the layout quantize_polar_bitpacked returns: the fused (K,N)
    kernel (512-column items, K slices whose partial sums a finish pass adds, plug entries
    replacing the amplitude; blocks of 4 tokens), against the float64 oracle."""
    seed = K + N + plug + M
    packed, bmax, amp_lut, cos_lut, sin_lut = kernel_layout_layer(K, N, seed)
    rng = np.random.default_rng(seed)
    base = 1000
    flat = np.sort(rng.choice(K * N, plug, replace=False)).astype(np.uint32)
    vals = np.abs(rng.standard_normal(plug) * 0.05).astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float16)
    kw = {}
    if plug:
        kw = dict(plug=(u32(flat + base).to(DEV), torch.from_numpy(vals).to(DEV)), elem_base=base)
    dv = to_dev(a, packed, bmax, amp_lut, cos_lut, sin_lut)
    o1, o2 = pk.polar_dual_bitpacked(*dv, **kw)
    route = pk.dual_call_route(dv[1], M, elem_base=base, plug_n=plug)
    W = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    ph = (packed.astype(np.int32) + 32768) & 1023
    kk, nn = flat // N, flat % N
    for w, lut in ((W[0], cos_lut), (W[1], sin_lut)):
        w[kk, nn] = vals.astype(np.float64) * np.asarray(lut, np.float64)[ph[kk, nn]]
    for o, w in ((o1, W[0]), (o2, W[1])):
        assert_gemv_close(o.float().cpu().numpy(), olay.gemm_f64(a, w), bound=prefill_bound(a, w, route))


def test_polar_dual_bitpacked_kn_output_view():
    """Outputs written through a strided (transposed) view on the direct-store path."""
    K, N, M = 512, 1024, 2
    packed, bmax, amp_lut, cos_lut, sin_lut = kernel_layout_layer(K, N, 77)
    a = np.random.default_rng(1).standard_normal((M, K)).astype(np.float16)
    W = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    from polar_pack_amd import _native as nat
    dev = to_dev(a, packed, bmax, amp_lut, cos_lut, sin_lut)
    o = torch.full((2, N, M), float("nan"), dtype=torch.float16, device=DEV)
    o1, o2 = o[0].t(), o[1].t()                   # (M, N) views with o_sm = 1, o_sn = M
    L = nat.lib()
    x, p, b, al, cl, sl = dev
    ws_bytes = L.pp_dual_gemm_workspace_size(x.data_ptr(), K, 1, p.data_ptr(), N, 1, 32, 0, 0, 0, M, N, K)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    lut_dt = 0 if al.dtype == torch.float16 else 1
    rc = L.pp_dual_gemm(x.data_ptr(), K, 1, p.data_ptr(), 0, N, 1, b.data_ptr(), 32, 0, al.data_ptr(), al.numel(),
                        cl.data_ptr(), sl.data_ptr(), 1024, lut_dt, None, None, 0, 0, o1.data_ptr(), o2.data_ptr(),
                        o1.stride(0), o1.stride(1), M, N, K, ws.data_ptr(), ws_bytes,
                        torch.cuda.current_stream().cuda_stream)
    nat.check(rc, "pp_dual_gemm")
    torch.cuda.synchronize()
    for out, w in ((o1, W[0]), (o2, W[1])):
        assert_gemv_close(out.float().cpu().numpy(), olay.gemm_f64(a, w))


@pytest.mark.parametrize("layout", ["i16", "u16be"])
def test_dual_dequant_f16_is_rounded_f32(layout):
    """The fp16 decode (the large-batch path's weights) is the float32 decode rounded to fp16."""
    K, N = 256, 512
    packed, bmax, amp_lut, cos_lut, sin_lut = kernel_layout_layer(K, N, 9)
    codes = torch.from_numpy(packed).to(DEV)
    if layout == "u16be":
        codes = torch.from_numpy(((packed.view(np.uint16) ^ 0x8000).byteswap()).view(np.int16)).to(DEV)
    args = to_dev(bmax, amp_lut, cos_lut, sin_lut)
    w32 = pk.dual_dequant(codes, *args, layout=layout)
    w16 = pk.dual_dequant(codes, *args, layout=layout, dtype=torch.float16)
    for a32, a16 in zip(w32, w16):
        assert a16.dtype == torch.float16
        # the fp16 store may round the exact product once (a mixed-precision multiply)
        # where the float32 path rounds twice: at most 1 ulp apart, and rarely
        d = fp16_ulp_distance(a16.cpu().numpy(), a32.cpu().numpy())
        assert d.max() <= 1 and (d > 0).mean() < 1e-3


@pytest.mark.parametrize("M", [1, 3])
def test_polar_dual_bitpacked_kn_file_layout(M):
    """Big-endian (file-layout) codes in a contiguous (K,N) tensor with the kernel's group
    rule (chunk_size 0): the (K,N) kernel reads either layout."""
    K, N = 256, 1024
    packed, bmax, amp_lut, cos_lut, sin_lut = kernel_layout_layer(K, N, 21)
    be = ((packed.view(np.uint16) ^ 0x8000).byteswap()).view(np.int16)
    a = np.random.default_rng(M).standard_normal((M, K)).astype(np.float16)
    x, c16, b, al, cl, sl = to_dev(a, be, bmax, amp_lut, cos_lut, sin_lut)
    o1, o2 = pk.polar_dual_bitpacked(x, c16, b, al, cl, sl, layout="u16be")
    W = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    for o, w in ((o1, W[0]), (o2, W[1])):
        assert_gemv_close(o.float().cpu().numpy(), olay.gemm_f64(a, w))
