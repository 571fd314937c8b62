"""GPU parity of the transposing fp16 decodes (pp_quad_dequant_f16_t, pp_dual_dequant_f16_t:
(K,N) codes -> weights (N,K) for the prefill GEMM) against the (K,N) decodes they transpose,
bit for bit, with plug entries, partial 64 x 64 tiles, a row stride wider than N and more
tiles than the grid has workgroups; and the
drop-in operators' prefill routes against the float64 oracle."""
import numpy as np
import pytest
import torch

import gen
from oracle import layer as olay
from parity import assert_gemv_close, fp16_weight_bound, normwise
from polar_pack_amd import _native as nat
from polar_pack_amd import polar_kernels as pk
from polar_pack_amd import quad_kernels as qk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


@pytest.mark.parametrize("K,N,ldk,plug", [(64, 64, 64, 0), (200, 136, 136, 50), (512, 384, 400, 300),
                                          (1000, 72, 80, 20)])
def test_quad_transposed_decode_is_the_transpose(K, N, ldk, plug):
    rng = np.random.default_rng(K + N + plug)
    wide = rng.integers(0, 2 ** 32, size=(K, ldk), dtype=np.uint64).astype(np.uint32)
    ws = [torch.from_numpy(w.reshape(64, 64)).to(torch.float16) for w in gen.correlated_models(K, [4096] * 4)]
    _, luts, scales = olay.pack_quad_layer(*ws)
    luts = [torch.from_numpy(l).to(DEV) for l in luts]
    codes = u32(wide).to(DEV)[:, :N]
    base = 5
    pos = np.sort(rng.choice(K * ldk, plug, replace=False)) if plug else np.zeros(0, np.int64)
    vals = (rng.standard_normal((plug, 4)) * 0.5).astype(np.float16)
    pidx = u32((pos + base).astype(np.uint32)).to(DEV)
    pval = torch.from_numpy(vals).to(DEV)
    L = nat.lib()
    lut_ptrs, lut_dtype = qk._lut_args(luts)
    sc = nat.float_array(scales)
    st = torch.cuda.current_stream(DEV).cuda_stream
    ref = torch.full((4, K, N), float("nan"), dtype=torch.float16, device=DEV)
    got = torch.full((4, N, K), float("nan"), dtype=torch.float16, device=DEV)
    pp = (pidx.data_ptr(), pval.data_ptr(), plug) if plug else (None, None, 0)
    nat.check(L.pp_quad_dequant_f16(codes.data_ptr(), ldk, 1, lut_ptrs, lut_dtype, sc, *pp, base,
                                    nat.ptr_array([ref[m].data_ptr() for m in range(4)]), N, K, st), "ref")
    nat.check(L.pp_quad_dequant_f16_t(codes.data_ptr(), ldk, lut_ptrs, lut_dtype, sc, *pp, base,
                                      nat.ptr_array([got[m].data_ptr() for m in range(4)]), N, K, st), "t")
    torch.cuda.synchronize()
    for m in range(4):
        assert torch.equal(got[m].view(torch.int16), ref[m].t().contiguous().view(torch.int16)), f"model {m}"


@pytest.mark.parametrize("K,N,ldk,plug,gs", [(64, 64, 64, 0, 32), (200, 136, 136, 60, 8), (512, 384, 400, 300, 64),
                                             (96, 1000, 1000, 40, 32)])
def test_dual_transposed_decode_is_the_transpose(K, N, ldk, plug, gs):
    rng = np.random.default_rng(K * 3 + N + plug)
    w1, w2 = (torch.from_numpy(w.reshape(K, N)).to(torch.float16) for w in gen.correlated_models(K + N, [K * N] * 2))
    packed, bmax, amp_lut, cos_lut, sin_lut = olay.quantize_polar_bitpacked(w1, w2, group_size=gs)
    wide = np.zeros((K, ldk), np.int16)
    wide[:, :N] = packed
    wide[:, N:] = rng.integers(-2 ** 15, 2 ** 15, size=(K, ldk - N)).astype(np.int16)
    codes = torch.from_numpy(wide).to(DEV)[:, :N]
    pos = (np.sort(rng.choice(K * N, plug, replace=False)) if plug else np.zeros(0, np.int64))
    pos = (pos // N) * ldk + pos % N
    amps = np.abs(rng.standard_normal(plug) * 0.05).astype(np.float16)
    pidx = u32(pos.astype(np.uint32)).to(DEV)
    pamp = torch.from_numpy(amps).to(DEV)
    L = nat.lib()
    dl = [torch.from_numpy(np.asarray(x)).to(DEV) for x in (bmax, amp_lut, cos_lut, sin_lut)]
    st = torch.cuda.current_stream(DEV).cuda_stream
    ref = torch.full((2, K, N), float("nan"), dtype=torch.float16, device=DEV)
    got = torch.full((2, N, K), float("nan"), dtype=torch.float16, device=DEV)
    pp = (pidx.data_ptr(), pamp.data_ptr(), plug) if plug else (None, None, 0)
    nat.check(L.pp_dual_dequant_f16(codes.data_ptr(), nat.PP_DUAL_I16_OFFSET, ldk, 1, dl[0].data_ptr(), gs, 0,
                                    dl[1].data_ptr(), dl[1].numel(), dl[2].data_ptr(), dl[3].data_ptr(), 1024,
                                    nat.PP_F16, *pp, 0, ref[0].data_ptr(), ref[1].data_ptr(), N, K, st), "ref")
    nat.check(L.pp_dual_dequant_f16_t(codes.data_ptr(), nat.PP_DUAL_I16_OFFSET, ldk, dl[0].data_ptr(), gs,
                                      dl[1].data_ptr(), dl[1].numel(), dl[2].data_ptr(), dl[3].data_ptr(), 1024,
                                      nat.PP_F16, *pp, 0, got[0].data_ptr(), got[1].data_ptr(), N, K, st), "t")
    torch.cuda.synchronize()
    for m in range(2):
        assert torch.equal(got[m].view(torch.int16), ref[m].t().contiguous().view(torch.int16)), f"model {m}"


@pytest.mark.parametrize("K,N,ldk", [(4096, 4096, 4096), (4104, 2056, 2064)])
def test_transposed_decode_many_tiles_per_workgroup(K, N, ldk):
    """Thousands of 64 x 64 tiles, more than the grid's workgroups: each workgroup walks
    several, loading the next tile's codes while it stores the current one."""
    rng = np.random.default_rng(K + N)
    L = nat.lib()
    st = torch.cuda.current_stream(DEV).cuda_stream
    # quad: any uint32 word is a code
    ws = [torch.from_numpy(w.reshape(64, 64)).to(torch.float16) for w in gen.correlated_models(7, [4096] * 4)]
    _, luts, scales = olay.pack_quad_layer(*ws)
    luts = [torch.from_numpy(l).to(DEV) for l in luts]
    lut_ptrs, lut_dtype = qk._lut_args(luts)
    codes = torch.randint(-2 ** 31, 2 ** 31, (K, ldk), dtype=torch.int64, device=DEV).to(torch.int32)[:, :N]
    ref = torch.full((4, K, N), float("nan"), dtype=torch.float16, device=DEV)
    got = torch.full((4, N, K), float("nan"), dtype=torch.float16, device=DEV)
    sc = nat.float_array(scales)
    nat.check(L.pp_quad_dequant_f16(codes.data_ptr(), ldk, 1, lut_ptrs, lut_dtype, sc, None, None, 0, 0,
                                    nat.ptr_array([ref[m].data_ptr() for m in range(4)]), N, K, st), "quad ref")
    nat.check(L.pp_quad_dequant_f16_t(codes.data_ptr(), ldk, lut_ptrs, lut_dtype, sc, None, None, 0, 0,
                                      nat.ptr_array([got[m].data_ptr() for m in range(4)]), N, K, st), "quad t")
    torch.cuda.synchronize()
    for m in range(4):
        assert torch.equal(got[m].view(torch.int16), ref[m].t().contiguous().view(torch.int16)), f"quad model {m}"
    del ref, got, codes
    # dual: a quantized 256 x 256 block tiled over the layer (valid amplitude indices),
    # random positive group scales
    gs = 32
    w1, w2 = (torch.from_numpy(w.reshape(256, 256)).to(torch.float16) for w in gen.correlated_models(11, [65536] * 2))
    packed, _, amp_lut, cos_lut, sin_lut = olay.quantize_polar_bitpacked(w1, w2, group_size=gs)
    wide = np.tile(np.asarray(packed), (K // 256 + 1, ldk // 256 + 1))[:K, :ldk]
    codes = torch.from_numpy(np.ascontiguousarray(wide)).to(DEV)[:, :N]
    bmax = (np.abs(rng.standard_normal(K * N // gs)) * 0.05 + 0.01).astype(np.float16)
    dl = [torch.from_numpy(np.asarray(x)).to(DEV) for x in (bmax, amp_lut, cos_lut, sin_lut)]
    ref = torch.full((2, K, N), float("nan"), dtype=torch.float16, device=DEV)
    got = torch.full((2, N, K), float("nan"), dtype=torch.float16, device=DEV)
    nat.check(L.pp_dual_dequant_f16(codes.data_ptr(), nat.PP_DUAL_I16_OFFSET, ldk, 1, dl[0].data_ptr(), gs, 0,
                                    dl[1].data_ptr(), dl[1].numel(), dl[2].data_ptr(), dl[3].data_ptr(), 1024,
                                    nat.PP_F16, None, None, 0, 0, ref[0].data_ptr(), ref[1].data_ptr(), N, K, st),
              "dual ref")
    nat.check(L.pp_dual_dequant_f16_t(codes.data_ptr(), nat.PP_DUAL_I16_OFFSET, ldk, dl[0].data_ptr(), gs,
                                      dl[1].data_ptr(), dl[1].numel(), dl[2].data_ptr(), dl[3].data_ptr(), 1024,
                                      nat.PP_F16, None, None, 0, 0, got[0].data_ptr(), got[1].data_ptr(), N, K, st),
              "dual t")
    torch.cuda.synchronize()
    for m in range(2):
        assert torch.equal(got[m].view(torch.int16), ref[m].t().contiguous().view(torch.int16)), f"dual model {m}"


def test_transposed_decode_rejects_bad_shapes():
    L = nat.lib()
    buf = torch.zeros(64 * 64, dtype=torch.int32, device=DEV)
    outs = [torch.zeros(64 * 64, dtype=torch.float16, device=DEV) for _ in range(4)]
    luts = qk.header_luts(1.0, device=DEV)
    lut_ptrs, lut_dtype = qk._lut_args(luts)
    rc = L.pp_quad_dequant_f16_t(buf.data_ptr(), 60, lut_ptrs, lut_dtype, nat.float_array([1, 1, 1, 1]), None, None,
                                 0, 0, nat.ptr_array([o.data_ptr() for o in outs]), 60, 64, None)
    assert rc != 0 and "N % 8" in L.pp_last_error().decode()


@pytest.mark.parametrize("M", [129, 300])
def test_prefill_routes_through_transposed_weights(M):
    """Above the fused sizes the operators decode (K,N) codes into (N,K) fp16 weights and run
    one batched GEMM: the fp16-weight bound and normwise 1e-3 against the exact decode."""
    K, N = 512, 256
    rng = np.random.default_rng(M)
    ws = [torch.from_numpy(w.reshape(K, N)).to(torch.float16) for w in gen.correlated_models(M, [K * N] * 4)]
    a = rng.standard_normal((M, K)).astype(np.float16)
    codes, luts, scales = olay.pack_quad_layer(*ws)
    outs = qk.quad_bitpacked(torch.from_numpy(a).to(DEV), u32(codes).to(DEV),
                             [torch.from_numpy(l).to(DEV) for l in luts], scales, fused=False)
    W = olay.quad_dequant(codes, [np.asarray(l, np.float32) for l in luts], scales)
    for m in range(4):
        exact = olay.gemm_f64(a, W[m])
        got = outs[m].float().cpu().numpy()
        assert_gemv_close(got, exact, f"quad model {m}", bound=fp16_weight_bound(a, W[m]))
        assert normwise(got, exact) <= 1e-3
    packed, bmax, amp_lut, cos_lut, sin_lut = olay.quantize_polar_bitpacked(ws[0], ws[1])
    o1, o2 = pk.polar_dual_bitpacked(*[torch.from_numpy(np.asarray(x)).to(DEV)
                                       for x in (a, packed, bmax, amp_lut, cos_lut, sin_lut)])
    Wd = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    for o, w, m in ((o1, Wd[0], 0), (o2, Wd[1], 1)):
        exact = olay.gemm_f64(a, w)
        got = o.float().cpu().numpy()
        assert_gemv_close(got, exact, f"dual model {m}", bound=fp16_weight_bound(a, w))
        assert normwise(got, exact) <= 1e-3
