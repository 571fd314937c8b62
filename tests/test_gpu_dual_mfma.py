"""GPU parity of the dual matrix-core decode (pp_dual_mfma, 2-64 tokens by default on the
int16 (K,N) layout quantize_polar_bitpacked returns, from 5 when N > K or with plug entries) against the float64 oracle: the fp16
operands the reference's tl.dot takes (the float32 decode (amp_lut * bmax) * cos/sin
rounded once, plug amplitudes substituted, polar_kernels.py:60-82) within rel 1e-3 plus the
float32 dot-product bound 2^-18 * sum |w x|, and normwise within 1e-3 of the exact decode."""
import ctypes

import numpy as np
import pytest
import torch

import gen
from oracle import layer as olay
from parity import assert_gemv_close, fp16_weight_bound, normwise
from polar_pack_amd import _native as nat
from polar_pack_amd import polar_kernels as pk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


def layer(K, N, seed, group_size=32):
    w1, w2 = (torch.from_numpy(w.reshape(K, N)).to(torch.float16) for w in gen.correlated_models(seed, [K * N] * 2))
    return olay.quantize_polar_bitpacked(w1, w2, group_size=group_size)


def check(outs, a, packed, bmax, amp_lut, cos_lut, sin_lut, group_size, plug=None, what=""):
    w32 = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut, group_size, dtype=np.float32, plug=plug)
    exact = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut, group_size, plug=plug)
    ad = np.asarray(a, np.float64)
    for m in range(2):
        w16 = w32[m].astype(np.float16).astype(np.float64)
        got = outs[m].float().cpu().numpy()
        assert_gemv_close(got, ad @ w16, f"{what} model {m}", bound=2.0 ** -18 * (np.abs(ad) @ np.abs(w16)))
        assert normwise(got, ad @ exact[m]) <= 1e-3, f"{what} model {m}: normwise {normwise(got, ad @ exact[m]):.2e}"


def to_dev(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(x)).to(DEV) for x in arrs]


@pytest.mark.parametrize("M", [9, 16, 32, 33, 64, 65, 128, 200, 300])
@pytest.mark.parametrize("K,N,plug,gs", [(1024, 384, 0, 32), (2048, 1000, 500, 32), (512, 4096, 300, 64),
                                         (96, 40, 40, 8), (256, 512, 0, 64), (512, 400, 0, 32), (128, 64, 0, 8),
                                         (320, 208, 0, 16)])
def test_kernel_layout_matches_oracle(K, N, plug, gs, M):
    """Several shapes (N not a multiple of 16, K = 96: one padded step), group sizes 8-64,
    plug amplitudes at random positions, 9-300 tokens (16-token tiles of 2, 4 or 8; one to
    two token blocks; K slices for the small batches), forced with fused=True above the
    operator's default range.  Without plug entries and with N a multiple of 16 and of the
    group size the kernel loads rows of 8 codes and transposes them through LDS (N = 400
    with 32-pair groups takes the column loads); from 65 tokens those rows go to the
    producer/consumer workgroups (64-column blocks: N = 208 ends in a partial block, K = 320
    in K slices of whole and partial super-steps; 128- and 256-token blocks)."""
    seed = K * 3 + N + plug + M + gs
    packed, bmax, amp_lut, cos_lut, sin_lut = layer(K, N, seed, gs)
    rng = np.random.default_rng(seed)
    base = 77
    flat = np.sort(rng.choice(K * N, plug, replace=False)).astype(np.uint32)
    vals = np.abs(rng.standard_normal(plug) * 0.05).astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float16)
    kw = {}
    if plug:
        kw = dict(plug=(u32(flat + base).to(DEV), torch.from_numpy(vals).to(DEV)), elem_base=base)
    o1, o2 = pk.polar_dual_bitpacked(*to_dev(a, packed, bmax, amp_lut, cos_lut, sin_lut), group_size=gs,
                                     fused=True, **kw)
    assert o1.shape == (M, N) and o1.dtype == torch.float16
    pl = (flat // N, flat % N, vals) if plug else None
    check((o1, o2), a, packed, bmax, amp_lut, cos_lut, sin_lut, gs, pl, f"K={K} N={N} M={M}")


@pytest.mark.parametrize("M", [12, 96])
def test_wider_row_stride_and_float32_luts(M):
    """(K,N) codes as a column slice of a wider tensor (row stride 520 > N = 300): plug
    entries in the block are applied, entries in the columns past N are not; float32 LUTs."""
    K, N, ldk = 512, 300, 520
    seed = 300 + M
    packed_w, bmax_w, amp_lut, cos_lut, sin_lut = layer(K, ldk, seed)
    # the block is the first N columns of the wide layer; its groups follow the block's own
    # (k*N + n) index, so give it the scales of that rule
    rng = np.random.default_rng(seed)
    bmax = (rng.random((K * N + 31) // 32) * 0.5 + 0.05).astype(np.float16)
    inside = rng.choice(K * N, 200, replace=False)
    pad = rng.integers(0, K, 40) * ldk + rng.integers(N, ldk, 40)
    pos = np.unique(np.concatenate([(inside // N) * ldk + inside % N, pad]))
    vals = np.abs(rng.standard_normal(pos.size) * 0.05).astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float16)
    luts32 = [np.asarray(l, np.float32) for l in (amp_lut, cos_lut, sin_lut)]
    view = torch.from_numpy(packed_w).to(DEV)[:, :N]
    assert view.stride(0) == ldk
    o1, o2 = pk.polar_dual_bitpacked(torch.from_numpy(a).to(DEV), view, torch.from_numpy(bmax).to(DEV),
                                     *[torch.from_numpy(l).to(DEV) for l in luts32],
                                     plug=(u32(pos.astype(np.uint32)).to(DEV), torch.from_numpy(vals).to(DEV)),
                                     fused=True)
    blk = (pos % ldk) < N
    pl = (pos[blk] // ldk, pos[blk] % ldk, vals[blk])
    check((o1, o2), a, packed_w[:, :N], bmax, *luts32, 32, pl, f"ldk={ldk} M={M}")


@pytest.mark.parametrize("M", [96, 300])
def test_producer_consumer_float32_luts_odd_output_stride(M):
    """The producer/consumer form (65 tokens and more, no plug table, N a multiple of 16 and
    of the group size) with float32 LUTs (its tables built from them) and outputs that are
    column slices of wider buffers (no 4-column stores); the columns past N untouched."""
    K, N, gs = 384, 144, 16
    seed = 900 + M
    packed, bmax, amp_lut, cos_lut, sin_lut = layer(K, N, seed, gs)
    luts32 = [np.asarray(l, np.float32) for l in (amp_lut, cos_lut, sin_lut)]
    a = np.random.default_rng(seed).standard_normal((M, K)).astype(np.float16)
    wide = [torch.full((M, N + 3), float("nan"), dtype=torch.float16, device=DEV) for _ in range(2)]
    o1, o2 = (w[:, :N] for w in wide)
    L = nat.lib()
    slices, cols = (ctypes.c_int64 * 1)(), (ctypes.c_int64 * 1)()
    nat.check(L.pp_dual_mfma_plan(M, N, K, slices, cols), "pp_dual_mfma_plan")
    s_, c_ = int(slices[0]), int(cols[0])
    ws_bytes = L.pp_dual_mfma_workspace_size(M, N, s_)
    ws = torch.zeros(max(ws_bytes, 16), dtype=torch.uint8, device=DEV)
    dv = to_dev(a, packed, bmax, *luts32)
    for rep in range(2):   # the second call reuses the workspace the first left zero
        rc = L.pp_dual_mfma(dv[1].data_ptr(), N, dv[0].data_ptr(), K, dv[2].data_ptr(), gs, dv[3].data_ptr(),
                            dv[3].numel(), dv[4].data_ptr(), dv[5].data_ptr(), dv[4].numel(), nat.PP_F32, None, None,
                            0, None, 0, K, s_, c_, o1.data_ptr(), o2.data_ptr(), N + 3, M, N, K, ws.data_ptr(),
                            ws_bytes, torch.cuda.current_stream(DEV).cuda_stream)
        nat.check(rc, "pp_dual_mfma")
        torch.cuda.synchronize()
        check((o1, o2), a, packed, bmax, *luts32, gs, None, f"float32 LUTs M={M} rep={rep}")
        for w in wide:
            assert bool(torch.isnan(w[:, N:]).all()), "a column past N was written"
    if ws_bytes:
        assert int(torch.count_nonzero(ws)) == 0, "the workspace is not left zero"


@pytest.mark.parametrize("M", [20, 70])
def test_wider_row_stride_row_loads(M):
    """No plug table, codes as a column slice of a wider tensor (row stride 536 > N = 320):
    the row loads read the block's 320 columns of each row only."""
    K, N, ldk = 256, 320, 536
    seed = 500 + M
    packed_w, _, amp_lut, cos_lut, sin_lut = layer(K, ldk, seed)
    rng = np.random.default_rng(seed)
    bmax = (rng.random((K * N + 31) // 32) * 0.5 + 0.05).astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float16)
    view = torch.from_numpy(packed_w).to(DEV)[:, :N]
    assert view.stride(0) == ldk
    o1, o2 = pk.polar_dual_bitpacked(torch.from_numpy(a).to(DEV), view, torch.from_numpy(bmax).to(DEV),
                                     *[torch.from_numpy(np.asarray(l)).to(DEV) for l in (amp_lut, cos_lut, sin_lut)],
                                     fused=True)
    check((o1, o2), a, packed_w[:, :N], bmax, amp_lut, cos_lut, sin_lut, 32, None, f"ldk={ldk} M={M}")


@pytest.mark.parametrize("M,K,N,plug,fused,mfma", [(2, 1024, 512, 0, None, True), (2, 512, 1024, 0, None, False),
                                                   (4, 512, 1024, 0, None, False), (5, 512, 1024, 0, None, True),
                                                   (3, 2048, 1000, 0, None, True), (4, 1024, 512, 300, None, False),
                                                   (1, 1024, 512, 0, True, True), (3, 1024, 512, 300, True, True)])
def test_few_tokens_route(monkeypatch, M, K, N, plug, fused, mfma):
    """int16 (K,N) codes: the matrix-core decode from 2 tokens when N <= K without plug
    entries, from 5 otherwise; fused=True at any size.  The route taken is recorded; the
    matrix cores are held to their fp16-operand bound, the fused (K,N) kernel to the float32
    decode's bound."""
    seed = 40 * M + K + N + plug
    packed, bmax, amp_lut, cos_lut, sin_lut = layer(K, N, seed)
    rng = np.random.default_rng(seed)
    base = 5
    flat = np.sort(rng.choice(K * N, plug, replace=False)).astype(np.uint32)
    vals = np.abs(rng.standard_normal(plug) * 0.05).astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float16)
    kw = dict(plug=(u32(flat + base).to(DEV), torch.from_numpy(vals).to(DEV)), elem_base=base) if plug else {}
    taken = []
    real = pk._dual_mfma
    monkeypatch.setattr(pk, "_dual_mfma", lambda *args: taken.append(1) or real(*args))
    o1, o2 = pk.polar_dual_bitpacked(*to_dev(a, packed, bmax, amp_lut, cos_lut, sin_lut), fused=fused, **kw)
    assert bool(taken) == mfma
    pl = (flat // N, flat % N, vals) if plug else None
    if mfma:
        check((o1, o2), a, packed, bmax, amp_lut, cos_lut, sin_lut, 32, pl, f"K={K} N={N} M={M}")
        return
    W = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut, 32, plug=pl)
    for o, w in zip((o1, o2), W):
        assert_gemv_close(o.float().cpu().numpy(), olay.gemm_f64(a, w))


@pytest.mark.parametrize("M,fused", [(40, False), (300, True)])
def test_fused_switch(M, fused):
    """fused=False takes the fp16 decode + batched GEMM (the fp16-weight bound), fused=True
    the matrix cores at any size."""
    K, N = 1024, 512
    packed, bmax, amp_lut, cos_lut, sin_lut = layer(K, N, 90 + M)
    a = np.random.default_rng(M).standard_normal((M, K)).astype(np.float16)
    o1, o2 = pk.polar_dual_bitpacked(*to_dev(a, packed, bmax, amp_lut, cos_lut, sin_lut), fused=fused)
    if fused:
        check((o1, o2), a, packed, bmax, amp_lut, cos_lut, sin_lut, 32, None, "fused")
        return
    W = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    for o, w in zip((o1, o2), W):
        got = o.float().cpu().numpy()
        assert_gemv_close(got, olay.gemm_f64(a, w), bound=fp16_weight_bound(a, w))
        assert normwise(got, olay.gemm_f64(a, w)) <= 1e-3


def test_full_size_layer_column_sample():
    """The reference benchmark's dual layer (4096 x 4096, quantize_polar_bitpacked of N(0,1)
    weights on the device) at 32 tokens: every output computed, 128 columns checked."""
    K = N = 4096
    M = 32
    g = torch.Generator(device=DEV).manual_seed(21)
    w1 = torch.randn(K, N, generator=g, device=DEV).to(torch.float16)
    w2 = torch.randn(K, N, generator=g, device=DEV).to(torch.float16)
    packed, bmax, amp_lut, cos_lut, sin_lut = pk.quantize_polar_bitpacked(w1, w2)
    del w1, w2
    a = torch.randn(M, K, generator=g, device=DEV).to(torch.float16)
    o1, o2 = pk.polar_dual_bitpacked(a, packed, bmax, amp_lut, cos_lut, sin_lut)
    torch.cuda.synchronize()
    cols = np.sort(np.random.default_rng(4).choice(N, 128, replace=False))
    p = packed.cpu().numpy()
    bm = bmax.cpu().numpy()
    # the sampled columns' own group scales: index (k*N + n) // 32 of the full layer
    sub = p[:, cols]
    g_idx = (np.arange(K)[:, None] * N + cols[None, :]) // 32
    luts = [l.cpu().numpy() for l in (amp_lut, cos_lut, sin_lut)]
    pp = sub.astype(np.int32) + 32768
    amp32 = luts[0].astype(np.float32)[(pp >> 10) & 63] * bm.astype(np.float32)[g_idx]
    ph = pp & 1023
    ad = a.cpu().numpy().astype(np.float64)
    for m, (o, lut) in enumerate(((o1, luts[1]), (o2, luts[2]))):
        w16 = (amp32 * lut.astype(np.float32)[ph]).astype(np.float16).astype(np.float64)
        exact = luts[0].astype(np.float64)[(pp >> 10) & 63] * bm.astype(np.float64)[g_idx] * lut.astype(np.float64)[ph]
        got = o[:, torch.from_numpy(cols).to(DEV)].float().cpu().numpy()
        assert_gemv_close(got, ad @ w16, f"model {m}", bound=2.0 ** -18 * (np.abs(ad) @ np.abs(w16)))
        assert normwise(got, ad @ exact) <= 1e-3
