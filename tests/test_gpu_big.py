"""GPU parity of the fused quad decode on the matrix cores (pp_quad_big: more than 64
tokens, and 9-64 tokens on (K,N) storage, in blocks of 1, 2, 4 or 8 token tiles of 16;
forced with ``fused=True`` above the size where the drop-in operator switches to the fp16
decode + library GEMM) against the float64 oracle: the fp16 operands the matrix cores
multiply (the float32 decode rounded once, plug tuples substituted, as the reference's
tl.dot takes them, quad_kernels.py:116-126) within rel 1e-3 plus the float32 dot-product
bound, and normwise within 1e-3 of the exact decode; and the batched decode + GEMM route
of the (K,N) layout against the fp16-weight bound."""
import ctypes
import functools
import math

import numpy as np
import pytest
import torch

import gen
from oracle import layer as olay
from oracle import quadpack as oqp
from polar_pack_amd import _native as nat
from polar_pack_amd import quad_kernels as qk
from polar_pack_amd.container import QuadPackFile
from parity import assert_gemv_close, fp16_weight_bound, normwise
from refs import check_mfma, kn_mfma_reference, mfma_reference

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


def random_codes(shape, seed):
    return np.random.default_rng(seed).integers(0, 2 ** 32, size=shape, dtype=np.uint64).astype(np.uint32)


def fp16_luts(seed, split=False):
    """LUTs as pack_quad_layer makes them (fp16); ``split``: q2 tables unlike the q1
    ones (the four-table LDS layout)."""
    ws = [torch.from_numpy(w.reshape(64, 64)).to(torch.float16) for w in gen.correlated_models(seed, [4096] * 4)]
    _, luts, scales = olay.pack_quad_layer(*ws)
    luts = [torch.from_numpy(l) for l in luts]
    if split:
        ang = torch.arange(256, dtype=torch.float64) / 255 * math.pi * 0.93 + 0.07
        luts[3] = torch.cos(ang).to(torch.float16)
        luts[4] = torch.sin(ang).to(torch.float16)
    return luts, scales


# two projections of one stream; the second starts mid-stream (plug positions relative)
SHAPES = [(100, 1024), (77, 512)]


@functools.lru_cache(maxsize=None)
def stream_pack():
    n = sum(a * b for a, b in SHAPES)
    qp = oqp.pack_quad(gen.correlated_models(77, [n] * 4), threshold=0.015)    # ~1.5% plugged
    dev = QuadPackFile(n=qp.n, s=qp.s, r_max=qp.r_max, codes=qp.codes, plug_idx=qp.plug_idx,
                       plug_vals=qp.plug_vals).to_device(DEV)
    return qp, dev


@pytest.mark.parametrize("M", [65, 100, 128, 129, 200, 333])
def test_container_rows_through_the_drop_in(M):
    """(N,K) container rows seen as the reference's (K,N) view, plug entries relative to
    the projection's stream position, header (float32) LUTs."""
    qp, pack = stream_pack()
    assert qp.plug_idx.size > 500
    pos = 0
    for p, (N, K) in enumerate(SHAPES):
        codes = pack.codes[pos:pos + N * K].reshape(N, K).t()
        luts = qk.header_luts(pack.r_max, device=DEV)
        x = np.random.default_rng(M + p).standard_normal((M, K)).astype(np.float16)
        outs = qk.quad_bitpacked(torch.from_numpy(x).to(DEV), codes, luts, list(pack.s),
                                 plug=(pack.plug_idx, pack.plug_vals), elem_base=pos, fused=True)
        check_mfma(outs, mfma_reference(qp, pos, N, K, x), f"proj {p} M={M}")
        pos += N * K


@pytest.mark.parametrize("M", [9, 16, 17, 33, 64, 65, 192])
@pytest.mark.parametrize("split", [False, True])
def test_kn_storage_with_plug_and_wider_rows(M, split):
    """(K,N) codes (pack_quad_layer's layout) as a column slice of a wider tensor (row stride
    520 > N = 300): plug entries of the block are moved to the kernel's (N,K) frame and
    applied, entries in the columns past N are not; fp16 LUTs, shared or split q1/q2; 9-192
    tokens (the one-wave form's 1 and 2 token tiles to 32 tokens, the producer/consumer
    form's 64- and 128-token blocks above, partial tiles and blocks)."""
    K, N, ldk = 1024, 300, 520
    seed = 500 + M + split
    wide = random_codes((K, ldk), seed)
    luts, scales = fp16_luts(seed, split)
    rng = np.random.default_rng(seed)
    base = 777
    inside = rng.choice(K * N, 400, replace=False)
    pad = rng.integers(0, K, 50) * ldk + rng.integers(N, ldk, 50)
    pos = np.unique(np.concatenate([(inside // N) * ldk + inside % N, pad]))
    vals = (rng.standard_normal((pos.size, 4)) * 0.5).astype(np.float16)
    view = u32(wide).to(DEV)[:, :N]
    a = rng.standard_normal((M, K)).astype(np.float16)
    outs = qk.quad_bitpacked(torch.from_numpy(a).to(DEV), view, [l.to(DEV) for l in luts], scales,
                             plug=(u32((pos + base).astype(np.uint32)).to(DEV), torch.from_numpy(vals).to(DEV)),
                             elem_base=base, fused=True)
    blk = (pos % ldk) < N
    ref = kn_mfma_reference(a, wide[:, :N], luts, scales, (pos[blk] // ldk, pos[blk] % ldk), vals[blk])
    check_mfma(outs, ref, f"kn M={M} split={split}")


def _call_big(x, codes_nk, luts, scales, plug, elem_base, slices, cols, o_sm):
    """pp_quad_big through the C-ABI on (N,K) rows with an explicit K-slice plan and an
    output row stride o_sm (outputs are column slices of wider buffers filled with NaN)."""
    M, K = x.shape
    N = codes_nk.shape[0]
    assert codes_nk.shape == (N, K)
    L = nat.lib()
    idx, vals = plug
    keys = (elem_base + np.arange(N, dtype=np.int64)[:, None] * K
            + np.arange(slices, dtype=np.int64)[None, :] * cols).reshape(-1)
    keys = np.concatenate([keys, [elem_base + N * K]])
    row_plug = torch.from_numpy(np.searchsorted(idx.cpu().view(torch.int32).numpy().view(np.uint32).astype(np.int64),
                                                keys)).to(DEV)
    wide = [torch.full((M, o_sm), float("nan"), dtype=torch.float16, device=DEV) for _ in range(4)]
    ws_bytes = L.pp_quad_big_workspace_size(M, N, slices)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    lut_ptrs, lut_dtype = qk._lut_args(luts)
    for rep in range(2):   # the second call reuses the workspace the first left zero
        rc = L.pp_quad_big(codes_nk.data_ptr(), nat.PP_QUAD_NK, K, x.data_ptr(), x.stride(0), lut_ptrs, lut_dtype,
                           nat.float_array(scales), idx.data_ptr(), vals.data_ptr(), idx.numel(),
                           row_plug.data_ptr(), elem_base, K, slices, cols,
                           nat.ptr_array([w.data_ptr() for w in wide]), o_sm, M, N, K, ws.data_ptr(), ws_bytes,
                           torch.cuda.current_stream(DEV).cuda_stream)
        nat.check(rc, "pp_quad_big")
        torch.cuda.synchronize()
        yield [w[:, :N] for w in wide], wide
    if ws_bytes:
        assert int(torch.count_nonzero(ws)) == 0, "the workspace is not left zero"


@pytest.mark.parametrize("M", [12, 30, 64, 150, 300])
@pytest.mark.parametrize("slices,cols", [(1, 512), (2, 256), (3, 192), (16, 32)])
def test_explicit_slices_and_odd_output_stride(slices, cols, M):
    """Every K-slice plan (one slice: direct fp16 stores; more: float32 atomics and the
    finish pass; slices shorter than a loop pass of 2 or 4 steps, or than a 64-column
    super-step), N = 70 (a partial 16-row tile, a partial 32-row block), 12-300 tokens (the
    one-wave form's 1, 2 and 4 token tiles to 64 tokens on these (N,K) rows, the
    producer/consumer form's 128- and 256-token blocks above), an odd output row stride (no
    4-row stores), and the columns past N left untouched."""
    N, K = 70, 512
    ws_ = gen.correlated_models(31, [N * K] * 4)
    qp = oqp.pack_quad(ws_, threshold=0.02)
    base = 96
    codes = u32(qp.codes).to(DEV).reshape(N, K)
    luts = qk.header_luts(qp.r_max, device=DEV)
    plug = (u32((qp.plug_idx.astype(np.int64) + base).astype(np.uint32)).to(DEV),
            torch.from_numpy(qp.plug_vals).to(DEV))
    x_np = np.random.default_rng(slices + M).standard_normal((M, K)).astype(np.float16)
    x = torch.from_numpy(x_np).to(DEV)
    ref = mfma_reference(qp, 0, N, K, x_np)
    for outs, wide in _call_big(x, codes, luts, list(qp.s), plug, base, slices, cols, N + 3):
        check_mfma(outs, ref, f"slices={slices} M={M}")
        for w in wide:
            assert bool(torch.isnan(w[:, N:]).all()), "a column past N was written"


def test_plan_covers_k():
    L = nat.lib()
    for M, N, K in ((65, 4096, 4096), (1024, 4096, 4096), (128, 11008, 2048), (300, 2048, 11008), (100, 7, 64),
                    (9, 4096, 4096), (16, 11008, 2048), (32, 2048, 11008), (64, 300, 96)):
        plan = (ctypes.c_int64 * 2)()
        for layout in (nat.PP_QUAD_NK, nat.PP_QUAD_KN):
            nat.check(L.pp_quad_big_plan(M, N, K, layout, ctypes.byref(plan, 0), ctypes.byref(plan, 8)), "plan")
            s, c = int(plan[0]), int(plan[1])
            assert c % 32 == 0 and s * c >= K and (s - 1) * c < K


def test_full_size_kn_layer_column_sample():
    """A 4096 x 4096 layer packed by pack_quad_layer at 1024 tokens (the reference
    benchmark's largest batch, quad_kernels.py:175-200): every output computed, a sample of
    96 columns checked against the oracle."""
    K = N = 4096
    M = 1024
    g = torch.Generator(device=DEV).manual_seed(11)
    ws = [torch.randn(K, N, generator=g, device=DEV).to(torch.float16) for _ in range(4)]
    codes, luts, scales = qk.pack_quad_layer(*ws)
    del ws
    a = torch.randn(M, K, generator=g, device=DEV).to(torch.float16)
    outs = qk.quad_bitpacked(a, codes, luts, scales, fused=True)
    torch.cuda.synchronize()
    cols = np.sort(np.random.default_rng(5).choice(N, 96, replace=False))
    codes_np = codes.view(torch.int32).cpu().numpy().view(np.uint32)
    ref = kn_mfma_reference(a.cpu().numpy(), codes_np, [l.cpu() for l in luts], scales, cols=cols)
    check_mfma([o[:, torch.from_numpy(cols).to(DEV)] for o in outs], ref, "4096x4096 M=1024")


@pytest.mark.parametrize("M", [10, 24, 48])
def test_kn_default_route_small_batches(M):
    """9-64 tokens on (K,N) storage take the fused kernel by default (no transposed copy of
    the codes): the matrix cores' fp16-operand bound, plug entries applied."""
    K, N = 512, 388
    seed = 950 + M
    codes = random_codes((K, N), seed)
    luts, scales = fp16_luts(seed)
    rng = np.random.default_rng(seed)
    flat = np.sort(rng.choice(K * N, 300, replace=False))
    vals = (rng.standard_normal((300, 4)) * 0.5).astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float16)
    outs = qk.quad_bitpacked(torch.from_numpy(a).to(DEV), u32(codes).to(DEV), [l.to(DEV) for l in luts], scales,
                             plug=(u32(flat.astype(np.uint32)).to(DEV), torch.from_numpy(vals).to(DEV)))
    ref = kn_mfma_reference(a, codes, luts, scales, (flat // N, flat % N), vals)
    check_mfma(outs, ref, f"kn default M={M}")


@pytest.mark.parametrize("M,N,plug,fused,big", [(2, 388, False, None, True), (2, 600, False, None, False),
                                                (3, 600, False, None, True), (5, 388, False, None, True),
                                                (8, 1000, False, None, True), (4, 388, True, None, False),
                                                (1, 388, False, True, True), (4, 388, True, True, True)])
def test_kn_few_tokens_route(monkeypatch, M, N, plug, fused, big):
    """2-8 tokens on (K,N) storage without plug entries take the fused matrix-core kernel by
    default (from 2 tokens when N <= K, from 3 when N > K), with plug entries the fused row
    kernel; fused=True takes the matrix-core kernel at 1 token and with plug entries.  The
    route taken is recorded; the matrix cores are held to their fp16-operand bound, the row
    kernel to the float32 decode's bound."""
    K = 512
    seed = 970 + 10 * M + N
    codes = random_codes((K, N), seed)
    luts, scales = fp16_luts(seed)
    rng = np.random.default_rng(seed)
    flat = np.sort(rng.choice(K * N, 250, replace=False)) if plug else None
    vals = (rng.standard_normal((250, 4)) * 0.5).astype(np.float16) if plug else None
    a = rng.standard_normal((M, K)).astype(np.float16)
    taken = []
    real = qk._quad_big
    monkeypatch.setattr(qk, "_quad_big", lambda *args: taken.append(1) or real(*args))
    pl = (u32(flat.astype(np.uint32)).to(DEV), torch.from_numpy(vals).to(DEV)) if plug else None
    outs = qk.quad_bitpacked(torch.from_numpy(a).to(DEV), u32(codes).to(DEV), [l.to(DEV) for l in luts], scales,
                             plug=pl, fused=fused)
    assert bool(taken) == big
    if big:
        ref = kn_mfma_reference(a, codes, luts, scales, (flat // N, flat % N) if plug else None, vals)
        check_mfma(outs, ref, f"kn M={M} N={N}")
        return
    W = olay.quad_dequant(codes, [l.float().numpy() for l in luts], scales)
    for m in range(4):
        if plug:
            W[m][flat // N, flat % N] = vals[:, m].astype(np.float64) * scales[m]
        assert_gemv_close(outs[m].float().cpu().numpy(), a.astype(np.float64) @ W[m], f"model {m}")


@pytest.mark.parametrize("M,fused", [(40, False), (100, False), (300, None)])
def test_kn_decode_and_batched_gemm_route(M, fused):
    """(K,N) storage through the fp16 decode + one batched library GEMM (the default above
    128 tokens, or fused=False): the fp16-weight bound and normwise 1e-3 against the exact
    decode, plug entries applied."""
    K, N = 512, 384
    seed = 900 + M
    codes = random_codes((K, N), seed)
    luts, scales = fp16_luts(seed)
    rng = np.random.default_rng(seed)
    flat = np.sort(rng.choice(K * N, 200, replace=False))
    vals = (rng.standard_normal((200, 4)) * 0.5).astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float16)
    outs = qk.quad_bitpacked(torch.from_numpy(a).to(DEV), u32(codes).to(DEV), [l.to(DEV) for l in luts], scales,
                             plug=(u32(flat.astype(np.uint32)).to(DEV), torch.from_numpy(vals).to(DEV)), fused=fused)
    W = olay.quad_dequant(codes, [l.float().numpy() for l in luts], scales)
    for m in range(4):
        W[m][flat // N, flat % N] = vals[:, m].astype(np.float64) * scales[m]
        exact = a.astype(np.float64) @ W[m]
        got = outs[m].float().cpu().numpy()
        assert outs[m].shape == (M, N) and outs[m].is_contiguous()
        assert_gemv_close(got, exact, f"model {m}", bound=fp16_weight_bound(a, W[m]))
        assert normwise(got, exact) <= 1e-3


def test_raw_stream_is_torch_current_stream():
    """The operators launch on torch's current stream: the handle they read is the one
    torch reports, also inside a side-stream context, and outputs computed there match."""
    assert nat.raw_stream(DEV) == torch.cuda.current_stream(DEV).cuda_stream
    K, N, M = 512, 256, 4
    codes = random_codes((K, N), 5)
    luts, scales = fp16_luts(5)
    a = torch.from_numpy(np.random.default_rng(5).standard_normal((M, K)).astype(np.float16)).to(DEV)
    cd, ld = u32(codes).to(DEV), [l.to(DEV) for l in luts]
    ref = qk.quad_bitpacked(a, cd, ld, scales)
    s = torch.cuda.Stream(DEV)
    s.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(s):
        assert nat.raw_stream(DEV) == s.cuda_stream != torch.cuda.default_stream(DEV).cuda_stream
        got = qk.quad_bitpacked(a, cd, ld, scales)
    torch.cuda.current_stream(DEV).wait_stream(s)
    for g, r in zip(got, ref):       # one fp16 ulp: K-slice sums are added in any order
        g32, r32 = g.float(), r.float()
        assert bool(((g32 - r32).abs() <= 2.0 ** -10 * r32.abs() + 2.0 ** -14 * r32.abs().max()).all())


@pytest.mark.parametrize("n,pos0,pld,rows,slices,cols", [(0, 0, 64, 10, 2, 32), (1000, 5, 300, 77, 3, 100),
                                                       (5000, 2 ** 31 + 7, 2 ** 19, 3000, 1, 0)])
def test_plug_search_matches_searchsorted(n, pos0, pld, rows, slices, cols):
    """pp_plug_search against numpy's left searchsorted, positions past 2^31 included."""
    rng = np.random.default_rng(n + rows)
    span = pos0 + rows * pld + 10
    assert span < 2 ** 32                                   # positions are uint32
    idx = np.unique(rng.integers(max(0, pos0 - 50), span, size=n, dtype=np.int64)).astype(np.uint32)
    keys = (pos0 + np.arange(rows, dtype=np.int64)[:, None] * pld + np.arange(slices)[None, :] * cols).reshape(-1)
    keys = np.append(keys, pos0 + rows * pld)
    ref = np.searchsorted(idx.astype(np.int64), keys, side="left")
    got = nat.plug_search(u32(idx).to(DEV), idx.size, pos0, pld, rows, slices, cols, DEV)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_operators_with_plug_entries_in_a_graph():
    """The drop-in operators with plug entries captured in a HIP graph: (N,K) rows on the batch
    decode (8 tokens) and the fused kernel (100 tokens), (K,N) codes on the fused kernel (16
    tokens, entries also in the columns past N, which the row stride holds), dual int16 (K,N)
    codes on the matrix cores (8 tokens).  Every replay, with eager work and
    synchronizations between them, matches the eager call to one fp16 ulp (K-slice sums
    are added in any order)."""
    from polar_pack_amd import polar_kernels as pk
    rng = np.random.default_rng(31)
    K, N, ldk = 512, 384, 400
    luts, scales = fp16_luts(31)
    L = [l.to(DEV) for l in luts]
    wide = random_codes((K, ldk), 31)
    nk = u32(np.ascontiguousarray(wide[:, :N].T)).to(DEV).t()
    kn = u32(wide).to(DEV)[:, :N]
    flat_nk = np.sort(rng.choice(K * N, 200, replace=False)).astype(np.uint32)
    flat_kn = np.sort(rng.choice(K * ldk, 260, replace=False)).astype(np.uint32)
    v_nk = torch.from_numpy((rng.standard_normal((200, 4)) * 0.5).astype(np.float16)).to(DEV)
    v_kn = torch.from_numpy((rng.standard_normal((260, 4)) * 0.5).astype(np.float16)).to(DEV)
    w1, w2 = (torch.from_numpy(w.reshape(K, N)).to(torch.float16) for w in gen.correlated_models(32, [K * N] * 2))
    dl = [torch.from_numpy(np.ascontiguousarray(t)).to(DEV) for t in olay.quantize_polar_bitpacked(w1, w2)]
    flat_d = np.sort(rng.choice(K * N, 150, replace=False)).astype(np.uint32)
    amp_d = torch.from_numpy(np.abs(rng.standard_normal(150) * 0.05).astype(np.float16)).to(DEV)
    xs = {M: torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(DEV) for M in (8, 16, 100)}
    p_nk, p_kn, p_d = (u32(flat_nk).to(DEV), v_nk), (u32(flat_kn).to(DEV), v_kn), (u32(flat_d).to(DEV), amp_d)
    calls = [
        lambda: qk.quad_bitpacked(xs[8], nk, L, scales, plug=p_nk),
        lambda: qk.quad_bitpacked(xs[100], nk, L, scales, plug=p_nk),
        lambda: qk.quad_bitpacked(xs[16], kn, L, scales, plug=p_kn),
        lambda: list(pk.polar_dual_bitpacked(xs[8], *dl, plug=p_d)),
    ]
    eager = [[o.clone() for o in c()] for c in calls]
    for c in calls:                       # warm the workspace caches outside the capture
        c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = [c() for c in calls]
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for e, o in zip(eager, got):
            for a, b in zip(e, o):
                a32, b32 = a.float(), b.float()
                lim = 2.0 ** -10 * a32.abs() + 2.0 ** -14 * a32.abs().max()     # one fp16 ulp
                assert bool(((b32 - a32).abs() <= lim).all()), f"replay {rep}"
        torch.randn(1 << 20, device=DEV).sum().item()     # eager work between the replays


def test_operator_workspace_reused_and_left_zero():
    """The drop-in operators keep one zeroed K-slice workspace per stream: repeated calls of
    different sizes (the buffer grows, then is reused) stay correct and leave it zero."""
    K, N = 1024, 512
    codes = random_codes((K, N), 77)
    luts, scales = fp16_luts(77)
    dl = [l.to(DEV) for l in luts]
    dc = u32(codes).to(DEV)
    for M in (12, 40, 12, 64, 20):
        a = np.random.default_rng(M).standard_normal((M, K)).astype(np.float16)
        outs = qk.quad_bitpacked(torch.from_numpy(a).to(DEV), dc, dl, scales)
        check_mfma(outs, kn_mfma_reference(a, codes, luts, scales), f"reuse M={M}")
    torch.cuda.synchronize()
    assert nat._zero_ws, "no cached workspace was used"
    for ws in nat._zero_ws.values():
        assert int(torch.count_nonzero(ws)) == 0, "a cached workspace is not left zero"
