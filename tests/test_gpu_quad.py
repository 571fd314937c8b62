"""GPU parity of the quad decode against the float64 oracle (same seeded inputs)."""
import math

import numpy as np
import pytest
import torch

import gen
from oracle import layer as olay
from oracle import quadpack as oqp
from parity import fp16_ulp_distance, fp16_weight_bound, normwise, assert_dequant_close, assert_gemv_close
from polar_pack_amd import quad_kernels as qk
from polar_pack_amd import routes
from refs import route_class

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


def np_u32(t):
    return t.cpu().view(torch.int32).numpy().view(np.uint32)


def random_codes(shape, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, 2 ** 32, size=shape, dtype=np.uint64).astype(np.uint32)


def correlated_codes(N, K, seed):
    """Codes of a real pack (correlated 4-model weights), (N,K) row-major."""
    ws = gen.correlated_models(seed, [N * K] * 4)
    qp = oqp.pack_quad(ws, threshold=0.01)
    return qp


def fp16_luts(seed=0):
    """LUTs as pack_quad_layer makes them (fp16)."""
    ws = [torch.from_numpy(w.reshape(64, 64)).to(torch.float16) for w in gen.correlated_models(seed, [4096] * 4)]
    _, luts, scales = olay.pack_quad_layer(*ws)
    return [torch.from_numpy(l) for l in luts], scales


def oracle_w(codes_kn, luts, scales):
    return olay.quad_dequant(codes_kn, [l.float().numpy() if torch.is_tensor(l) else l for l in luts], scales)


def test_quad_dequant_all_byte_values_fp16_and_fp32_luts():
    codes = random_codes((64, 300), 1)
    codes[0, :256] = np.arange(256, dtype=np.uint32) * 0x01010101
    for luts, scales in (fp16_luts(), (qk.header_luts(7.5), [0.02, 0.021, 0.0225, 0.019])):
        got = qk.quad_dequant(u32(codes).to(DEV), [l.to(DEV) for l in luts], scales)
        ref = oracle_w(codes, luts, scales)
        for k in range(4):
            assert_dequant_close(got[k].cpu().numpy(), ref[k], f"model {k}")


def test_quad_dequant_f16_is_rounded_f32():
    """The fp16 decode (the large-batch path's weights) is the float32 decode rounded to fp16."""
    codes = random_codes((64, 300), 4)
    luts, scales = fp16_luts(2)
    args = (u32(codes).to(DEV), [l.to(DEV) for l in luts], scales)
    w32 = qk.quad_dequant(*args)
    w16 = qk.quad_dequant(*args, dtype=torch.float16)
    for a32, a16 in zip(w32, w16):
        assert a16.dtype == torch.float16
        # the fp16 store may round the exact product once (a mixed-precision multiply)
        # where the float32 path rounds twice: at most 1 ulp apart, and rarely
        d = fp16_ulp_distance(a16.cpu().numpy(), a32.cpu().numpy())
        assert d.max() <= 1 and (d > 0).mean() < 1e-3


@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_quad_dequant_plug_positions_exact(layout):
    K, N = 48, 40
    codes = random_codes((K, N), 2)
    luts, scales = fp16_luts(1)
    rng = np.random.default_rng(3)
    base = 1000
    flat = np.sort(rng.choice(K * N, 77, replace=False)).astype(np.uint32)
    vals = (rng.standard_normal((77, 4)) * 3).astype(np.float16)
    if layout == "kn":
        view = u32(codes).to(DEV)                        # storage offset k*N + n
        kk, nn = flat // N, flat % N
    else:
        store = np.ascontiguousarray(codes.T)            # (N,K) rows, view (K,N) with strides (1,K)
        view = u32(store).to(DEV).t()
        nn, kk = flat // K, flat % K
    idx = (flat + base).astype(np.uint32)
    # entries outside the matrix are ignored
    idx = np.concatenate([np.array([3], np.uint32), idx, np.array([base + K * N + 5], np.uint32)])
    vals = np.concatenate([np.ones((1, 4), np.float16), vals, np.ones((1, 4), np.float16)])
    got = qk.quad_dequant(view, [l.to(DEV) for l in luts], scales,
                          plug=(u32(idx).to(DEV), torch.from_numpy(vals).to(DEV)), elem_base=base)
    ref = oracle_w(codes, luts, scales)
    for k in range(4):
        ref[k][kk, nn] = vals[1:-1, k].astype(np.float64) * scales[k]
        g = got[k].cpu().numpy()
        assert_dequant_close(g, ref[k], f"model {k}")
        np.testing.assert_array_equal(g[kk, nn], (vals[1:-1, k].astype(np.float32) * np.float32(scales[k])))


SHAPES = [(2048, 256), (11008, 64), (512, 1024), (130, 40), (96, 7)]


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16])
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("K,N", SHAPES)
def test_quad_gemm_matches_oracle(K, N, layout, M):
    seed = K * 7 + N * 3 + M
    codes = random_codes((K, N), seed)
    luts, scales = fp16_luts(seed)
    view = u32(codes).to(DEV) if layout == "kn" else u32(np.ascontiguousarray(codes.T)).to(DEV).t()
    rng = np.random.default_rng(seed)
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    outs = qk.quad_bitpacked(a.to(DEV), view, [l.to(DEV) for l in luts], scales)
    W = oracle_w(codes, luts, scales)
    # more than 8 tokens on (N,K) rows: the matrix-core path, fp16 weights into the dot
    # product (as the reference's tl.dot); held to the fp16-rounded decode + the fp32
    # dot-product bound (see test_gpu_mfma.py)
    cls = route_class(qk.quad_call_route(view, M))
    mfma, prefill = cls == "mfma", cls == "prefill"
    W32 = olay.quad_dequant(codes, [l.float().numpy() for l in luts], dtype=np.float32) if mfma else None
    for k in range(4):
        assert outs[k].shape == (M, N) and outs[k].dtype == torch.float16
        w = W[k]
        bound = None
        if mfma:
            w = W32[k].astype(np.float16).astype(np.float64) * float(np.float32(scales[k]))
            bound = 2.0 ** -18 * (np.abs(a.numpy().astype(np.float64)) @ np.abs(w))
            assert normwise(outs[k].float().cpu().numpy(), olay.gemm_f64(a.numpy(), W[k])) <= 1e-3
        if prefill:
            bound = fp16_weight_bound(a.numpy(), w)
            assert normwise(outs[k].float().cpu().numpy(), olay.gemm_f64(a.numpy(), W[k])) <= 1e-3
        assert_gemv_close(outs[k].float().cpu().numpy(), olay.gemm_f64(a.numpy(), w), f"model {k}", bound=bound)


@pytest.mark.parametrize("M", [1, 4, 8, 300])
def test_quad_gemm_real_pack_with_plug_fast_path(M):
    """A real packed layer (N,K) = (1024, 2048) with plug entries, container (N,K) layout."""
    N, K = 1024, 2048
    qp = correlated_codes(N, K, 5)
    assert qp.plug_idx.size > 100
    base = 4096                                         # the layer sits at stream offset 4096
    codes_nk = qp.codes.reshape(N, K)
    luts = qk.header_luts(qp.r_max)
    rng = np.random.default_rng(M)
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    view = u32(codes_nk).to(DEV).t()
    outs = qk.quad_bitpacked(a.to(DEV), view, [l.to(DEV) for l in luts], list(qp.s),
                             plug=(u32(qp.plug_idx + base).to(DEV), torch.from_numpy(qp.plug_vals).to(DEV)),
                             elem_base=base)
    cls = route_class(qk.quad_call_route(view, M, qp.plug_idx.size))
    W = oqp.unpack_quad_f64(qp, 0, N * K)                # float64, plug applied, times s_k
    for k in range(4):
        w = W[k].reshape(N, K).T
        # fp16 weights into the product on the matrix cores and the fp16 decode + library GEMM
        bound = fp16_weight_bound(a.numpy(), w) if cls != "fused" else None
        if bound is not None:
            assert normwise(outs[k].float().cpu().numpy(), olay.gemm_f64(a.numpy(), w)) <= 1e-3
        assert_gemv_close(outs[k].float().cpu().numpy(), olay.gemm_f64(a.numpy(), w), f"model {k}", bound=bound)


def test_quad_gemm_plug_generic_layout():
    K, N = 256, 96
    codes = random_codes((K, N), 9)
    luts, scales = fp16_luts(9)
    rng = np.random.default_rng(9)
    flat = np.sort(rng.choice(K * N, 300, replace=False)).astype(np.uint32)
    vals = (rng.standard_normal((300, 4))).astype(np.float16)
    a = torch.from_numpy(rng.standard_normal((3, K)).astype(np.float16))
    outs = qk.quad_bitpacked(a.to(DEV), u32(codes).to(DEV), [l.to(DEV) for l in luts], scales,
                             plug=(u32(flat).to(DEV), torch.from_numpy(vals).to(DEV)))
    W = oracle_w(codes, luts, scales)
    kk, nn = flat // N, flat % N
    for k in range(4):
        W[k][kk, nn] = vals[:, k].astype(np.float64) * scales[k]
        assert_gemv_close(outs[k].float().cpu().numpy(), olay.gemm_f64(a.numpy(), W[k]), f"model {k}")


def test_quad_gemm_gate_proj_shape_batch1():
    """The gate_proj shape (N,K) = (11008, 2048) at batch 1, (N,K) stream layout."""
    N, K = 11008, 2048
    codes_nk = random_codes((N, K), 11)
    luts = qk.header_luts(9.0)
    scales = [0.02, 0.021, 0.022, 0.023]
    a = torch.from_numpy(np.random.default_rng(11).standard_normal((1, K)).astype(np.float16))
    outs = qk.quad_bitpacked(a.to(DEV), u32(codes_nk).to(DEV).t(), [l.to(DEV) for l in luts], scales)
    W = olay.quad_dequant(codes_nk, [l.double().numpy() for l in luts], scales)
    for k in range(4):
        assert_gemv_close(outs[k].float().cpu().numpy(), a.double().numpy() @ W[k].T, f"model {k}")


def test_quad_gemm_edge_cases():
    luts, scales = fp16_luts(0)
    L = [l.to(DEV) for l in luts]
    a = torch.zeros(0, 8, dtype=torch.float16, device=DEV)
    outs = qk.quad_bitpacked(a, u32(random_codes((8, 4), 0)).to(DEV), L, scales)
    assert all(o.shape == (0, 4) for o in outs)
    a = torch.ones(2, 0, dtype=torch.float16, device=DEV)
    outs = qk.quad_bitpacked(a, u32(np.zeros((0, 5), np.uint32)).to(DEV), L, scales)
    assert all(o.shape == (2, 5) and float(o.abs().sum()) == 0 for o in outs)
    with pytest.raises(AssertionError):
        qk.quad_bitpacked(torch.ones(1, 8, dtype=torch.float16, device=DEV), u32(random_codes((9, 4), 0)).to(DEV),
                          L, scales)
    # non-contiguous activations (a column slice) go through the same kernels
    codes = random_codes((64, 32), 4)
    big = torch.from_numpy(np.random.default_rng(4).standard_normal((3, 130)).astype(np.float16))
    a = big[:, 1:65]
    outs = qk.quad_bitpacked(a.to(DEV), u32(np.ascontiguousarray(codes.T)).to(DEV).t(), L, scales)
    W = oracle_w(codes, luts, scales)
    for k in range(4):
        assert_gemv_close(outs[k].float().cpu().numpy(), olay.gemm_f64(a.numpy(), W[k]), f"model {k}")


def test_pack_quad_layer_on_gpu_matches_oracle():
    ws = [torch.from_numpy(w.reshape(256, 96)).to(torch.float16) for w in gen.correlated_models(77, [256 * 96] * 4)]
    codes, luts, scales = qk.pack_quad_layer(*[w.to(DEV) for w in ws])
    rc, rl, rs = olay.pack_quad_layer(*ws)
    got = np_u32(codes)
    diff = got != rc
    # device transcendentals may round differently at a tie: at most a few codes, by one step in one field
    assert diff.mean() < 2e-3, diff.mean()
    for sh in (0, 8, 16, 24):
        d = np.abs(((got >> sh) & 255).astype(np.int32) - ((rc >> sh) & 255).astype(np.int32))
        assert d.max() <= 1
    for k in range(4):
        assert abs(scales[k] - rs[k]) <= 1e-6 * rs[k]
    for i in range(1, 7):
        np.testing.assert_array_equal(luts[i].cpu().numpy().view(np.uint16), rl[i].view(np.uint16))


def kn_route(K, N, M, plug):
    """How quad_bitpacked's route for contiguous (K,N) codes is held to the oracle
    (:func:`refs.route_class` of the routing table's cell)."""
    caps = routes.quad_storage(N, 1, 0, K, N, 1 if plug else 0)
    return route_class(routes.quad_route(M, K, N, caps, bool(plug)))


def check_route(outs, a, codes, luts, scales, route, plug_at=None, plug_vals=None, what=""):
    """Outputs of one route against the float64 oracle: the exact decode for the fused
    kernels (rel 1e-3); for the matrix cores the fp16 operands they multiply (the float32
    decode rounded once, plug tuples substituted) with the float32 dot-product bound, and
    normwise 1e-3 against the exact decode; for the fp16 decode + GEMM the fp16-weight
    bound, and normwise 1e-3."""
    an = a.numpy() if torch.is_tensor(a) else a
    W = oracle_w(codes, luts, scales)
    W32 = olay.quad_dequant(codes, [l.float().numpy() for l in luts], dtype=np.float32) if route == "mfma" else None
    for k in range(4):
        if plug_at is not None:
            W[k][plug_at] = plug_vals[:, k].astype(np.float64) * scales[k]
        got = outs[k].float().cpu().numpy()
        exact = olay.gemm_f64(an, W[k])
        if route == "fused":
            assert_gemv_close(got, exact, f"{what} model {k}")
            continue
        assert normwise(got, exact) <= 1e-3, f"{what} model {k}: normwise {normwise(got, exact):.2e}"
        if route == "mfma":
            h = W32[k].astype(np.float16)
            if plug_at is not None:
                h[plug_at] = plug_vals[:, k]
            w = h.astype(np.float64) * float(np.float32(scales[k]))
            bound = 2.0 ** -18 * (np.abs(an.astype(np.float64)) @ np.abs(w))
            assert_gemv_close(got, olay.gemm_f64(an, w), f"{what} model {k}", bound=bound)
        else:
            assert_gemv_close(got, exact, f"{what} model {k}", bound=fp16_weight_bound(an, W[k]))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 8, 13, 40, 64, 100])
@pytest.mark.parametrize("K,N,plug", [(2048, 1000, 0), (2048, 1000, 700), (64, 96, 0), (520, 4096, 300)])
def test_quad_gemm_kn_layout_fast_path(K, N, plug, M):
    """Contiguous (K,N) codes, the layout pack_quad_layer returns: the fused (K,N) kernel
    (256-column items for 1-4 tokens, 128-column items for 5-8, K slices whose partial
    sums a finish pass adds, plug corrections per entry; blocks of 8 tokens), the codes
    transposed for the matrix cores, or the fp16 decode + GEMM, each against its oracle."""
    seed = K + N + plug + M
    codes = random_codes((K, N), seed)
    luts, scales = fp16_luts(seed)
    rng = np.random.default_rng(seed)
    base = 1000
    flat = np.sort(rng.choice(K * N, plug, replace=False)).astype(np.uint32)
    vals = (rng.standard_normal((plug, 4)) * 0.5).astype(np.float16)
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    kw = {}
    if plug:
        kw = dict(plug=(u32(flat + base).to(DEV), torch.from_numpy(vals).to(DEV)), elem_base=base)
    outs = qk.quad_bitpacked(a.to(DEV), u32(codes).to(DEV), [l.to(DEV) for l in luts], scales, **kw)
    check_route(outs, a, codes, luts, scales, kn_route(K, N, M, plug), (flat // N, flat % N), vals, f"M={M}")


@pytest.mark.parametrize("M", [4, 40, 200])
def test_quad_gemm_kn_layout_wider_row_stride(M):
    """(K,N) codes that are a column slice of a wider tensor (row stride ldk > N, ldk % 4 ==
    0): plug entries in the block are applied, entries in the columns past N are not."""
    K, N, ldk = 1024, 500, 520
    seed = 71 + M
    wide = random_codes((K, ldk), seed)
    luts, scales = fp16_luts(seed)
    rng = np.random.default_rng(seed)
    base = 333
    inside = rng.choice(K * N, 260, replace=False)
    kk_in, nn_in = inside // N, inside % N
    pad_k = rng.integers(0, K, 40)
    pad_n = rng.integers(N, ldk, 40)
    pos = np.concatenate([kk_in * ldk + nn_in, pad_k * ldk + pad_n])
    order = np.argsort(pos)
    pos = pos[order]
    pos, first = np.unique(pos, return_index=True)
    vals = (rng.standard_normal((pos.size, 4)) * 0.5).astype(np.float16)
    view = u32(wide).to(DEV)[:, :N]
    assert view.stride(0) == ldk
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    outs = qk.quad_bitpacked(a.to(DEV), view, [l.to(DEV) for l in luts], scales,
                             plug=(u32((pos + base).astype(np.uint32)).to(DEV), torch.from_numpy(vals).to(DEV)),
                             elem_base=base)
    in_block = (pos % ldk) < N
    check_route(outs, a, wide[:, :N], luts, scales, kn_route(K, N, M, True), (pos[in_block] // ldk, pos[in_block] % ldk),
                vals[in_block], f"ldk={ldk} M={M}")


def split_luts(seed):
    """fp16 LUTs whose q2 tables (cos2, sin2) differ from the q1 ones: the decode kernels'
    four-table LDS layout (the reference's 7-table interface allows any tables)."""
    luts, scales = fp16_luts(seed)
    ang = torch.arange(256, dtype=torch.float64) / 255 * math.pi * 0.93 + 0.07
    luts = list(luts)
    luts[3] = torch.cos(ang).to(torch.float16)
    luts[4] = torch.sin(ang).to(torch.float16)
    assert not torch.equal(luts[1], luts[3])
    return luts, scales


@pytest.mark.parametrize("layout,M", [("nk", 1), ("nk", 3), ("nk", 8), ("kn", 1), ("kn", 5), ("nk", 16), ("nk", 64),
                                      ("kn", 40)])
def test_quad_split_tables_every_route(layout, M):
    K, N = 1024, 384
    seed = 90 + M
    codes = random_codes((K, N), seed)
    luts, scales = split_luts(seed)
    rng = np.random.default_rng(seed)
    flat = np.sort(rng.choice(K * N, 150, replace=False)).astype(np.uint32)
    vals = (rng.standard_normal((150, 4)) * 0.5).astype(np.float16)
    if layout == "kn":
        view = u32(codes).to(DEV)
        idx = flat
        at = (flat // N, flat % N)
        route = kn_route(K, N, M, True)
    else:
        view = u32(np.ascontiguousarray(codes.T)).to(DEV).t()
        nn, kk = flat // K, flat % K          # storage offsets of (N,K) rows
        idx = flat
        at = (kk, nn)
        route = route_class(qk.quad_call_route(view, M, flat.size))
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    L = [l.to(DEV) for l in luts]
    outs = qk.quad_bitpacked(a.to(DEV), view, L, scales, plug=(u32(idx).to(DEV), torch.from_numpy(vals).to(DEV)))
    check_route(outs, a, codes, luts, scales, route, at, vals, f"{layout} M={M}")
    w = qk.quad_dequant(view, L, scales, plug=(u32(idx).to(DEV), torch.from_numpy(vals).to(DEV)))
    ref = oracle_w(codes, luts, scales)
    for k in range(4):
        ref[k][at] = vals[:, k].astype(np.float64) * scales[k]
        assert_dequant_close(w[k].cpu().numpy(), ref[k], f"dequant model {k}")
