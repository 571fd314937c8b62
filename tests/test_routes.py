"""The drop-in operators' routing tables (polar_pack_amd/routes.py), cell by cell, on the CPU:
which kernel quad_bitpacked / polar_dual_bitpacked runs for every storage class, plug
presence, ``fused`` setting and token count; the Python storage classes against the C
library's own choice (pp_quad_gemm_kernel / pp_dual_gemm_kernel); the 32-bit offset limits
that keep huge layers off the kernels that cannot address them; the plug-table sort."""
import numpy as np
import pytest
import torch

from polar_pack_amd import _native as nat
from polar_pack_amd import plugs, routes

INF = routes.INF


def cells(spec):
    """'rows:1-4 mfma:5-64 prefill:65-' -> [(kernel, lo, hi)]"""
    out = []
    for part in spec.split():
        k, rng = part.split(":")
        lo, hi = rng.split("-")
        out.append((k, int(lo), int(hi) if hi else INF))
    return out


MS = list(range(1, 140)) + [255, 256, 333, 1024, 4096]


def expect(route_fn, caps, K, N, plug, fused, spec):
    want = cells(spec)
    for M in MS:
        exp = [k for k, lo, hi in want if lo <= M <= hi]
        assert len(exp) == 1, (spec, M)
        got = route_fn(M, K, N, caps, plug, fused)
        assert got == exp[0], f"M={M} plug={plug} fused={fused}: {got} != {exp[0]} ({spec})"


# quad storages: (c_sk, c_sn, ptr, K, N) of the (K,N) view
def nk(K, N, ptr=256):
    return (1, K, ptr, K, N)          # (N,K) container rows seen as (K,N)


def kn(K, N, ptr=256):
    return (N, 1, ptr, K, N)          # pack_quad_layer's (K,N) codes


QUAD_TABLE = [
    # storage, plug, fused, expected cells
    (nk(2048, 512), (False, True), None, "rows:1-4 mfma:5-64 big_nk:65-128 prefill:129-"),
    (nk(512, 2048), (False, True), None, "rows:1-4 mfma:5-64 big_nk:65-128 prefill:129-"),
    (nk(2048, 512), (False, True), True, "rows:1-4 mfma:5-64 big_nk:65-"),
    (nk(2048, 512), (False, True), False, "rows:1-4 mfma:5-64 prefill:65-"),
    (nk(2056, 512), (False, True), None, "rows:1-8 prefill:9-"),                 # K % 32 != 0
    (nk(2056, 512), (False, True), True, "rows:1-8 prefill:9-"),
    (nk(2048, 512, ptr=8), (False, True), None, "generic:1-8 prefill:9-"),        # not 16-byte aligned
    (kn(2048, 512), (False,), None, "kn:1-1 big_kn:2-256 prefill:257-"),           # N <= K
    (kn(512, 2048), (False,), None, "kn:1-2 big_kn:3-256 prefill:257-"),           # N > K
    (kn(2048, 512), (True,), None, "kn:1-8 big_kn:9-256 prefill:257-"),
    (kn(512, 2048), (True,), None, "kn:1-8 big_kn:9-256 prefill:257-"),
    (kn(2048, 512), (False, True), True, "big_kn:1-"),
    (kn(2048, 512), (False, True), False, "kn:1-8 kn_mfma:9-64 prefill:65-"),
    (kn(2056, 512), (False, True), None, "kn:1-16 prefill:17-"),                  # K % 32 != 0
    (kn(2056, 512), (False, True), True, "kn:1-16 prefill:17-"),
    ((512, 1, 256, 2048, 510), (False,), None, "generic:1-1 big_kn:2-256 prefill:257-"),   # N % 4 != 0
    ((3000, 2, 256, 2048, 512), (False, True), None, "generic:1-8 prefill:9-"),    # no unit stride
    # lm_head-sized (K,N) codes: K * ldk >= 2^29 words is past the fused kernel's 2 GiB record,
    # so it stays on the (K,N) row kernel, then the decode + GEMM
    (kn(8192, 128256), (False,), None, "kn:1-16 prefill:17-"),
    (kn(8192, 128256), (False, True), True, "kn:1-16 prefill:17-"),
    (kn(8192, 128256), (False, True), False, "kn:1-8 kn_mfma:9-64 prefill:65-"),
]


@pytest.mark.parametrize("storage,plugs_,fused,spec", QUAD_TABLE)
def test_quad_route_cells(storage, plugs_, fused, spec):
    c_sk, c_sn, ptr, K, N = storage
    for plug in plugs_:
        caps = routes.quad_storage(c_sk, c_sn, ptr, K, N, 10 if plug else 0)
        expect(routes.quad_route, caps, K, N, plug, fused, spec)


def dkn(K, N, ptr=256):
    return dict(c_sk=N, c_sn=1, ptr=ptr, K=K, N=N, layout="i16", group_size=32, chunk_size=0, elem_base=0)


def dnk(K, N, ptr=256, elem_base=0):
    return dict(c_sk=1, c_sn=K, ptr=ptr, K=K, N=N, layout="u16be", group_size=32, chunk_size=50_000_000,
                elem_base=elem_base)


DUAL_TABLE = [
    (dkn(2048, 512), (False,), None, "dual_kn:1-1 dual_mfma:2-128 prefill:129-"),
    (dkn(2048, 520), (False,), None, "dual_kn:1-1 dual_mfma:2-64 prefill:65-"),      # N % 16 != 0
    (dkn(2048, 512), (True,), None, "dual_kn:1-4 dual_mfma:5-64 prefill:65-"),
    (dkn(512, 2048), (False,), None, "dual_kn:1-4 dual_mfma:5-128 prefill:129-"),
    (dkn(512, 2048), (True,), None, "dual_kn:1-4 dual_mfma:5-64 prefill:65-"),
    (dkn(2048, 512), (False, True), True, "dual_mfma:1-"),
    (dkn(2048, 512), (False, True), False, "dual_kn:1-8 prefill:9-"),
    (dict(dkn(2048, 512), layout="u16be"), (False, True), None, "dual_kn:1-8 prefill:9-"),
    (dkn(2056, 512), (False, True), None, "dual_kn:1-8 prefill:9-"),            # K % 32 != 0
    (dnk(2048, 512), (False, True), None, "dual_nk_mfma:1-64 prefill:65-"),     # .dualpack rows, N <= K
    (dnk(512, 2048), (False, True), None, "dual_rows:1-2 dual_nk_mfma:3-64 prefill:65-"),   # N > K
    (dnk(2048, 512), (False, True), True, "dual_nk_mfma:1-"),
    (dnk(2048, 512), (False, True), False, "dual_rows:1-4 prefill:5-"),
    (dict(dnk(2048, 512), chunk_size=24), (False, True), None, "dual_rows:1-4 prefill:5-"),   # chunks < 32 pairs
    (dnk(2056, 512), (False, True), None, "dual_rows:1-4 prefill:5-"),          # K % 32 != 0
    (dnk(2048, 512, elem_base=4), (False, True), None, "generic:1-4 prefill:5-"),
    # K * ldk * 2 >= 2^31 bytes: neither the matrix cores nor the (K,N) kernel address it
    (dkn(16384, 65536), (False, True), None, "generic:1-4 prefill:5-"),
]


@pytest.mark.parametrize("storage,plugs_,fused,spec", DUAL_TABLE)
def test_dual_route_cells(storage, plugs_, fused, spec):
    s = dict(storage)
    K, N = s["K"], s["N"]
    for plug in plugs_:
        caps = routes.dual_storage(s["c_sk"], s["c_sn"], s["ptr"], K, N, s["layout"], s["group_size"],
                                   s["chunk_size"], s["elem_base"], 10 if plug else 0)
        expect(routes.dual_route, caps, K, N, plug, fused, spec)


def test_routes_have_a_catch_all():
    for table in (routes.QUAD_ROUTES, routes.DUAL_ROUTES):
        last = table[-1]
        assert last.kernel == "prefill" and last.m_lo == 1 and last.m_hi == INF
        assert last.plug == routes.ANY_PLUG and last.fused == routes.ANY_FUSED


QUAD_C = {nat.PP_GEMM_ROWS: "rows", nat.PP_GEMM_KN: "kn", nat.PP_GEMM_GENERIC: "generic"}


def test_quad_storage_matches_the_library():
    """Where the table names rows / kn / generic, pp_quad_gemm runs that kernel (the C library's
    own choice, asked without device work); contiguous activations, as the operator passes."""
    L = nat.lib()
    n = 0
    for K in (32, 40, 64, 2048, 2050, 2056):
        for N in (1, 6, 96, 512):
            for ptr in (256, 260, 264):
                for c_sk, c_sn in ((1, K), (1, K + 4), (1, K + 1), (N, 1), (N + 4, 1), (N + 2, 1), (3 * N + 8, 2)):
                    caps = routes.quad_storage(c_sk, c_sn, ptr, K, N)
                    for M in (1, 3, 8, 16):
                        r = routes.quad_route(M, K, N, caps, False)
                        if r not in QUAD_C.values():
                            continue
                        mm = min(M, 8)
                        got = L.pp_quad_gemm_kernel(4096, K, 1, ptr, c_sk, c_sn, mm, N, K)
                        assert QUAD_C[got] == r, (K, N, ptr, c_sk, c_sn, M, r, got)
                        n += 1
    assert n > 500


DUAL_C = {nat.PP_GEMM_ROWS: "dual_rows", nat.PP_GEMM_KN: "dual_kn", nat.PP_GEMM_GENERIC: "generic"}


def test_dual_storage_matches_the_library():
    L = nat.lib()
    n = 0
    for K in (64, 96, 2048, 2056, 2052):
        for N in (8, 96, 512, 500):
            for ptr in (256, 264):
                for c_sk, c_sn, chunk, base in ((1, K, 4096, 0), (1, K + 8, 4096, 8), (1, K, 4096, 4), (1, K, 0, 0),
                                                (N, 1, 0, 0), (N + 8, 1, 0, 0), (N + 4, 1, 0, 0), (N, 1, 4096, 0)):
                    caps = routes.dual_storage(c_sk, c_sn, ptr, K, N, "i16", 32, chunk, base)
                    for M in (1, 3, 4, 8):
                        r = routes.dual_route(M, K, N, caps, False, fused=False)
                        if r not in DUAL_C.values():
                            continue
                        got = L.pp_dual_gemm_kernel(4096, K, 1, ptr, c_sk, c_sn, 32, chunk, base, M, N, K)
                        assert DUAL_C[got] == r, (K, N, ptr, c_sk, c_sn, chunk, base, M, r, got)
                        n += 1
    assert n > 300


def _u32(a):
    return torch.from_numpy(np.asarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


def test_plug_table_sorted_with_values():
    rng = np.random.default_rng(3)
    pos = rng.choice(1 << 32, 500, replace=False).astype(np.uint32)
    vals = rng.standard_normal((500, 4)).astype(np.float16)
    idx_t, vals_t = _u32(pos), torch.from_numpy(vals)
    si, sv = plugs.ascending(idx_t, vals_t)
    order = np.argsort(pos, kind="stable")
    np.testing.assert_array_equal(si.view(torch.int32).numpy().view(np.uint32), pos[order])
    np.testing.assert_array_equal(sv.numpy(), vals[order])
    assert si.dtype == torch.uint32
    # cached: the same objects come back; an in-place change makes a new sorted copy
    assert plugs.ascending(idx_t, vals_t)[0] is si
    vals_t[0] = 7.0
    si2, sv2 = plugs.ascending(idx_t, vals_t)
    assert si2 is not si and float(sv2[int(np.where(order == 0)[0][0]), 0]) == 7.0


def test_plug_table_duplicates_keep_the_last():
    """Duplicate positions: the last entry in the caller's order stays (the reference's
    fancy-indexed store, quaternion_packer.py:187-193), the others move to 0xFFFFFFFF."""
    pos = np.array([40, 7, 40, 3, 7, 40], np.uint32)
    amp = np.arange(6, dtype=np.float16)
    idx = torch.from_numpy(pos.view(np.int32))                          # int32 holding uint32 bits
    si, sv = plugs.ascending(idx, torch.from_numpy(amp))
    got = si.numpy().view(np.uint32)
    np.testing.assert_array_equal(got, [3, 7, 40, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF])
    np.testing.assert_array_equal(sv.numpy()[:3], [3, 4, 5])
    assert si.dtype == torch.int32


def test_stream_planning_rejects_an_unsorted_table():
    from polar_pack_amd.container import QuadPackDevice
    p = QuadPackDevice(n=100, s=(1.0,) * 4, r_max=1.0, codes=torch.zeros(100, dtype=torch.int32),
                       plug_idx=_u32([5, 3, 9]), plug_vals=torch.zeros((3, 4), dtype=torch.float16), tails=[])
    with pytest.raises(ValueError, match="ascending"):
        p.plug_host()
