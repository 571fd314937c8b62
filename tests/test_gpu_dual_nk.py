"""GPU parity of the matrix-core dual decode over .dualpack container rows (pp_dual_nk_mfma:
5-64 tokens by default, any size with ``fused=True``) against the float64 oracle
(oracle.dualpack.decode_pairs_f64, the restatement of unpack_dual_models,
polar_bitpack.py:228-247): weights rounded to fp16 before the product, as the reference's
kernel rounds them (polar_kernels.py:78-82), so the outputs are held to the fp16-weight
bound and normwise 1e-3 of the exact products."""
import numpy as np
import pytest
import torch

import gen
from oracle import dualpack as odp
from oracle import layer as olay
from parity import assert_gemv_close, fp16_weight_bound, normwise
from polar_pack_amd import _native as nat
from polar_pack_amd import polar_kernels as pk
from test_gpu_dual import be_codes_tensor

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


def pack(n1, n2, seed, cap, chunk, gs=32):
    w1, w2 = gen.correlated_models(seed, [n1, n2], delta_growth=False)
    return odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=cap, chunk_size=chunk, group_size=gs))


def run(dp, pos, N, K, M, fused=None, shuffle=False, seed=0):
    """Projection (N,K) at stream position pos through the drop-in operator; returns the
    route, the outputs and the float64 weights (N,K) of both models."""
    amp, cs, sn = pk.header_luts(mu=dp.mu, device=DEV)
    view = be_codes_tensor(dp)[pos:pos + N * K].reshape(N, K).t()
    scales = torch.from_numpy(dp.scales).to(DEV)
    order = np.random.default_rng(seed).permutation(dp.plug_idx.size) if shuffle else np.arange(dp.plug_idx.size)
    plug = (u32(dp.plug_idx[order]).to(DEV), torch.from_numpy(dp.plug_val[order]).to(DEV))
    route = pk.dual_call_route(view, M, layout="u16be", group_size=dp.group_size, chunk_size=dp.chunk_size,
                               elem_base=pos, plug_n=dp.plug_idx.size, fused=fused)
    a = np.random.default_rng(seed + M).standard_normal((M, K)).astype(np.float16)
    o1, o2 = pk.polar_dual_bitpacked(torch.from_numpy(a).to(DEV), view, scales, amp, cs, sn, layout="u16be",
                                     group_size=dp.group_size, chunk_size=dp.chunk_size, elem_base=pos, plug=plug,
                                     fused=fused)
    d1, d2 = odp.decode_pairs_f64(dp, pos, pos + N * K)
    return route, a, (o1, o2), (d1.reshape(N, K), d2.reshape(N, K))


def check(a, outs, ws, what):
    for m, (o, w) in enumerate(zip(outs, ws)):
        exact = olay.gemm_f64(a, w.T)
        got = o.float().cpu().numpy()
        assert_gemv_close(got, exact, f"{what} model {m}", bound=fp16_weight_bound(a, w.T))
        assert normwise(got, exact) <= 1e-3, f"{what} model {m}: normwise {normwise(got, exact):.2e}"


@pytest.mark.parametrize("M", [5, 8, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("N,K,chunk,gs,cap", [(96, 512, 4096, 32, 0.02), (70, 1024, 1000, 64, 0.03),
                                              (33, 256, 50_000_000, 32, 0.0), (128, 2048, 2048, 8, 0.01)])
def test_container_rows_match_oracle(N, K, chunk, gs, cap, M):
    """Rows crossing chunk boundaries (chunks of 1000 and 4096 pairs; group scales restart at
    each), 8- to 64-pair groups, N not a multiple of 16, plug tables of 0-3 % of pairs, and the
    K slices the plan gives for these sizes (2-4 tokens tiles of 16)."""
    dp = pack(N * K + 900, N * K + 300, 100 + N + M, cap, chunk, gs)
    route, a, outs, ws = run(dp, 0, N, K, M)
    assert route == "dual_nk_mfma", route
    check(a, outs, ws, f"N={N} K={K} chunk={chunk} gs={gs} M={M}")


@pytest.mark.parametrize("M", [12, 40])
def test_second_projection_mid_stream_shuffled_plug(M):
    """A projection that starts mid-stream (elem_base 56,008: stream positions, chunk
    offsets and plug positions all shifted), plug table passed in shuffled order."""
    N1, N, K = 70, 48, 800
    pos = N1 * K + 8
    dp = pack(pos + N * K + 64, pos + N * K, 7, 0.03, 3000)
    route, a, outs, ws = run(dp, pos, N, K, M, shuffle=True, seed=3)
    assert route == "dual_nk_mfma", route
    check(a, outs, ws, f"mid-stream M={M}")


@pytest.mark.parametrize("M", [1, 3, 65, 128, 300])
def test_fused_switch_any_size(M):
    """fused=True takes the container-row matrix-core decode at any token count."""
    N, K = 80, 512
    dp = pack(N * K, N * K, 11, 0.02, 4096)
    route, a, outs, ws = run(dp, 0, N, K, M, fused=True)
    assert route == "dual_nk_mfma", route
    check(a, outs, ws, f"fused M={M}")


def test_workspace_left_zero_and_repeatable():
    """A sliced launch through the C-ABI twice in a row: the same outputs, the float32
    workspace left zero after each."""
    N, K, M = 64, 4096, 16
    dp = pack(N * K, N * K, 21, 0.01, 8192)
    amp, cs, sn = pk.header_luts(mu=dp.mu, device=DEV)
    codes = be_codes_tensor(dp)[:N * K]
    scales = torch.from_numpy(dp.scales).to(DEV)
    idx, val = u32(dp.plug_idx).to(DEV), torch.from_numpy(dp.plug_val).to(DEV)
    L = nat.lib()
    slices, cols = 4, 1024
    row_plug = nat.plug_search(idx, idx.numel(), 0, K, N, slices, cols, DEV)
    ws_bytes = L.pp_dual_mfma_workspace_size(M, N, slices)
    assert ws_bytes > 0
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
    a = torch.from_numpy(np.random.default_rng(5).standard_normal((M, K)).astype(np.float16)).to(DEV)
    res = []
    for rep in range(2):
        o1, o2 = (torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV) for _ in range(2))
        rc = L.pp_dual_nk_mfma(codes.data_ptr(), nat.PP_DUAL_U16_BE, K, 0, a.data_ptr(), K, scales.data_ptr(),
                               scales.numel(), dp.group_size, dp.chunk_size, amp.data_ptr(), amp.numel(),
                               cs.data_ptr(), sn.data_ptr(), cs.numel(), nat.PP_F32, idx.data_ptr(), val.data_ptr(),
                               idx.numel(), row_plug.data_ptr(), slices, cols, o1.data_ptr(), o2.data_ptr(), N, M, N,
                               K, ws.data_ptr(), ws_bytes, torch.cuda.current_stream(DEV).cuda_stream)
        nat.check(rc, "pp_dual_nk_mfma")
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(ws)) == 0, "the workspace is not left zero"
        res.append((o1.float().cpu().numpy(), o2.float().cpu().numpy()))
    d1, d2 = odp.decode_pairs_f64(dp, 0, N * K)
    check(a.cpu().numpy(), [torch.from_numpy(r) for r in res[0]], (d1.reshape(N, K), d2.reshape(N, K)), "C-ABI")
    for m in range(2):
        np.testing.assert_allclose(res[1][m], res[0][m], rtol=2e-3, atol=2e-3)


def test_rejects_unaligned_rows():
    """Rows not a multiple of 8 pairs apart: the entry point refuses them."""
    L = nat.lib()
    z = torch.zeros(64, dtype=torch.uint8, device=DEV)
    rc = L.pp_dual_nk_mfma(z.data_ptr(), nat.PP_DUAL_U16_BE, 36, 0, z.data_ptr(), 32, z.data_ptr(), 1, 32, 4096,
                           z.data_ptr(), 64, z.data_ptr(), z.data_ptr(), 1024, nat.PP_F32, None, None, 0, None, 1, 64,
                           z.data_ptr(), z.data_ptr(), 4, 1, 4, 32, None, 0, None)
    assert rc != 0
