"""pp_quad_gemm_noalloc (the entry point for callers that cannot allocate) against
pp_quad_gemm with a caller workspace, through the C ABI, on consecutive calls (the second
smaller, so it runs over what the first left in the library's scratch array)."""
import ctypes as C

import numpy as np
import pytest
import torch

from parity import assert_gemv_close
from polar_pack_amd import _native as nat
from polar_pack_amd import quad_kernels as qk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _codes(shape, seed):
    rng = np.random.default_rng(seed)
    c = rng.integers(0, 2 ** 32, size=shape, dtype=np.uint64).astype(np.uint32)
    return torch.from_numpy(c.view(np.int32)).to(DEV)


def _case(layout, K, N, M, plug, seed):
    """Operands of one call: (K,N) codes contiguous ('kn'), (N,K) rows seen as (K,N) ('nk'),
    or a strided (K,N) view ('generic'), with plug entries at sorted storage offsets."""
    rng = np.random.default_rng(seed)
    if layout == "kn":
        store = _codes((K, N), seed)
        c_sk, c_sn, span = N, 1, K * N
    elif layout == "nk":
        store = _codes((N, K), seed)
        c_sk, c_sn, span = 1, K, K * N
    else:
        store = _codes((K, 2 * N), seed)
        c_sk, c_sn, span = 2 * N, 2, 2 * K * N
    pos = np.sort(rng.choice(span, plug, replace=False)).astype(np.int64)
    if layout == "generic":
        pos = pos[pos % 2 == 0]
    idx = torch.from_numpy(pos.astype(np.uint32).view(np.int32)).to(DEV)
    vals = torch.from_numpy((rng.standard_normal((pos.size, 4)) * 0.5).astype(np.float16)).to(DEV)
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(DEV)
    luts = [t.to(DEV) for t in qk.header_luts(7.0 + seed % 3)]
    return dict(a=a, store=store, c_sk=c_sk, c_sn=c_sn, idx=idx, vals=vals, luts=luts, M=M, N=N, K=K,
                scales=[0.02, 0.021, 0.019, 0.0205])


def _call(cs, noalloc):
    L = nat.lib()
    outs = [torch.full((cs["M"], cs["N"]), float("nan"), dtype=torch.float16, device=DEV) for _ in range(4)]
    a = cs["a"]
    lut_ptrs = nat.ptr_array([t.data_ptr() for t in cs["luts"]])
    sc = nat.float_array(cs["scales"])
    out_ptrs = nat.ptr_array([o.data_ptr() for o in outs])
    P = int(cs["idx"].numel())
    common = (a.data_ptr(), a.stride(0), a.stride(1), cs["store"].data_ptr(), cs["c_sk"], cs["c_sn"], lut_ptrs,
              nat.PP_F32, sc, cs["idx"].data_ptr() if P else None, cs["vals"].data_ptr() if P else None, P, 0,
              out_ptrs, outs[0].stride(0), outs[0].stride(1), cs["M"], cs["N"], cs["K"])
    stream = torch.cuda.current_stream(DEV).cuda_stream
    if noalloc:
        rc = L.pp_quad_gemm_noalloc(*common, stream)
        ws = None
    else:
        need = L.pp_quad_gemm_workspace_size(a.data_ptr(), a.stride(0), a.stride(1), cs["store"].data_ptr(),
                                             cs["c_sk"], cs["c_sn"], P, cs["M"], cs["N"], cs["K"])
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
        rc = L.pp_quad_gemm(*common, ws.data_ptr() if need else None, need, stream)
    nat.check(rc, "pp_quad_gemm_noalloc" if noalloc else "pp_quad_gemm")
    torch.cuda.synchronize()
    return [o.float().cpu().numpy() for o in outs], ws


PAIRS = [  # (first call, second smaller call): the scratch array holds the first call's data
    (("kn", 2048, 1024, 4, 300), ("kn", 512, 256, 1, 40)),
    (("kn", 4096, 512, 8, 0), ("kn", 1024, 64, 3, 9)),
    (("nk", 2048, 2048, 1, 500), ("nk", 1024, 256, 2, 30)),
    (("generic", 96, 64, 3, 0), ("generic", 32, 16, 1, 0)),     # no plug: it needs a unit stride
]


@pytest.mark.parametrize("first,second", PAIRS, ids=[p[0][0] for p in PAIRS])
def test_noalloc_matches_the_workspace_entry_point(first, second):
    for spec, seed in ((first, 1), (second, 2)):
        cs = _case(*spec, seed=seed)
        got, _ = _call(cs, noalloc=True)
        ref, _ = _call(cs, noalloc=False)
        for m in range(4):
            assert np.isfinite(got[m]).all()
            assert_gemv_close(got[m], ref[m], f"{spec} model {m}")


def test_noalloc_rejects_calls_beyond_its_scratch():
    L = nat.lib()
    K, N = 4096, 2048                      # generic strided layout: 4*K*N floats = 128 MiB of workspace
    cs = _case("generic", K, N, 1, 0, seed=3)
    a = cs["a"]
    need = L.pp_quad_gemm_workspace_size(a.data_ptr(), a.stride(0), a.stride(1), cs["store"].data_ptr(), cs["c_sk"],
                                         cs["c_sn"], 0, 1, N, K)
    assert need > (64 << 20)
    outs = [torch.zeros((1, N), dtype=torch.float16, device=DEV) for _ in range(4)]
    rc = L.pp_quad_gemm_noalloc(a.data_ptr(), a.stride(0), a.stride(1), cs["store"].data_ptr(), cs["c_sk"],
                                cs["c_sn"], nat.ptr_array([t.data_ptr() for t in cs["luts"]]), nat.PP_F32,
                                nat.float_array(cs["scales"]), None, None, 0, 0,
                                nat.ptr_array([o.data_ptr() for o in outs]), N, 1, 1, N, K,
                                torch.cuda.current_stream(DEV).cuda_stream)
    assert rc == nat.PP_EINVAL
    assert "scratch" in L.pp_last_error().decode()
    torch.cuda.synchronize()
    assert all(float(o.abs().sum()) == 0 for o in outs)     # nothing was launched
