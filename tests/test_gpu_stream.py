"""GPU parity of the one-launch stream decode (pp_quad_stream) on .quadpack files."""
import numpy as np
import pytest
import torch

from polar_pack_amd import _native as nat

import gen
from oracle import quadpack as oqp
from parity import assert_gemv_close
from polar_pack_amd import quad_kernels as qk
from polar_pack_amd.container import QuadPackFile
from polar_pack_amd.packer import pack_quad_device
from polar_pack_amd.stream import QuadStream

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# (N, K) projections in stream order; the last one reaches into the FP16 tails
SHAPES = [(64, 256), (8, 2048), (16, 4096), (40, 1024), (24, 11008), (3, 12), (12, 512)]


def make_file(tmp_path, tails, seed=1, threshold=0.006):
    n = sum(nn * k for nn, k in SHAPES[:-1]) + 5 * 512 + 100     # row 5 of the last projection straddles n
    models = gen.correlated_models(seed, [n + t for t in tails])
    qp = oqp.pack_quad(models, threshold=threshold)
    path = tmp_path / "s.quadpack"
    path.write_bytes(qp.to_bytes())
    return qp, path


def oracle_outputs(qp, xs):
    outs = []
    pos = 0
    for (N, K), x in zip(SHAPES, xs):
        W = oqp.unpack_quad_f64(qp, pos, pos + N * K)
        per = []
        for k in range(4):
            w = W[k].reshape(N, K)
            first_missing = np.isnan(w[:, 0])
            y = x.astype(np.float64) @ np.nan_to_num(w, nan=0.0).T
            y[:, first_missing] = 0.0
            per.append(y)
        outs.append(per)
        pos += N * K
    return outs


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_stream_matches_oracle_with_plug_and_tails(tmp_path, M, split):
    tails = (0, 12 * 512 - 5 * 512 - 100 + 7, 1000, 12 * 512 - 5 * 512 - 100)
    qp, path = make_file(tmp_path, tails)
    f = QuadPackFile.read(path)
    assert f.n == qp.n and f.plug_idx.size == qp.plug_idx.size > 0
    pack = f.to_device(DEV)
    st = QuadStream(pack, SHAPES, M=M, split=split)
    assert st.split == split                      # few tasks per wavefront: the planner splits
    xs_np = [np.random.default_rng(100 + p).standard_normal((M, k)).astype(np.float16) for p, (_, k) in enumerate(SHAPES)]
    xs = [torch.from_numpy(x).to(DEV) for x in xs_np]
    outs = [[torch.full((M, n), float("nan"), dtype=torch.float16, device=DEV) for _ in range(4)] for n, _ in SHAPES]
    st.bind(xs, outs)
    ref = oracle_outputs(qp, xs_np)
    for rep in range(2):                          # launches are repeatable
        st()
        torch.cuda.synchronize()
        for p in range(len(SHAPES)):
            for k in range(4):
                assert_gemv_close(outs[p][k].float().cpu().numpy(), ref[p][k], f"rep {rep} proj {p} model {k}")


def test_stream_equals_single_calls_and_device_pack():
    """Device-packed stream (norm plug selection): the one-launch decode equals per-projection calls."""
    shapes = [(128, 2048), (32, 2048), (64, 11008), (256, 512)]
    g = torch.Generator(device=DEV).manual_seed(3)
    models = [[], [], [], []]
    for n, k in shapes:
        w0 = torch.randn(n * k, generator=g, device=DEV) * 0.02
        for m in range(4):
            models[m].append((w0 + torch.randn(n * k, generator=g, device=DEV) * 0.002 * (m + 1)).to(torch.float16))
    pack = pack_quad_device(models, plug_cap=0.001, select="norm")
    assert abs(pack.plug_idx.numel() / pack.n - 0.001) < 0.0005
    st = QuadStream(pack, shapes, M=1)
    xs, outs = st.make_buffers()
    for x in xs:
        x.normal_()
    st.bind(xs, outs)
    st()
    torch.cuda.synchronize()
    pos = 0
    luts = qk.header_luts(pack.r_max, device=DEV)
    for p, (n, k) in enumerate(shapes):
        codes = pack.codes[pos:pos + n * k].reshape(n, k).t()
        single = qk.quad_bitpacked(xs[p], codes, luts, list(pack.s), plug=(pack.plug_idx, pack.plug_vals),
                                   elem_base=pos)
        for m in range(4):
            a = outs[p][m].float().cpu().numpy()
            b = single[m].float().cpu().numpy()
            assert_gemv_close(a, b, f"proj {p} model {m}", rtol=2e-3)
        pos += n * k


def test_container_file_round_trip_and_validation(tmp_path):
    qp, path = make_file(tmp_path, (0, 0, 0, 0))
    f = QuadPackFile.read(path)
    out = tmp_path / "copy.quadpack"
    f.write(out)
    assert out.read_bytes() == path.read_bytes()
    bad = tmp_path / "short.quadpack"
    bad.write_bytes(path.read_bytes()[:-3])
    with pytest.raises(ValueError, match="shorter|implies"):
        QuadPackFile.read(bad)


@pytest.mark.parametrize("one_linear", [True, False])
@pytest.mark.parametrize("shape", [(256, 2048), (64, 11008), (600, 4100), (512, 1536)])
@pytest.mark.parametrize("M", [1, 2, 8])
def test_single_linear_split_k(shape, M, one_linear):
    """One projection, its tasks cut into column slices that meet in the workspace or, when
    a workgroup holds a task's slices, in LDS (K not
    a multiple of the 512-column chunk, slices of unequal block counts), on the one-Linear
    launch (pp_quad_rows) and on the segment plan: equal to the oracle, on repeated
    launches, and the workspace is left zero."""
    N, K = shape
    models = gen.correlated_models(7, [N * K] * 4)
    qp = oqp.pack_quad(models, threshold=0.004)
    pack = QuadPackFile(n=qp.n, s=qp.s, r_max=qp.r_max, codes=qp.codes, plug_idx=qp.plug_idx,
                        plug_vals=qp.plug_vals).to_device(DEV)
    st = QuadStream(pack, [shape], M=M, one_linear=one_linear)
    ws_bytes = int(nat.lib().pp_quad_rows_workspace_size(M, N, K))
    # slices meeting in the workspace at one token: the segment plan; in LDS: the one-Linear launch
    assert st.direct == (one_linear and (M > 1 or ws_bytes == 0))
    assert st.split and (st.workspace is not None or (st.direct and ws_bytes == 0))
    x_np = np.random.default_rng(5).standard_normal((M, K)).astype(np.float16)
    xs = [torch.from_numpy(x_np).to(DEV)]
    outs = [[torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV) for _ in range(4)]]
    st.bind(xs, outs)
    W = oqp.unpack_quad_f64(qp, 0, N * K)
    for rep in range(3):
        st()
        torch.cuda.synchronize()
        for m in range(4):
            ref = x_np.astype(np.float64) @ W[m].reshape(N, K).T
            assert_gemv_close(outs[0][m].float().cpu().numpy(), ref, f"rep {rep} model {m}")
        if st.workspace is not None:
            assert int(torch.count_nonzero(st.workspace)) == 0



def test_plug_side_table(tmp_path):
    """pp_quad_plug_codes: each plug entry's code word (0 for an entry past n)."""
    qp, path = make_file(tmp_path, tails=(0, 12 * 512 - 5 * 512 - 100, 0, 7))
    pack = QuadPackFile.read(path).to_device(DEV)
    assert qp.plug_idx.size > 0
    st = QuadStream(pack, SHAPES, M=1)
    want = qp.codes[qp.plug_idx.astype(np.int64)]
    got = st.plug_code.cpu().numpy().view(np.uint32)[:want.size]
    np.testing.assert_array_equal(got, want)
