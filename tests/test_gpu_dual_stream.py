"""GPU parity of the one-launch dual stream decode (pp_dual_stream) against the float64 oracle."""
import numpy as np
import pytest
import torch

import gen
from oracle import dualpack as odp
from parity import assert_gemv_close
from polar_pack_amd.container import DualPackDevice, DualPackFile
from polar_pack_amd.stream import DualStream

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# (N, K) projections in stream order, K % 8 == 0; rows of 2048-11008 pairs and short ones
SHAPES = [(24, 1024), (8, 2048), (16, 4096), (40, 512), (12, 11008), (3, 16), (9, 520)]
TOTAL = sum(n * k for n, k in SHAPES)


def oracle_pairs(dp, tails=None):
    """float64 (w1, w2) over the whole stream: codes below dp.n_pairs, tails after."""
    w1, w2 = odp.decode_pairs_f64(dp, 0, dp.n_pairs)
    if tails is not None:
        t1, t2 = tails
        w1 = np.concatenate([w1, t1.astype(np.float64), np.full(TOTAL, np.nan)])[:TOTAL]
        w2 = np.concatenate([w2, t2.astype(np.float64), np.full(TOTAL, np.nan)])[:TOTAL]
    return w1, w2


def oracle_outputs(w, xs, shapes=SHAPES):
    outs, pos = [], 0
    for (N, K), x in zip(shapes, xs):
        per = []
        for m in range(2):
            wm = w[m][pos:pos + N * K].reshape(N, K)
            missing = np.isnan(wm[:, 0])                 # a model without the row reads 0
            y = x.astype(np.float64) @ np.nan_to_num(wm, nan=0.0).T
            y[:, missing] = 0.0
            per.append(y)
        outs.append(per)
        pos += N * K
    return outs


def to_i16(codes_be_u8):
    """File layout -> int16 kernel layout (code - 32768)."""
    code = odp.from_be_bytes(codes_be_u8).astype(np.uint16)
    return (code ^ np.uint16(0x8000)).view(np.int16)


def device_pack(dp, layout, tails=None, n_codes=None):
    f = DualPackFile(n_pairs=dp.n_pairs, n1=dp.n1, n2=dp.n2, codes_be=dp.codes_be, scales=dp.scales,
                     plug_idx=dp.plug_idx, plug_val=dp.plug_val, amp_bits=dp.amp_bits, phase_bits=dp.phase_bits,
                     mu=dp.mu, group_size=dp.group_size, chunk_size=dp.chunk_size)
    pack = f.to_device(DEV)
    if layout == "i16":
        pack.codes = torch.from_numpy(to_i16(dp.codes_be)).to(DEV)
        pack.layout = "i16"
    if tails is not None:
        pack.tails = [torch.from_numpy(np.ascontiguousarray(t)).to(DEV) for t in tails]
    return pack


def run_stream(pack, M, seed=5, plug_windows=None, split=True):
    st = DualStream(pack, SHAPES, M=M, plug_windows=plug_windows, split=split)
    # these streams hold few row tasks, so split=True cuts the K > 512 projections into slices
    assert st.split == split
    xs_np = [np.random.default_rng(seed + p).standard_normal((M, k)).astype(np.float16)
             for p, (_, k) in enumerate(SHAPES)]
    xs = [torch.from_numpy(x).to(DEV) for x in xs_np]
    outs = [[torch.full((M, n), float("nan"), dtype=torch.float16, device=DEV) for _ in range(2)] for n, _ in SHAPES]
    st.bind(xs, outs)
    return st, xs_np, outs


@pytest.mark.parametrize("layout", ["u16be", "i16"])
@pytest.mark.parametrize("chunk", [50_000_000, 1000])     # groups aligned / restarting mid-group
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("split", [False, True])
def test_dual_stream_zero_padded_file(layout, chunk, M, split):
    """The .dualpack format itself: model 2 shorter and zero-padded, plug cap 3%."""
    w1, w2 = gen.correlated_models(11, [TOTAL, TOTAL - 3000], delta_growth=False)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=0.03, chunk_size=chunk))
    assert dp.plug_idx.size > 0
    pack = device_pack(dp, layout)
    st, xs_np, outs = run_stream(pack, M, split=split)
    ref = oracle_outputs(oracle_pairs(dp), xs_np)
    for rep in range(2):
        st()
        torch.cuda.synchronize()
        for p in range(len(SHAPES)):
            for m in range(2):
                assert_gemv_close(outs[p][m].float().cpu().numpy(), ref[p][m], f"rep {rep} proj {p} model {m}")
        if st.workspace is not None:
            assert int(torch.count_nonzero(st.workspace)) == 0


@pytest.mark.parametrize("layout", ["u16be", "i16"])
def test_dual_stream_fp16_tails(layout):
    """Tail mode: codes cover the shorter model's length; model 1's rest is fp16 tail, model
    2 has no weights there (rows past its end read 0, the straddling row its prefix)."""
    n2 = TOTAL - 9 * 520 + 100          # the last projection's row 0 straddles n2
    w1, w2 = gen.correlated_models(13, [TOTAL, n2], delta_growth=False)
    dp = odp.pack_dual(w1[:n2], w2, odp.DualConfig(plug_cap=0.01, chunk_size=50_000_000))
    t1 = np.asarray(w1[n2:], np.float32).astype(np.float16)
    t2 = np.zeros(0, np.float16)
    pack = device_pack(dp, layout, tails=(t1, t2))
    st, xs_np, outs = run_stream(pack, 1)
    assert st.n_tail == 9
    ref = oracle_outputs(oracle_pairs(dp, tails=(t1, t2)), xs_np)
    st()
    torch.cuda.synchronize()
    for p in range(len(SHAPES)):
        for m in range(2):
            assert_gemv_close(outs[p][m].float().cpu().numpy(), ref[p][m], f"proj {p} model {m}")


@pytest.mark.parametrize("plug_windows", [1, 2])
@pytest.mark.parametrize("cap,M", [(0.2, 1), (0.2, 4), (0.03, 1), (0.03, 2)])
@pytest.mark.parametrize("split", [False, True])
def test_dual_stream_dense_plug_tasks(plug_windows, cap, M, split):
    """Plug tables dense enough that tasks hold more entries than their steps take
    (64 or 128 per step): the rest is corrected when the task finishes (with column
    slices, each slice walks its task's entries and applies those in its columns)."""
    w1, w2 = gen.correlated_models(17, [TOTAL, TOTAL], delta_growth=False)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=cap, chunk_size=50_000_000))
    pack = device_pack(dp, "u16be")
    st, xs_np, outs = run_stream(pack, M, plug_windows=plug_windows, split=split)
    n_t = st.task_plug_np[:, 1] - st.task_plug_np[:, 0]
    nck = np.array([(-(-SHAPES[p][1] // 512)) for p in np.repeat(np.arange(len(SHAPES)),
                                                                   [-(-n // st.rows_per_item) for n, _ in SHAPES])])
    if cap == 0.2:
        assert np.any(n_t > 64 * plug_windows * nck)          # the finishing path runs
    ref = oracle_outputs(oracle_pairs(dp), xs_np)
    st()
    torch.cuda.synchronize()
    for p in range(len(SHAPES)):
        for m in range(2):
            assert_gemv_close(outs[p][m].float().cpu().numpy(), ref[p][m], f"proj {p} model {m}")


def device_pack_to_oracle(pack):
    """The device pack as an oracle DualPack (codes as file bytes) for decode_pairs_f64."""
    be = pack.codes.cpu().numpy().view(np.uint16)
    if pack.layout == "i16":
        be = (be ^ np.uint16(0x8000)).byteswap()
    return odp.DualPack(n_pairs=pack.n_codes, n1=pack.n_codes, n2=pack.n_codes, codes_be=be.view(np.uint8).copy(),
                        scales=pack.scales.cpu().numpy(), plug_idx=pack.plug_host().copy(),
                        plug_val=pack.plug_val.cpu().numpy(), mu=pack.mu, group_size=pack.group_size,
                        chunk_size=pack.chunk_size)


@pytest.mark.parametrize("chunk", [1000, 50_000_000])
def test_device_packer_on_gpu_matches_oracle_packer(chunk):
    from parity import assert_same_dual_pack
    from polar_pack_amd.packer import pack_dual_device
    w1, w2 = gen.correlated_models(19, [60_000, 57_000], delta_growth=False)
    pack = pack_dual_device(torch.from_numpy(w1).to(DEV), torch.from_numpy(w2).to(DEV), plug_cap=0.03,
                            chunk_size=chunk)
    assert_same_dual_pack(pack, odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=0.03, chunk_size=chunk)))


@pytest.mark.parametrize("layout", ["u16be", "i16"])
def test_device_packed_tail_stream(layout):
    """The benchmark's pipeline at small size: device pack in tail mode (model 2 truncated),
    stream decode, against the float64 decode of the same device pack + its fp16 tail."""
    from polar_pack_amd.packer import pack_dual_device
    n2 = TOTAL - 9 * 520 - 3 * 16 - 12 * 11008 + 2 * 11008 + 40      # inside the 11008-wide projection
    w1, w2 = gen.correlated_models(23, [TOTAL, n2], delta_growth=False)
    pack = pack_dual_device(torch.from_numpy(w1).to(DEV), torch.from_numpy(w2).to(DEV), plug_cap=0.01,
                            select="ref", tails=True, layout=layout)
    assert pack.n_codes == n2 and pack.tail_lengths == [TOTAL - n2, 0]
    st, xs_np, outs = run_stream(pack, 1)
    t1 = pack.tails[0].cpu().numpy()
    ref = oracle_outputs(oracle_pairs(device_pack_to_oracle(pack), tails=(t1, np.zeros(0, np.float16))), xs_np)
    st()
    torch.cuda.synchronize()
    for p in range(len(SHAPES)):
        for m in range(2):
            assert_gemv_close(outs[p][m].float().cpu().numpy(), ref[p][m], f"proj {p} model {m}")


@pytest.mark.parametrize("M", [1, 3])
def test_dual_stream_fp16_tail_rows(M):
    """Aligned tails (n_codes % 8 == 0): rows wholly in a tail take the vectorized fp16
    path, with model 2's tail ending at a row boundary of one projection and inside a
    row of a later one (that row element by element, the rows after it 0 for model 2)."""
    n_codes = 24 * 1024 + 8 * 2048 + 16 * 4096 + 40 * 512 + 2 * 11008        # row 2 of the 12x11008 block
    w1, w2 = gen.correlated_models(29, [TOTAL, TOTAL], delta_growth=False)
    dp = odp.pack_dual(w1[:n_codes], w2[:n_codes], odp.DualConfig(plug_cap=0.03, chunk_size=50_000_000))
    t1 = np.asarray(w1[n_codes:], np.float32).astype(np.float16)
    t2 = np.asarray(w2[n_codes:n_codes + 7 * 11008 + 500], np.float32).astype(np.float16)
    pack = device_pack(dp, "i16", tails=(t1, t2))
    st, xs_np, outs = run_stream(pack, M)
    flags = st.tail_items_np["flags"]
    assert np.any(flags == 2) and np.any(flags == 1) and st.tail_items_np["nrows"].max() == 8
    ref = oracle_outputs(oracle_pairs(dp, tails=(t1, t2)), xs_np)
    st()
    torch.cuda.synchronize()
    for p in range(len(SHAPES)):
        for m in range(2):
            assert_gemv_close(outs[p][m].float().cpu().numpy(), ref[p][m], f"proj {p} model {m}")



@pytest.mark.parametrize("one_linear", [True, False])
@pytest.mark.parametrize("shape", [(256, 2048), (64, 11008), (1000, 1000), (2048, 520)])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_single_linear_split_k(shape, M, one_linear):
    """One projection whose tasks are cut into column slices that meet in the workspace, on
    the one-Linear launch (pp_dual_rows) and on the segment plan: equal to the oracle on
    repeated launches, and the workspace is left zero."""
    N, K = shape
    w1, w2 = gen.correlated_models(19, [N * K, N * K], delta_growth=False)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=0.01, chunk_size=50_000_000))
    pack = device_pack(dp, "i16")
    st = DualStream(pack, [shape], M=M, one_linear=one_linear)
    assert st.direct == one_linear
    # slices when the launch has fewer than half as many row tasks as wavefronts
    assert st.split == (K > 512 and 2 * -(-N // st.rows_per_item) < st.n_waves)
    assert st.workspace is None or st.split
    x_np = np.random.default_rng(23).standard_normal((M, K)).astype(np.float16)
    outs = [[torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV) for _ in range(2)]]
    st.bind([torch.from_numpy(x_np).to(DEV)], outs)
    w = odp.decode_pairs_f64(dp, 0, N * K)
    for rep in range(3):
        st()
        torch.cuda.synchronize()
        for m in range(2):
            ref = x_np.astype(np.float64) @ w[m].reshape(N, K).T
            assert_gemv_close(outs[0][m].float().cpu().numpy(), ref, f"rep {rep} model {m}")
        if st.workspace is not None:
            assert int(torch.count_nonzero(st.workspace)) == 0


@pytest.mark.parametrize("shape,cap", [((256, 2048), 0.01), ((512, 2048), 0.001), ((64, 11008), 0.05),
                                       ((1000, 1000), 0.0)])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_single_linear_task_records(shape, cap, M):
    """The one-Linear launch reading each task's plug records from a block of its own
    (pp_dual_task_entries: the task's records in order, null records after them) and from the
    records' ranges (task_cap 0): equal to the oracle, and to each other bit for bit where no
    column slices meet through atomics."""
    N, K = shape
    w1, w2 = gen.correlated_models(41, [N * K, N * K], delta_growth=False)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=cap, chunk_size=50_000_000))
    pack = device_pack(dp, "u16be")
    st = DualStream(pack, [shape], M=M)
    assert st.direct and st.task_cap >= 1
    P = dp.plug_idx.size
    cnt = st.task_plug_np[:, 1] - st.task_plug_np[:, 0]
    if P:
        assert st.task_cap == cnt.max()
        blk = st.task_ent.cpu().numpy().view(np.uint32).reshape(st.n_tasks, st.task_cap, 2)
        ent = st.plug_ent.cpu().numpy().view(np.uint32).reshape(-1, 2)
        for t in range(st.n_tasks):
            lo, hi = st.task_plug_np[t]
            np.testing.assert_array_equal(blk[t, :hi - lo], ent[lo:hi])
            assert np.all(blk[t, hi - lo:, 0] == 0x7FFFF) and np.all(blk[t, hi - lo:, 1] == 0)
    else:
        assert st.task_ent is None
    x_np = np.random.default_rng(43).standard_normal((M, K)).astype(np.float16)
    outs = [[torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV) for _ in range(2)]]
    st.bind([torch.from_numpy(x_np).to(DEV)], outs)
    w = odp.decode_pairs_f64(dp, 0, N * K)
    got = {}
    for mode, tc in (("blocks", st.task_cap), ("ranges", 0)):
        st.task_cap = tc
        st()
        torch.cuda.synchronize()
        got[mode] = [o.float().cpu().numpy() for o in outs[0]]
        for m in range(2):
            ref = x_np.astype(np.float64) @ w[m].reshape(N, K).T
            assert_gemv_close(got[mode][m], ref, f"{mode} model {m}")
    if st.workspace is None:
        for m in range(2):
            np.testing.assert_array_equal(got["blocks"][m], got["ranges"][m])


@pytest.mark.parametrize("layout", ["u16be", "i16"])
@pytest.mark.parametrize("chunk", [50_000_000, 1000])
def test_plug_records(layout, chunk):
    """pp_dual_plug_table: each entry's column, row in its task and phase, and the float32
    correction d = plug amplitude - amp_lut[aq] * group scale (groups restart every chunk,
    polar_bitpack.py:201-203), rounded once."""
    w1, w2 = gen.correlated_models(31, [TOTAL, TOTAL], delta_growth=False)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=0.03, chunk_size=chunk))
    pack = device_pack(dp, layout)
    st = DualStream(pack, SHAPES, M=1)
    code = odp.from_be_bytes(dp.codes_be).astype(np.uint32)
    p = dp.plug_idx.astype(np.int64)
    g = (p // chunk) * (-(-chunk // dp.group_size)) + (p % chunk) // dp.group_size
    pos0 = np.cumsum([0] + [n * k for n, k in SHAPES])
    proj = np.searchsorted(pos0, p, side="right") - 1
    K = np.array([k for _, k in SHAPES])[proj]
    row, col = (p - pos0[proj]) // K, (p - pos0[proj]) % K
    ent = st.plug_ent.cpu().numpy().view(np.uint32)[:2 * p.size].reshape(-1, 2)
    np.testing.assert_array_equal(ent[:, 0], col | ((row % st.rows_per_item) << 19) | ((code[p] & 0x3FF) << 22))
    amp = st.luts[0].cpu().numpy().astype(np.float64)
    d = dp.plug_val.astype(np.float64) - amp[code[p] >> 10] * dp.scales[g].astype(np.float64)
    np.testing.assert_array_equal(ent[:, 1], d.astype(np.float32).view(np.uint32))


# Projections on which the one-token decode reads the regrouped scales (N % 8 == 0,
# K % 32 == 0, positions multiples of 8 * 32).
SHAPES_T = [(24, 1024), (8, 2048), (16, 4096), (40, 512), (16, 11008), (8, 64)]


def stream_outputs(pack, shapes, M, seed, **kw):
    st = DualStream(pack, shapes, M=M, **kw)
    xs_np = [np.random.default_rng(seed + p).standard_normal((M, k)).astype(np.float16)
             for p, (_, k) in enumerate(shapes)]
    xs = [torch.from_numpy(x).to(DEV) for x in xs_np]
    outs = [[torch.full((M, n), float("nan"), dtype=torch.float16, device=DEV) for _ in range(2)] for n, _ in shapes]
    st.bind(xs, outs)
    st()
    torch.cuda.synchronize()
    return st, xs_np, [[o.float().cpu().numpy() for o in per] for per in outs]


@pytest.mark.parametrize("layout", ["u16be", "i16"])
@pytest.mark.parametrize("chunk", [50_000_000, 4096])     # one chunk; groups restarting every 4096 pairs
@pytest.mark.parametrize("cap", [0.03, 0.2])
@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("M", [1, 2, 3])                  # 8, 4 and 2 rows per task
def test_dual_stream_scale_table(layout, chunk, cap, split, M):
    """Projections that admit the regrouped scales: the decode reads them from
    pp_dual_scale_table's table and matches the oracle, and (without column slices, whose
    float32 partial sums arrive in any order) the same stream reading the scales array bit
    for bit."""
    total = sum(n * k for n, k in SHAPES_T)
    w1, w2 = gen.correlated_models(23, [total, total - 5000], delta_growth=False)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=cap, chunk_size=chunk))
    pack = device_pack(dp, layout)
    st_t, xs_np, got_t = stream_outputs(pack, SHAPES_T, M, 3, split=split)
    st_s, _, got_s = stream_outputs(pack, SHAPES_T, M, 3, split=split, scale_table=False)
    assert st_t.scale_tab is not None and st_s.scale_tab is None
    assert st_t.split == split
    ref = oracle_outputs(oracle_pairs(dp), xs_np, SHAPES_T)
    for p in range(len(SHAPES_T)):
        for m in range(2):
            assert_gemv_close(got_t[p][m], ref[p][m], f"proj {p} model {m}")
            if not split:
                assert np.array_equal(got_t[p][m], got_s[p][m]), f"proj {p} model {m}"


def test_dual_stream_scale_table_not_applicable():
    """Shapes or batches that the regrouped scales do not fit read the scales array; asking
    for the table there is an error."""
    n = sum(n * k for n, k in SHAPES_T) + 1000
    dp = odp.pack_dual(*gen.correlated_models(29, [n, n], delta_growth=False),
                       odp.DualConfig(plug_cap=0.01, chunk_size=50_000_000))
    pack = device_pack(dp, "u16be")
    assert DualStream(pack, SHAPES_T, M=1).scale_tab is not None
    assert DualStream(pack, SHAPES, M=1).scale_tab is None            # N = 3, 9 and K = 16, 520
    assert DualStream(pack, [(26, 1024)], M=2).scale_tab is None      # 26 rows: not whole tasks of 4
    assert DualStream(pack, [(26, 1024)], M=4).scale_tab is not None  # whole tasks of 2
    shifted = [8 + sum(a * b for a, b in SHAPES_T[:i]) for i in range(len(SHAPES_T))]
    assert DualStream(pack, SHAPES_T, M=1, positions=shifted).scale_tab is None
    with pytest.raises(ValueError):
        DualStream(pack, SHAPES, M=1, scale_table=True)


@pytest.mark.parametrize("R", [8, 4, 2])
def test_scale_table_layout(R):
    """pp_dual_scale_table against its definition: for rows Rb..Rb+R-1 of a projection
    (starting at position P), tab[P/gs + Rj + q] = scales[(P + q K)/gs + j]; positions
    outside every projection (gaps, the end) keep the scales array, 0 past its end."""
    from polar_pack_amd import _native as nat
    gs = 32
    shapes = [(16, 64), (8, 4096), (24, 1024)]
    pos0 = [256, 256 + 16 * 64 + 512, 256 + 16 * 64 + 512 + 8 * 4096]     # gaps before and between
    end = pos0[-1] + 24 * 1024
    n_groups = end // gs - 5                                               # the last rows run past the scales
    rng = np.random.default_rng(31)
    scales = rng.standard_normal(n_groups).astype(np.float16)
    n_tab = end // gs + 7
    tab = torch.full((n_tab,), float("nan"), dtype=torch.float16, device=DEV)
    sc_d = torch.from_numpy(scales).to(DEV)
    p_d = torch.tensor(pos0, dtype=torch.int64, device=DEV)
    n_d = torch.tensor([n for n, _ in shapes], dtype=torch.int32, device=DEV)
    k_d = torch.tensor([k for _, k in shapes], dtype=torch.int32, device=DEV)
    rc = nat.lib().pp_dual_scale_table(sc_d.data_ptr(), n_groups, gs, p_d.data_ptr(), n_d.data_ptr(), k_d.data_ptr(),
                                       len(shapes), R, tab.data_ptr(), n_tab, torch.cuda.current_stream().cuda_stream)
    nat.check(rc, "pp_dual_scale_table")
    got = tab.cpu().numpy()
    want = np.concatenate([scales, np.zeros(n_tab - n_groups, np.float16)])
    for (N, K), p in zip(shapes, pos0):
        gk = K // gs
        for r in range(N):
            for j in range(gk):
                src = (p + r * K) // gs + j
                dst = p // gs + (r // R) * R * gk + R * j + r % R
                want[dst] = scales[src] if src < n_groups else 0
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
