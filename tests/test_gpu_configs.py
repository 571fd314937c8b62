"""GPU parity at the five benchmark workloads' own shapes, through the routes bench.py times.

* dual 2048x2048 Linear, 2 models, plug 0.1% of pairs, 1 token: the split-K ``DualStream``
  and the drop-in ``polar_dual_bitpacked`` on the container layout, whole Linear against the
  oracle's float64 decode (polar_bitpack.py:228-247);
* quad gate_proj 11008x2048 and down_proj 2048x11008, 4 models, plug 0.1% of tuples, at
  1, 4, 16 and 64 tokens: the split-K ``QuadStream`` (1-8 tokens) or the matrix-core
  ``QuadBatch`` (16, 64), and the drop-in ``quad_bitpacked`` on the reference's (K,N) view
  of the container rows, whole Linear against the oracle (quaternion_packer.py:169-196);
* quad Qwen2.5-3B-shaped stream (36 x 7 projections, 2,774,532,096 tuples), 1 token: the
  one-launch ``QuadStream``, a row sample of every projection (first, last, random rows and
  the row with the most plug entries) against the oracle's float64 decode of those rows,
  and every projection against the per-projection drop-in operator;
* dual 3B-shaped heavy-tail stream (model 2 truncated by 5%, model 1's rest in fp16 tails,
  plug 1% of pairs): the one-launch ``DualStream``, a row sample of every projection
  including the row that straddles the end of the codes and rows inside and past the
  tails, against the oracle decode plus the tails, and the projections below the tails
  against the drop-in operator.

Weights are synthesized and packed exactly as bench.py does (its generator functions).
"""
import numpy as np
import pytest
import torch

import bench
from parity import assert_gemv_close, normwise
from polar_pack_amd import polar_kernels as pk
from polar_pack_amd import quad_kernels as qk
from polar_pack_amd.stream import DualStream, QuadStream
from refs import check_mfma, dual_pack_host, dual_rows_ref, quad_pack_host, quad_rows_ref, route_class
from test_gpu_dual import prefill_bound

from oracle import dualpack as odp
from oracle import layer as olay
from oracle import quadpack as oqp

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _x(M, K, seed):
    return np.random.default_rng(seed).standard_normal((M, K)).astype(np.float16)


def _sample_rows(plug_host, pos0, N, K, rng, n_random=4, limit=None):
    """First, last, a few random rows and the row holding the most plug entries (all below
    ``limit`` rows when given)."""
    R = N if limit is None else limit
    starts = pos0 + np.arange(R + 1, dtype=np.int64) * K
    counts = np.diff(np.searchsorted(plug_host, starts, side="left"))
    rows = {0, R - 1, int(counts.argmax())} | {int(r) for r in rng.integers(0, R, n_random)}
    return np.array(sorted(rows), np.int64), counts


def _segment_edges(st):
    """Per projection, the rows where the stream's planner cuts: the first and last row of
    every segment of the launch's segment table (so the first and last row of every wave's
    run, and the rows on either side of every projection boundary inside one wave's run), and
    the number of such (projection, row) pairs."""
    edges = {}
    for g in st.segs_np:
        p = int(g["proj"])
        edges.setdefault(p, set()).update({int(g["row0"]), int(g["row1"]) - 1})
    # a projection boundary inside one wave's run: the last row before it and the first after
    for w in range(st.n_waves):
        lo, hi = int(st.bounds_np[w]), int(st.bounds_np[w + 1])
        for i in range(lo, hi - 1):
            a, b = st.segs_np[i], st.segs_np[i + 1]
            if int(a["proj"]) != int(b["proj"]):
                edges[int(a["proj"])].add(int(a["row1"]) - 1)
                edges[int(b["proj"])].add(int(b["row0"]))
    return edges, sum(len(v) for v in edges.values())


# ------------------------------------------------------------------ dual 2048x2048 Linear

def test_dual_2048_linear_split_stream_and_drop_in():
    pack = bench.dual2048_pack(DEV)
    N = K = 2048
    assert pack.plug_idx.numel() == int(0.001 * N * K)
    st = DualStream(pack, [(N, K)], M=1)
    assert st.split, "one 2048-row Linear at 1 token runs on split-K slices"
    xs, outs = st.make_buffers()
    x_np = _x(1, K, 21)
    xs[0].copy_(torch.from_numpy(x_np))
    st.bind(xs, outs)
    dp = dual_pack_host(pack)
    w = odp.decode_pairs_f64(dp, 0, N * K)
    ref = [x_np.astype(np.float64) @ w[m].reshape(N, K).T for m in range(2)]
    for rep in range(3):                          # a split workspace is left zero for the next launch
        for o in outs[0]:
            o.fill_(float("nan"))
        st()
        torch.cuda.synchronize()
        for m in range(2):
            assert_gemv_close(outs[0][m].float().cpu().numpy(), ref[m], f"stream rep {rep} model {m}")
        if st.workspace is not None:              # (none when the slices meet in LDS)
            assert int(torch.count_nonzero(st.workspace)) == 0
    amp, cos, sin = pk.header_luts(pack.amp_bits, pack.phase_bits, pack.mu, device=DEV)
    view = pack.codes.reshape(N, K).t()
    got = pk.polar_dual_bitpacked(xs[0], view, pack.scales, amp, cos, sin, plug=(pack.plug_idx, pack.plug_val),
                                  layout=pack.layout, chunk_size=pack.chunk_size)
    torch.cuda.synchronize()
    # the drop-in's route for these rows: the matrix cores multiply fp16-rounded weights (the
    # reference's own operands, polar_kernels.py:78-82), held to the fp16-weight bound
    route = pk.dual_call_route(view, 1, layout=pack.layout, chunk_size=pack.chunk_size,
                               plug_n=pack.plug_idx.numel())
    for m in range(2):
        assert_gemv_close(got[m].float().cpu().numpy(), ref[m], f"drop-in model {m} route {route}",
                          bound=prefill_bound(x_np, w[m].reshape(N, K).T, route))


# ------------------------------------------------------------------ quad gate / down, 1-64 tokens

_LINEAR = {}


def _linear(name):
    """(device pack, float64 exact weights, fp16-operand weights) of gate_proj / down_proj."""
    if name not in _LINEAR:
        _LINEAR.clear()
        torch.cuda.empty_cache()
        N, K = (11008, 2048) if name == "gate_proj" else (2048, 11008)
        pack = bench.quad_linear_pack(N, K, DEV, bench.seed_of(4, 0, 0 if name == "gate_proj" else 1))
        qp = quad_pack_host(pack)
        W = oqp.unpack_quad_f64(qp)
        exact = [W[m].reshape(N, K) for m in range(4)]
        del W
        luts = [l.numpy() for l in qk.header_luts(qp.r_max)]
        wn = olay.quad_dequant(qp.codes.reshape(1, -1), luts, dtype=np.float32)
        at = qp.plug_idx.astype(np.int64)
        w16 = []
        for m in range(4):
            h = wn[m][0].astype(np.float16)
            h[at] = qp.plug_vals[:, m]
            w16.append(h.astype(np.float64).reshape(N, K) * float(np.float32(qp.s[m])))
        del wn
        _LINEAR[name] = (pack, N, K, exact, w16)
    return _LINEAR[name]


@pytest.mark.parametrize("M", [1, 4, 16, 64])
@pytest.mark.parametrize("name", ["gate_proj", "down_proj"])
def test_quad_gate_down_sweep(name, M):
    pack, N, K, exact, w16 = _linear(name)
    assert abs(pack.plug_idx.numel() / (N * K) - 0.001) < 0.0002
    x_np = _x(M, K, 30 + M)
    xd = x_np.astype(np.float64)
    ref_exact = [xd @ exact[m].T for m in range(4)]
    if M <= 8:
        st = QuadStream(pack, [(N, K)], M=M)     # split-K slices when the rows are few (down_proj)
    else:
        st = bench._batch_as_stream(pack, [(N, K)], M)
    xs, outs = st.make_buffers()
    xs[0].copy_(torch.from_numpy(x_np))
    st.bind(xs, outs)
    ref_mfma = None
    if M > 8:
        ref_mfma = (ref_exact, [xd @ w16[m].T for m in range(4)],
                    [2.0 ** -18 * (np.abs(xd) @ np.abs(w16[m]).T) for m in range(4)])
    for rep in range(2):
        for o in outs[0]:
            o.fill_(float("nan"))
        st()
        torch.cuda.synchronize()
        if M <= 8:
            for m in range(4):
                assert_gemv_close(outs[0][m].float().cpu().numpy(), ref_exact[m], f"{name} M={M} rep {rep} model {m}")
        else:
            check_mfma(outs[0], ref_mfma, f"{name} M={M} rep {rep}")
    # the drop-in operator on the reference's (K, N) view of the container rows
    luts = qk.header_luts(pack.r_max, device=DEV)
    got = qk.quad_bitpacked(xs[0], pack.codes.reshape(N, K).t(), luts, list(pack.s),
                            plug=(pack.plug_idx, pack.plug_vals))
    torch.cuda.synchronize()
    if M <= 8:
        for m in range(4):
            assert_gemv_close(got[m].float().cpu().numpy(), ref_exact[m], f"drop-in {name} M={M} model {m}")
    else:
        check_mfma(got, ref_mfma, f"drop-in {name} M={M}")


# ------------------------------------------------------------------ quad 3B-shaped stream

def test_quad_3b_stream_row_sample_and_per_projection():
    _LINEAR.clear()
    torch.cuda.empty_cache()
    shapes = bench.stream_shapes(36)
    pack = bench.quad3b_pack(36, DEV)
    assert pack.n == 2_774_532_096
    plug = pack.plug_host()
    st = QuadStream(pack, shapes, M=1)
    assert not st.split and st.n_tail == 0
    xs, outs = st.make_buffers()
    g = torch.Generator(device=DEV).manual_seed(7)
    for x in xs:
        x.copy_(torch.randn(x.shape, generator=g, device=DEV).to(torch.float16))
    for o in outs:
        for t in o:
            t.fill_(float("nan"))
    st.bind(xs, outs)
    st()
    torch.cuda.synchronize()
    rng = np.random.default_rng(2026)
    luts = qk.header_luts(pack.r_max, device=DEV)
    edges, n_edges = _segment_edges(st)
    plugged = checked_edges = 0
    for p, (N, K) in enumerate(shapes):
        pos0 = int(st.pos0[p])
        rows, counts = _sample_rows(plug, pos0, N, K, rng)
        edge = edges.get(p, set())
        rows = np.array(sorted(set(rows.tolist()) | edge), np.int64)
        checked_edges += len(edge)
        x_np = xs[p].cpu().numpy()
        ref, n_plug = quad_rows_ref(pack, plug, pos0, K, rows, x_np)
        plugged += n_plug
        for m in range(4):
            got = outs[p][m].float().cpu().numpy()
            assert_gemv_close(got[:, rows], ref[m], f"projection {p} ({N}x{K}) model {m} rows {rows.tolist()}")
        # the whole projection against the per-projection drop-in operator
        single = qk.quad_bitpacked(xs[p], pack.codes[pos0:pos0 + N * K].reshape(N, K).t(), luts, list(pack.s),
                                   plug=(pack.plug_idx, pack.plug_vals), elem_base=pos0)
        for m in range(4):
            assert_gemv_close(outs[p][m].float().cpu().numpy(), single[m].float().cpu().numpy(),
                              f"projection {p} model {m}: stream vs drop-in")
    assert plugged > 1000
    # every wave's first and last row and both sides of every projection cut, against the oracle
    assert checked_edges == n_edges and n_edges >= st.n_waves, (checked_edges, n_edges, st.n_waves)
    print(f"quad 3B stream: {n_edges} segment-edge rows checked against the float64 oracle")


# ------------------------------------------------------------------ dual 3B-shaped heavy-tail stream

def test_dual_3b_stream_with_tails_row_sample():
    _LINEAR.clear()
    torch.cuda.empty_cache()
    shapes = bench.stream_shapes(36)
    pack = bench.dual3b_pack(36, DEV, tails=True)
    n1 = sum(n * k for n, k in shapes)
    n2 = int(np.floor(0.95 * n1))
    assert pack.n1 == n1 and pack.n2 == n2 and pack.n_codes == 8 * (n2 // 8)
    assert pack.tail_lengths == [n1 - pack.n_codes, n2 - pack.n_codes]
    plug = pack.plug_host()
    st = DualStream(pack, shapes, M=1)
    assert st.n_tail > 0
    xs, outs = st.make_buffers()
    g = torch.Generator(device=DEV).manual_seed(7)
    for x in xs:
        x.copy_(torch.randn(x.shape, generator=g, device=DEV).to(torch.float16))
    for o in outs:
        for t in o:
            t.fill_(float("nan"))
    st.bind(xs, outs)
    st()
    torch.cuda.synchronize()
    dp = dual_pack_host(pack)
    tails = [t.cpu().numpy() for t in pack.tails]
    amp, cos, sin = pk.header_luts(pack.amp_bits, pack.phase_bits, pack.mu, device=DEV)
    rng = np.random.default_rng(2027)
    n = pack.n_codes
    saw_straddle = saw_tail = saw_past = False
    edges, n_edges = _segment_edges(st)
    checked_edges = 0
    for p, (N, K) in enumerate(shapes):
        pos0 = int(st.pos0[p])
        rows, _ = _sample_rows(plug, pos0, N, K, rng, n_random=3)
        edge = edges.get(p, set())
        rows = np.array(sorted(set(rows.tolist()) | edge), np.int64)
        checked_edges += len(edge)
        if pos0 < n < pos0 + N * K:                   # the projection the codes end in
            r = (n - pos0) // K
            extra = [r - 1, r, r + 1, N - 1] if (n - pos0) % K else [r - 1, r, N - 1]
            rows = np.array(sorted(set(rows.tolist()) | {int(v) for v in extra if 0 <= v < N}), np.int64)
        starts = pos0 + rows * K
        saw_straddle |= bool(np.any((starts < n) & (starts + K > n)))
        saw_tail |= bool(np.any(starts >= n))
        saw_past |= bool(np.any(starts + K > n + pack.tail_lengths[1]))
        x_np = xs[p].cpu().numpy()
        ref = dual_rows_ref(dp, tails, pos0, K, rows, x_np)
        for m in range(2):
            got = outs[p][m].float().cpu().numpy()
            assert_gemv_close(got[:, rows], ref[m], f"projection {p} ({N}x{K}) model {m} rows {rows.tolist()}")
        if pos0 + N * K <= n:
            view = pack.codes[pos0:pos0 + N * K].reshape(N, K).t()
            single = pk.polar_dual_bitpacked(xs[p], view, pack.scales, amp, cos, sin,
                                             plug=(pack.plug_idx, pack.plug_val), elem_base=pos0,
                                             layout=pack.layout, chunk_size=pack.chunk_size)
            route = pk.dual_call_route(view, 1, layout=pack.layout, chunk_size=pack.chunk_size, elem_base=pos0,
                                       plug_n=pack.plug_idx.numel())
            for m in range(2):
                got, other = outs[p][m].float().cpu().numpy(), single[m].float().cpu().numpy()
                what = f"projection {p} model {m}: stream vs drop-in ({route})"
                if route_class(route) == "fused":
                    assert_gemv_close(got, other, what)
                else:   # fp16 weights on the drop-in's route: the whole output, normwise
                    assert normwise(other, got) <= 1e-3, what
    assert saw_straddle and saw_tail and saw_past
    assert checked_edges == n_edges and n_edges >= st.n_waves, (checked_edges, n_edges, st.n_waves)
    print(f"dual 3B stream: {n_edges} segment-edge rows checked against the float64 oracle")
