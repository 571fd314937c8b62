"""GPU parity of the container path: reference-written ``.dualpack`` files read by the
product's reader and decoded on the device, the device quad packer against the
reference-written ``.quadpack`` files, and whole-step streams planned from the
reference's layer map (polar_main.py:33-46) over models of unequal length."""
import os
import struct

import numpy as np
import pytest
import torch

import gen
import make_golden as mg
from oracle import dualpack as odp
from oracle import quadpack as oqp
from parity import assert_gemv_close
from polar_pack_amd import polar_kernels as pk
from polar_pack_amd.container import DualPackFile
from polar_pack_amd.packer import pack_quad_device
from polar_pack_amd.stream import DualStream, QuadStream
from refs import quad_pack_host

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _layer_outputs(w, shapes, positions, xs):
    """float64 outputs per projection; a model without a weight at a position (NaN in the
    oracle's output) reads 0 there, and a row it has no weights for at all outputs 0."""
    outs = []
    for (N, K), pos, x in zip(shapes, positions, xs):
        per = []
        for wm in w:
            blk = wm[pos:pos + N * K].reshape(N, K)
            missing = np.isnan(blk[:, 0])
            y = x.astype(np.float64) @ np.nan_to_num(blk, nan=0.0).T
            y[:, missing] = 0.0
            per.append(y)
        outs.append(per)
    return outs


# ------------------------------------------------------------------ .dualpack files from the reference

DUAL_MAP = {   # layer maps over the reference-written streams: a 1-D entry is skipped, K % 8 == 0
    "dp_small": [{"name": "l.q", "shape": [10, 256], "numel": 2560}, {"name": "l.norm", "shape": [256], "numel": 256},
                 {"name": "l.k", "shape": [4, 512], "numel": 2048}, {"name": "l.o", "shape": [17, 8], "numel": 136}],
    "dp_longer2": [{"name": "l.q", "shape": [8, 2048], "numel": 16384}, {"name": "l.norm", "shape": [72], "numel": 72},
                   {"name": "l.k", "shape": [7, 1000], "numel": 7000}],
}


@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("name", sorted(DUAL_MAP))
def test_reference_dualpack_file_stream_from_layer_map(tmp_path, name, M):
    raw = np.load(os.path.join(HERE, name + ".npz"))["packed"].tobytes()
    path = tmp_path / "g.dualpack"
    path.write_bytes(raw)
    f = DualPackFile.read(path)
    pack = f.to_device(DEV)
    st = DualStream.from_layer_map(pack, DUAL_MAP[name], M=M)
    assert st.names == [e["name"] for e in DUAL_MAP[name] if len(e["shape"]) == 2]
    xs_np = [np.random.default_rng(7 + p).standard_normal((M, k)).astype(np.float16) for p, (_, k) in
             enumerate(st.shapes)]
    xs = [torch.from_numpy(x).to(DEV) for x in xs_np]
    outs = [[torch.full((M, n), float("nan"), dtype=torch.float16, device=DEV) for _ in range(2)] for n, _ in st.shapes]
    st.bind(xs, outs)
    dp = odp.DualPack.from_bytes(raw)
    w = odp.decode_pairs_f64(dp, 0, dp.n_pairs)
    ref = _layer_outputs(w, st.shapes, st.pos0, xs_np)
    for rep in range(2):
        st()
        torch.cuda.synchronize()
        for p in range(len(st.shapes)):
            for m in range(2):
                assert_gemv_close(outs[p][m].float().cpu().numpy(), ref[p][m], f"{st.names[p]} model {m} rep {rep}")


@pytest.mark.parametrize("M", [1, 4])
def test_reference_dualpack_file_with_odd_chunks_through_the_drop_in(tmp_path, M):
    """dp_cap003: chunks of 10,001 pairs (groups restart mid-row), 3% plug: (N,K) Linears cut
    from the file, through polar_dual_bitpacked on the container layout."""
    raw = np.load(os.path.join(HERE, "dp_cap003.npz"))["packed"].tobytes()
    path = tmp_path / "g.dualpack"
    path.write_bytes(raw)
    pack = DualPackFile.read(path).to_device(DEV)
    dp = odp.DualPack.from_bytes(raw)
    amp, cos, sin = pk.header_luts(pack.amp_bits, pack.phase_bits, pack.mu, device=DEV)
    for base, N, K in ((0, 20, 1000), (20_000, 48, 1000), (69_000, 1, 1000)):
        x = np.random.default_rng(base + M).standard_normal((M, K)).astype(np.float16)
        got = pk.polar_dual_bitpacked(torch.from_numpy(x).to(DEV), pack.codes[base:base + N * K].reshape(N, K).t(),
                                      pack.scales, amp, cos, sin, plug=(pack.plug_idx, pack.plug_val), elem_base=base,
                                      layout=pack.layout, chunk_size=pack.chunk_size)
        d = odp.decode_pairs_f64(dp, base, base + N * K)
        for m in range(2):
            assert_gemv_close(got[m].float().cpu().numpy(), x.astype(np.float64) @ d[m].reshape(N, K).T,
                              f"base {base} model {m}")


# ------------------------------------------------------------------ device quad packer vs the reference's files

@pytest.mark.parametrize("case", mg.QUADPACK_CASES, ids=[c[0] for c in mg.QUADPACK_CASES])
def test_device_quad_packer_matches_reference_file(case):
    """pack_quad_device with the reference's plug rule (select="ref": relative-error
    percentile over the seeded windows, quaternion_packer.py:79-113) on the GPU, against the
    file the reference wrote for the same weights: header RMS and r_max bit-equal, codes
    equal but for one-step flips at rounding ties, the plug set and values, the tails."""
    name, n, tails, seed, cap = case
    g = np.load(os.path.join(HERE, name + ".npz"))
    hdr = struct.unpack(oqp.HEADER_FMT, g["header"].tobytes())
    models = mg.quadpack_inputs(n, tails, seed)
    pack = pack_quad_device([[torch.from_numpy(m).to(DEV)] for m in models], plug_cap=cap, select="ref")
    assert pack.n == hdr[3] == n and pack.tail_lengths == list(hdr[15:19])
    assert pack.s == tuple(hdr[10:14]), (pack.s, hdr[10:14])
    assert pack.r_max == hdr[14]
    assert abs(pack.plug_idx.numel() - hdr[9]) <= 0.01 * hdr[9]
    # the oracle's codes for the reference's header values reproduce the reference file's
    # codes (SHA-256); the device codes match them but for rare one-step ties
    wc = [np.asarray(m[:n], np.float32) / np.float32(sk) for m, sk in zip(models, hdr[10:14])]
    ref_codes = oqp.quantize_chunk(wc, hdr[14])
    import hashlib
    assert hashlib.sha256(ref_codes.astype("<u4").tobytes()).hexdigest() == str(g["codes_sha"])
    got = pack.codes.view(torch.int32).cpu().numpy().view(np.uint32)
    flips = np.flatnonzero(got != ref_codes)
    assert flips.size <= 1e-4 * n, f"{flips.size} codes differ"
    for f in flips:
        d = sorted(abs(int(got[f] >> s & 255) - int(ref_codes[f] >> s & 255)) for s in (24, 16, 8, 0))
        assert d[:3] == [0, 0, 0] and d[3] in (1, 255)
    head = g["plug_idx_head"]
    vals_head = g["plug_vals_head"].reshape(-1, 4)
    pi = pack.plug_idx.view(torch.int32).cpu().numpy().view(np.uint32)
    mine = pi[pi <= head[-1]]
    common, ia, ib = np.intersect1d(mine, head, return_indices=True)
    assert common.size >= 0.99 * max(mine.size, head.size)
    np.testing.assert_array_equal(pack.plug_vals[:mine.size].cpu().numpy()[ia].view(np.uint16),
                                  vals_head[ib].view(np.uint16))
    for k in range(4):
        np.testing.assert_array_equal(pack.tails[k].cpu().numpy().view(np.uint16),
                                      models[k][n:].astype(np.float16).view(np.uint16))


# ------------------------------------------------------------------ quad stream from a layer map, unequal lengths

QUAD_MAP = [{"name": "l0.q", "shape": [64, 256], "numel": 64 * 256},
            {"name": "l0.norm", "shape": [256], "numel": 256},
            {"name": "l0.k", "shape": [16, 512], "numel": 16 * 512},
            {"name": "l0.gate", "shape": [40, 1024], "numel": 40 * 1024},
            {"name": "l0.down", "shape": [24, 2048], "numel": 24 * 2048}]


@pytest.mark.parametrize("M", [1, 4])
def test_quad_stream_from_layer_map_with_device_packed_tails(M):
    """4 models of unequal length packed on the device (tails, quaternion_packer.py:54-56,
    121-126; the reference's plug rule at a fixed threshold), the stream planned from a
    layer map with a skipped entry, against the oracle's decode of the device pack, and the
    device pack against the oracle packer on the same weights."""
    total = sum(e["numel"] for e in QUAD_MAP)
    n = total - 5 * 2048 - 100                       # row 18 of l0.down straddles n
    tails = (0, total - n + 7, 1000, total - n)
    models = gen.correlated_models(81, [n + t for t in tails])
    cuts = [[16384], [100, 30_000], [], [n - 3]]
    lists = [[torch.from_numpy(p).to(DEV) for p in np.split(m, c)] for m, c in zip(models, cuts)]
    pack = pack_quad_device(lists, select="ref", threshold=0.006)
    qp_ref = oqp.pack_quad(models, threshold=0.006)
    assert pack.s == qp_ref.s and pack.r_max == qp_ref.r_max and pack.tail_lengths == list(tails)
    got_codes = pack.codes.view(torch.int32).cpu().numpy().view(np.uint32)
    assert np.count_nonzero(got_codes != qp_ref.codes) <= 1e-3 * n
    st = QuadStream.from_layer_map(pack, QUAD_MAP, M=M)
    assert st.names == ["l0.q", "l0.k", "l0.gate", "l0.down"] and st.n_tail > 0
    xs_np = [np.random.default_rng(50 + p).standard_normal((M, k)).astype(np.float16) for p, (_, k) in
             enumerate(st.shapes)]
    xs = [torch.from_numpy(x).to(DEV) for x in xs_np]
    outs = [[torch.full((M, nn), float("nan"), dtype=torch.float16, device=DEV) for _ in range(4)]
            for nn, _ in st.shapes]
    st.bind(xs, outs)
    w = oqp.unpack_quad_f64(quad_pack_host(pack), 0, total)
    ref = _layer_outputs(w, st.shapes, st.pos0, xs_np)
    for rep in range(2):
        st()
        torch.cuda.synchronize()
        for p in range(len(st.shapes)):
            for m in range(4):
                assert_gemv_close(outs[p][m].float().cpu().numpy(), ref[p][m], f"{st.names[p]} model {m} rep {rep}")
