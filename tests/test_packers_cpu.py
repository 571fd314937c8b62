"""The product's kernel-layout packers (torch ops) against the reference-written golden
vectors, on CPU tensors (the same code runs on the GPU inside the parity tests)."""
import os

import numpy as np
import pytest
import torch

import make_golden as mg
from polar_pack_amd import polar_kernels as pk
from polar_pack_amd import quad_kernels as qk

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SAME_LIBS = np.__version__ == "2.2.6" and torch.__version__.startswith("2.10.0")
needs_same_libs = pytest.mark.skipif(not SAME_LIBS, reason="golden vectors were written with numpy 2.2.6 / torch 2.10.0")


@needs_same_libs
@pytest.mark.parametrize("case", mg.QUAD_LAYER_CASES, ids=[c[0] for c in mg.QUAD_LAYER_CASES])
def test_pack_quad_layer_cpu_equals_reference(case):
    name, K, N, seed, corr = case
    g = np.load(os.path.join(HERE, name + ".npz"))
    codes, luts, scales = qk.pack_quad_layer(*[torch.from_numpy(w) for w in mg.quad_layer_inputs(K, N, seed, corr)])
    assert codes.dtype == torch.uint32 and codes.shape == (K, N)
    np.testing.assert_array_equal(codes.view(torch.int32).numpy().view(np.uint32), g["codes"])
    np.testing.assert_array_equal(torch.stack(luts).numpy().view(np.uint16), g["luts"].view(np.uint16))
    assert scales == list(g["scales"])


@needs_same_libs
@pytest.mark.parametrize("case", mg.DUAL_LAYER_CASES, ids=[c[0] for c in mg.DUAL_LAYER_CASES])
def test_quantize_polar_bitpacked_cpu_equals_reference(case):
    name, K, N, seed, dt = case
    g = np.load(os.path.join(HERE, name + ".npz"))
    w1, w2 = [torch.from_numpy(w) for w in mg.dual_layer_inputs(K, N, seed, dt)]
    packed, bmax, amp_lut, cos_lut, sin_lut = pk.quantize_polar_bitpacked(w1, w2)
    np.testing.assert_array_equal(packed.numpy(), g["packed"])
    for t, key in ((bmax, "bmax"), (amp_lut, "amp_lut"), (cos_lut, "cos_lut"), (sin_lut, "sin_lut")):
        np.testing.assert_array_equal(t.numpy().view(np.uint16), g[key].view(np.uint16))


def test_pack_amp_phase_closed_form():
    amp = torch.arange(64).repeat_interleave(1024)
    ph = torch.arange(1024).repeat(64)
    p = pk.pack_amp_phase(amp, ph)
    assert p.dtype == torch.int16
    u = (p.to(torch.int32) + 32768)
    assert torch.equal(u >> 10, amp) and torch.equal(u & 1023, ph)
    assert int(p.min()) == -32768 and int(p.max()) == 32767


def test_operators_reject_cpu_tensors():
    a = torch.zeros(1, 8, dtype=torch.float16)
    codes = torch.zeros(8, 4, dtype=torch.int32).view(torch.uint32)
    luts = [torch.zeros(256, dtype=torch.float16)] * 7
    with pytest.raises(ValueError, match="ROCm device"):
        qk.quad_bitpacked(a, codes, luts, [1.0] * 4)


def test_header_luts_closed_form():
    l = qk.header_luts(3.0)
    assert all(t.dtype == torch.float32 and t.numel() == 256 for t in l)
    assert float(l[0][0]) == 0.0 and abs(float(l[0][255]) - 3.0) < 1e-6
    assert torch.equal(l[1], l[3]) and torch.equal(l[2], l[4])
    d = pk.header_luts()
    assert d[0].numel() == 64 and d[1].numel() == 1024
    assert abs(float(d[0][63]) - 1.0) < 1e-7 and float(d[1][0]) == -1.0 and float(d[2][512]) == 0.0


def test_transposed_plug_positions():
    """Plug entries of a (K,N) tensor moved to its (N,K) transpose (the matrix-core route
    for (K,N) storage): positions remapped, out-of-block entries moved to N*K (past every
    row's range, so the count stays that of the input), re-sorted."""
    import torch
    from polar_pack_amd.quad_kernels import transposed_plug
    K, N, ldk, base = 6, 5, 8, 100
    rng = np.random.default_rng(0)
    pos = np.sort(rng.choice(K * ldk + 20, 25, replace=False)).astype(np.int64) - 10   # some below 0, past the end
    vals = rng.standard_normal((pos.size, 4)).astype(np.float16)
    idx = torch.from_numpy((pos + base).astype(np.int64)).to(torch.int32)
    got_pos, got_vals = transposed_plug(idx, torch.from_numpy(vals), base, ldk, K, N)
    keep = [(p, v) for p, v in zip(pos, vals) if p >= 0 and p // ldk < K and p % ldk < N]
    want = sorted(((p % ldk) * K + p // ldk, tuple(v)) for p, v in keep)
    assert got_pos.dtype == torch.int32 and got_pos.numel() == pos.size and got_vals.shape == (pos.size, 4)
    n_in = len(want)
    assert 0 < n_in < pos.size
    np.testing.assert_array_equal(got_pos.numpy()[:n_in], [w[0] for w in want])
    np.testing.assert_array_equal(got_pos.numpy()[n_in:], N * K)
    np.testing.assert_array_equal(got_vals.numpy()[:n_in], np.array([w[1] for w in want], np.float16).reshape(-1, 4))


def test_pack_quad_device_tails_and_threshold_rule_match_the_oracle():
    """Models of unequal length (per-model fp16 tails, quaternion_packer.py:54-56, 121-126),
    given as lists cut at different places, with the reference's relative-error plug rule
    at a fixed threshold: the oracle packer's header, codes, plug table and tails."""
    import gen
    from oracle import quadpack as oqp
    from polar_pack_amd.packer import pack_quad_device
    n, tails = 60_000, (0, 517, 1031, 13)
    models = gen.correlated_models(61, [n + t for t in tails])
    cuts = [[], [1000, 30_000], [n], [7, 59_999, 60_500]]
    lists = [[torch.from_numpy(p) for p in np.split(m, c)] for m, c in zip(models, cuts)]
    pack = pack_quad_device(lists, select="ref", threshold=0.006)
    qp = oqp.pack_quad(models, threshold=0.006)
    assert pack.n == qp.n == n and pack.tail_lengths == list(tails)
    assert pack.s == qp.s and pack.r_max == qp.r_max
    got = pack.codes.view(torch.int32).numpy().view(np.uint32)
    flips = np.flatnonzero(got != qp.codes)
    assert flips.size <= 6, f"{flips.size} codes differ"
    for f in flips:            # a flip moves one byte field by one step (a rounding tie)
        d = [abs(int(got[f] >> s & 255) - int(qp.codes[f] >> s & 255)) for s in (24, 16, 8, 0)]
        assert sorted(d) == [0, 0, 0, 1] or sorted(d)[-1] == 255
    pi = pack.plug_idx.view(torch.int32).numpy().view(np.uint32)
    common, ia, ib = np.intersect1d(pi, qp.plug_idx, return_indices=True)
    assert qp.plug_idx.size > 100 and common.size >= 0.99 * max(pi.size, qp.plug_idx.size)
    np.testing.assert_array_equal(pack.plug_vals.numpy()[ia].view(np.uint16), qp.plug_vals[ib].view(np.uint16))
    for k in range(4):
        np.testing.assert_array_equal(pack.tails[k].numpy().view(np.uint16), qp.tails[k].view(np.uint16))


def test_pack_quad_device_list_cuts_do_not_change_the_pack():
    import gen
    from polar_pack_amd.packer import pack_quad_device
    models = gen.correlated_models(62, [30_000] * 4)
    one = pack_quad_device([[torch.from_numpy(m)] for m in models], plug_cap=0.01)
    cut = pack_quad_device([[torch.from_numpy(p) for p in np.split(m, [100 * (k + 1), 20_000])]
                            for k, m in enumerate(models)], plug_cap=0.01)
    assert one.s == cut.s and one.r_max == cut.r_max
    assert torch.equal(one.codes.view(torch.int32), cut.codes.view(torch.int32))
    assert torch.equal(one.plug_idx.view(torch.int32), cut.plug_idx.view(torch.int32))
    assert torch.equal(one.plug_vals, cut.plug_vals)
