"""Pin the oracle's packers to golden vectors written by the reference's own packers.

The vectors were produced in the build container (numpy 2.2.6, torch
2.10.0 CPU) by tests/golden/make_golden.py; inputs are regenerated here from
the bit-stable generator in tests/golden/gen.py.  Float32 transcendental
results can differ between numpy/torch builds at rounding ties, so the
bit-exact packer checks are skipped on other library versions.
"""
import hashlib
import os

import numpy as np
import pytest
import torch

import gen
import make_golden as mg
from oracle import dualpack as odp
from oracle import layer as olay
from oracle import quadpack as oqp

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SAME_LIBS = np.__version__ == "2.2.6" and torch.__version__.startswith("2.10.0")
needs_same_libs = pytest.mark.skipif(not SAME_LIBS, reason="golden vectors were written with numpy 2.2.6 / torch 2.10.0")


def load(name):
    return np.load(os.path.join(HERE, name + ".npz"))


def test_generator_is_bit_stable():
    # a few fixed words of the integer-hash generator (catches any change to gen.py)
    u = gen.uniform(7, 3, 5)
    assert u.dtype == np.float32
    assert hashlib.sha256(u.tobytes()).hexdigest()[:16] == "af5b5e6ad33a651f"
    w = gen.correlated_models(1, [1000, 1000])
    assert hashlib.sha256(w[1].tobytes()).hexdigest()[:16] == "d2b6152731500fe0"
    assert all(x.dtype == np.float32 for x in w)
    assert 0.005 < float(np.std(w[0])) < 0.05


@needs_same_libs
@pytest.mark.parametrize("case", mg.QUAD_LAYER_CASES, ids=[c[0] for c in mg.QUAD_LAYER_CASES])
def test_pack_quad_layer_matches_reference(case):
    name, K, N, seed, corr = case
    g = load(name)
    ws = [torch.from_numpy(w) for w in mg.quad_layer_inputs(K, N, seed, corr)]
    codes, luts, scales = olay.pack_quad_layer(*ws)
    assert codes.shape == (K, N)
    np.testing.assert_array_equal(codes, g["codes"])
    np.testing.assert_array_equal(np.stack(luts).view(np.uint16), g["luts"].view(np.uint16))
    assert list(scales) == list(g["scales"])


@needs_same_libs
@pytest.mark.parametrize("case", mg.DUAL_LAYER_CASES, ids=[c[0] for c in mg.DUAL_LAYER_CASES])
def test_quantize_polar_bitpacked_matches_reference(case):
    name, K, N, seed, dt = case
    g = load(name)
    w1, w2 = [torch.from_numpy(w) for w in mg.dual_layer_inputs(K, N, seed, dt)]
    packed, bmax, amp_lut, cos_lut, sin_lut = olay.quantize_polar_bitpacked(w1, w2)
    np.testing.assert_array_equal(packed, g["packed"])
    np.testing.assert_array_equal(bmax.view(np.uint16), g["bmax"].view(np.uint16))
    for a, b in ((amp_lut, "amp_lut"), (cos_lut, "cos_lut"), (sin_lut, "sin_lut")):
        np.testing.assert_array_equal(a.view(np.uint16), g[b].view(np.uint16))


@needs_same_libs
@pytest.mark.slow
@pytest.mark.parametrize("case", mg.QUADPACK_CASES, ids=[c[0] for c in mg.QUADPACK_CASES])
def test_pack_quad_matches_reference_file(case):
    name, n, tails, seed, cap = case
    g = load(name)
    models = mg.quadpack_inputs(n, tails, seed)
    qp = oqp.pack_quad(models, plug_cap=cap)
    buf = qp.to_bytes()
    assert len(buf) == int(g["file_size"])
    assert bytes(buf[:oqp.HEADER_SIZE]) == g["header"].tobytes()
    assert hashlib.sha256(qp.codes.astype("<u4").tobytes()).hexdigest() == str(g["codes_sha"])
    assert int(qp.plug_idx.size) == int(g["plug_n"])
    np.testing.assert_array_equal(qp.plug_idx[:g["plug_idx_head"].size], g["plug_idx_head"])
    assert hashlib.sha256(buf).hexdigest() == str(g["file_sha"])


@needs_same_libs
@pytest.mark.parametrize("case", mg.DUALPACK_CASES, ids=[c[0] for c in mg.DUALPACK_CASES])
def test_pack_dual_matches_reference_file(case):
    name, n1, n2, seed, cap, chunk = case
    g = load(name)
    w1, w2 = mg.dualpack_inputs(n1, n2, seed)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=cap, chunk_size=chunk))
    assert dp.to_bytes() == g["packed"].tobytes()


@pytest.mark.parametrize("case", mg.DUALPACK_CASES, ids=[c[0] for c in mg.DUALPACK_CASES])
def test_dualpack_reader_round_trips_reference_file(case):
    g = load(case[0])
    buf = g["packed"].tobytes()
    dp = odp.DualPack.from_bytes(buf)
    assert dp.to_bytes() == buf
    assert (dp.n1, dp.n2, dp.chunk_size) == (case[1], case[2], case[5])
    assert dp.scales.size == odp.n_groups_for(dp.n_pairs, dp.chunk_size, dp.group_size)
    assert np.all(np.diff(dp.plug_idx.astype(np.int64)) > 0)


@pytest.mark.parametrize("case", mg.DUALPACK_CASES, ids=[c[0] for c in mg.DUALPACK_CASES])
def test_dual_unpack_of_reference_file_reconstructs_inputs(case):
    """The reference-written file decodes back to its inputs (cosine, amplitude, plug exactness)."""
    name, n1, n2, seed, cap, chunk = case
    g = load(name)
    dp = odp.DualPack.from_bytes(g["packed"].tobytes())
    o1, o2 = odp.unpack_dual(dp)
    w1, w2 = mg.dualpack_inputs(n1, n2, seed)
    for o, w in ((o1, w1), (o2, w2)):
        cos = float(np.dot(o.astype(np.float64), w) / (np.linalg.norm(o) * np.linalg.norm(w)))
        assert cos > 0.999, cos
    # plugged pairs carry the exact fp16 amplitude of the (zero-padded) input pair
    wp1 = np.pad(w1, (0, dp.n_pairs - n1))
    wp2 = np.pad(w2, (0, dp.n_pairs - n2))
    d1, d2 = odp.decode_pairs_f64(dp)
    pi = dp.plug_idx.astype(np.int64)
    amp_dec = np.hypot(d1[pi], d2[pi])
    np.testing.assert_allclose(amp_dec, dp.plug_val.astype(np.float64), rtol=1e-6, atol=1e-12)
    amp32 = np.sqrt(wp1[pi] ** 2 + wp2[pi] ** 2)          # float32, as the packer computes it
    np.testing.assert_array_equal(dp.plug_val, amp32.astype(np.float16))


@pytest.mark.parametrize("case", mg.QUADPACK_CASES, ids=[c[0] for c in mg.QUADPACK_CASES])
def test_quadpack_header_fields_of_reference_file(case):
    name, n, tails, seed, cap = case
    g = load(name)
    import struct
    hdr = struct.unpack(oqp.HEADER_FMT, g["header"].tobytes())
    assert hdr[0] == b"QUAD" and hdr[1] == 2 and hdr[2] == 4 and hdr[3] == n
    assert hdr[4:8] == (8, 8, 8, 8) and hdr[8] == 255.0
    assert hdr[9] == int(g["plug_n"])
    assert tuple(hdr[15:19]) == tuple(int(t) for t in tails)
    size = oqp.HEADER_SIZE + 4 * n + 12 * hdr[9] + 2 * sum(tails)
    assert size == int(g["file_size"])
    # plug count is ~cap * n (threshold is a sampled percentile, not an exact top-k)
    assert abs(hdr[9] / n - cap) < 0.2 * cap
