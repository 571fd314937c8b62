"""Pin the oracle's decoders by what the mathematics fixes.

Each check is chosen so that a plausible slip in the oracle (a dropped sin
factor, swapped angle bytes, a wrong phase offset, a wrong group index, a
missing RMS scale) fails it: norms and angles of decoded tuples are recovered
by an independent inverse map, not by re-typing the decode formula.
"""
import math
import struct

import numpy as np
import pytest
import torch

import gen
from oracle import dualpack as odp
from oracle import layer as olay
from oracle import quadpack as oqp


def test_header_sizes():
    assert struct.calcsize(oqp.HEADER_FMT) == 82 == oqp.HEADER_SIZE
    assert struct.calcsize(odp.HEADER_FMT) == 62 == odp.HEADER_SIZE


def all_codes_sample(n=200_000, seed=5):
    rng = np.random.default_rng(seed)
    c = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    # include every value of every byte lane at least once
    lane = np.arange(256, dtype=np.uint32)
    extra = np.concatenate([lane << 24 | lane << 16 | lane << 8 | lane, (lane << 24) | 0x55AA33,
                            0x7F000000 | lane])
    return np.concatenate([c, extra])


def test_quad_fields_round_trip_exhaustive_bytes():
    c = all_codes_sample()
    nq, q1, q2, q3 = oqp.decode_fields(c)
    assert nq.max() == 255 and q3.max() == 255
    np.testing.assert_array_equal((nq << 24) | (q1 << 16) | (q2 << 8) | q3, c)
    # byte order of a little-endian file word: [q3, q2, q1, nq]
    b = c.astype("<u4").view(np.uint8).reshape(-1, 4)
    np.testing.assert_array_equal(b[:, 0], q3)
    np.testing.assert_array_equal(b[:, 3], nq)


def test_quad_decode_norm_is_norm_code():
    """|decoded tuple| == (256^(nq/255) - 1) * r_max / mu, independent of the angles."""
    c = all_codes_sample()
    r_max = 7.25
    w = oqp.decode_normalised(c, r_max)
    norm = np.sqrt(sum(x * x for x in w))
    nq = (c >> 24).astype(np.float64)
    expect = (256.0 ** (nq / 255.0) - 1.0) * r_max / 255.0
    np.testing.assert_allclose(norm, expect, rtol=1e-13, atol=1e-300)
    assert np.all(norm[nq == 0] == 0)
    np.testing.assert_allclose(norm[nq == 255], r_max, rtol=1e-14)


def test_quad_decode_angles_invert():
    """Recover (t1, t2, t3) from the decoded tuple with an independent inverse map."""
    rng = np.random.default_rng(1)
    q = rng.integers(1, 255, (4, 50_000)).astype(np.uint32)   # avoid the poles where angles degenerate
    q[0] = rng.integers(64, 256, 50_000)
    c = (q[0] << 24) | (q[1] << 16) | (q[2] << 8) | q[3]
    w1, w2, w3, w4 = oqp.decode_normalised(c, 3.0)
    t1 = np.arccos(w1 / np.sqrt(w1 ** 2 + w2 ** 2 + w3 ** 2 + w4 ** 2))
    t2 = np.arccos(w2 / np.sqrt(w2 ** 2 + w3 ** 2 + w4 ** 2))
    t3 = np.mod(np.arctan2(w4, w3), 2 * np.pi)
    np.testing.assert_allclose(t1, q[1] * np.pi / 255, atol=1e-9)
    np.testing.assert_allclose(t2, q[2] * np.pi / 255, atol=1e-9)
    d3 = np.abs(np.angle(np.exp(1j * (t3 - q[3] * 2 * np.pi / 255))))
    assert d3.max() < 1e-9


def test_quad_special_tuples():
    # single-axis tuples and (1,1,1,1): codes of the angles are known in closed form
    r_max = 4.0 * 1.001
    wc = [np.array([1.0, 0.0, 0.0, 0.0, -1.0, 1.0], np.float32),
          np.array([0.0, 1.0, 0.0, 0.0, 0.0, 1.0], np.float32),
          np.array([0.0, 0.0, 1.0, 0.0, 0.0, 1.0], np.float32),
          np.array([0.0, 0.0, 0.0, 1.0, 0.0, 1.0], np.float32)]
    nq, q1, q2, q3 = oqp.decode_fields(oqp.quantize_chunk(wc, r_max))
    assert list(q1[:5]) == [0, 128, 128, 128, 255]            # pi/2 * 255/pi = 127.5 -> 128 (float32 rounding)
    assert list(q2[:4]) == [0, 0, 128, 128]
    assert list(q3[:4]) == [0, 0, 0, 64]                       # pi/2 / 2pi * 255 = 63.75 -> 64
    # (1,1,1,1): t1 = pi/3, t2 = atan(sqrt 2), t3 = pi/4
    assert q1[5] == round(255 / 3) and q2[5] == round(math.atan(math.sqrt(2)) / math.pi * 255) and q3[5] == round(255 / 8)
    # zero tuple decodes to exactly zero
    z = oqp.decode_normalised(np.array([0x00123456], np.uint32), r_max)
    assert all(float(x[0]) == 0.0 for x in z)
    # q3 = 0 and q3 = 255 both mean angle 0 == 2 pi (cos = 1)
    a = oqp.decode_normalised(np.array([(255 << 24) | (128 << 16) | (128 << 8) | 0, (255 << 24) | (128 << 16) | (128 << 8) | 255], np.uint32), r_max)
    np.testing.assert_allclose(a[2][0], a[2][1], rtol=1e-12)


def _tiny_container(seed=3, n=5000, tails=(0, 7, 0, 13), cap=0.01):
    models = gen.correlated_models(seed, [n + t for t in tails])
    qp = oqp.pack_quad(models, plug_cap=cap, threshold=0.006)
    return models, qp


def test_quad_pack_unpack_reconstruction_and_plug_exactness():
    models, qp = _tiny_container()
    outs = oqp.unpack_quad(qp)
    n = qp.n
    # RMS scales are the float32-rounded RMS of the common part
    for k in range(4):
        s = math.sqrt(float(np.sum(models[k][:n].astype(np.float64) ** 2)) / n)
        assert qp.s[k] == float(np.float32(s))
    for k in range(4):
        w = models[k][:n].astype(np.float64)
        o = outs[k][:n].astype(np.float64)
        assert np.dot(o, w) / (np.linalg.norm(o) * np.linalg.norm(w)) > 0.999
    assert qp.plug_idx.size > 0
    for k in range(4):
        got = outs[k][qp.plug_idx.astype(np.int64)]
        want = (qp.plug_vals[:, k].astype(np.float64) * qp.s[k]).astype(np.float32)
        np.testing.assert_array_equal(got, want)
        # tails are the fp16 copy of the model's extra weights
        t = qp.tail_lengths[k]
        np.testing.assert_array_equal(outs[k][n:], models[k][n:].astype(np.float16).astype(np.float32))
        assert outs[k].size == n + t


def test_quad_container_bytes_round_trip():
    _, qp = _tiny_container()
    buf = qp.to_bytes()
    qp2 = oqp.QuadPack.from_bytes(buf)
    assert qp2.to_bytes() == buf
    assert len(buf) == oqp.HEADER_SIZE + 4 * qp.n + 12 * qp.plug_idx.size + 2 * sum(qp.tail_lengths)
    f64 = oqp.unpack_quad_f64(qp2)
    f32 = oqp.unpack_quad(qp2)
    for k in range(4):
        L = f32[k].size
        np.testing.assert_array_equal(f64[k][:L].astype(np.float32), f32[k])
        assert np.all(np.isnan(f64[k][L:]))


def test_quad_unpack_f64_window_matches_full():
    _, qp = _tiny_container()
    full = oqp.unpack_quad_f64(qp)
    win = oqp.unpack_quad_f64(qp, 4990, 5010)
    for k in range(4):
        np.testing.assert_array_equal(win[k], full[k][4990:5010])


def test_dual_be_identity_with_kernel_int16():
    """bswap16(file u16) ^ 0x8000 == the kernel's int16 bit pattern (pack_amp_phase)."""
    amp = np.repeat(np.arange(64), 1024)
    ph = np.tile(np.arange(1024), 64)
    code = (amp << 10) | ph
    be = odp.to_be_bytes(code)
    np.testing.assert_array_equal(odp.from_be_bytes(be), code)
    file_u16_le = be.view("<u2")
    swapped = ((file_u16_le >> 8) | ((file_u16_le & 0xFF) << 8)).astype(np.uint16)
    k16 = olay.pack_amp_phase(amp, ph).astype(np.int16)
    np.testing.assert_array_equal(swapped ^ 0x8000, k16.view(np.uint16))


def test_dual_decode_amplitude_and_angle():
    cfg = odp.DualConfig(plug_cap=0.0, chunk_size=96)
    amp = np.repeat(np.arange(64, dtype=np.uint32), 16)
    ph = (np.arange(amp.size, dtype=np.uint32) * 37) % 1024
    ph[16] = 0                                          # a nonzero amplitude at phase index 0
    n = amp.size
    scales = (np.arange(odp.n_groups_for(n, cfg.chunk_size, 32)) % 5 + 1).astype(np.float16) * np.float16(0.01)
    dp = odp.DualPack(n_pairs=n, n1=n, n2=n, codes_be=odp.to_be_bytes((amp << 10) | ph), scales=scales,
                      plug_idx=np.zeros(0, np.uint32), plug_val=np.zeros(0, np.float16), chunk_size=96)
    w1, w2 = odp.decode_pairs_f64(dp)
    g = (np.arange(n) // 96) * 3 + (np.arange(n) % 96) // 32
    expect_amp = (256.0 ** (amp / 63.0) - 1.0) / 255.0 * scales[g].astype(np.float64)
    np.testing.assert_allclose(np.hypot(w1, w2), expect_amp, rtol=2e-7)
    assert np.all(np.hypot(w1, w2)[amp == 0] == 0)
    np.testing.assert_allclose(np.hypot(w1, w2)[amp == 63], scales[g][amp == 63].astype(np.float64), rtol=2e-7)
    ang = np.arctan2(w2, w1)
    sel = amp > 0
    d = np.angle(np.exp(1j * (ang[sel] - (ph[sel] / 1024.0 * 2 * np.pi - np.pi))))
    assert np.abs(d).max() < 1e-9
    # phase 0 is -pi: w1 = -amp, w2 = 0 (up to float rounding of sin(-pi))
    i = np.nonzero((ph == 0) & (amp > 0))[0][0]
    assert w1[i] < 0 and abs(w2[i]) < 1e-15


def test_dual_group_index_restarts_per_chunk():
    pos = np.arange(0, 250)
    g = odp.group_index(pos, 100, 32)
    # chunk of 100 has ceil(100/32) = 4 groups; positions 96..99 are group 3, position 100 starts group 4
    assert g[95] == 2 and g[96] == 3 and g[99] == 3 and g[100] == 4 and g[249] == 4 + 4 + (49 // 32)
    assert odp.n_groups_for(250, 100, 32) == 4 + 4 + 2


def test_dual_pack_w2_zero_phase_index():
    # w2 = 0: phase is 0 (index 512) for w1 > 0 and pi (index 0 == 1024 mod 1024) for w1 < 0
    w1 = np.array([0.3, -0.3, 0.01, -0.02] * 8, np.float32)
    w2 = np.zeros_like(w1)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=0.0))
    ph = dp.codes_u16() & 1023
    assert set(ph[w1 > 0]) == {512} and set(ph[w1 < 0]) == {0}


def test_quad_layer_dequant_matches_container_decode():
    """Kernel-layout LUT decode (fp64 LUTs built from the same r_max) == container decode."""
    c = all_codes_sample(5000)
    r_max = 5.5
    i = np.arange(256, dtype=np.float64)
    luts = [(np.exp(i / 255 * math.log1p(255.0)) - 1) * r_max / 255.0,
            np.cos(i / 255 * np.pi), np.sin(i / 255 * np.pi), np.cos(i / 255 * np.pi), np.sin(i / 255 * np.pi),
            np.cos(i / 255 * 2 * np.pi), np.sin(i / 255 * 2 * np.pi)]
    a = olay.quad_dequant(c.reshape(1, -1), luts)
    b = oqp.decode_normalised(c, r_max)
    for k in range(4):
        np.testing.assert_allclose(a[k][0], b[k], rtol=1e-12, atol=1e-15)


def test_quad_layer_dequant_float32_mode_is_the_rounded_float64():
    """The float32 evaluation is the float64 decode up to the 3 roundings of its products
    (and the float32 LUTs), and every value is exactly a float32 product chain."""
    c = all_codes_sample(20000)
    i = np.arange(256, dtype=np.float64)
    r_max = 6.25
    luts64 = [(np.exp(i / 255 * math.log1p(255.0)) - 1) * r_max / 255.0,
              np.cos(i / 255 * np.pi), np.sin(i / 255 * np.pi), np.cos(i / 255 * np.pi), np.sin(i / 255 * np.pi),
              np.cos(i / 255 * 2 * np.pi), np.sin(i / 255 * 2 * np.pi)]
    luts32 = [l.astype(np.float32) for l in luts64]
    a = olay.quad_dequant(c.reshape(1, -1), luts32, dtype=np.float32)
    b = olay.quad_dequant(c.reshape(1, -1), luts32)                    # float64 on the same LUTs
    for k in range(4):
        assert a[k].dtype == np.float32
        np.testing.assert_allclose(a[k], b[k], rtol=4 * 2.0 ** -24, atol=1e-30)
    # spot-check one word against an explicit float32 chain
    w = int(c[123])
    nq, q1, q2, q3 = w >> 24, (w >> 16) & 255, (w >> 8) & 255, w & 255
    r = luts32[0][nq]
    rs = np.float32(r * luts32[2][q1])
    rss = np.float32(rs * luts32[4][q2])
    assert a[2][0, 123] == np.float32(rss * luts32[5][q3]) and a[1][0, 123] == np.float32(rs * luts32[3][q2])


def test_dual_layer_dequant_float32_mode_and_plug():
    """The float32 evaluation of the kernel-layout dual decode is the float64 one up to
    its two product roundings, each value is the explicit float32 chain
    (amp_lut * bmax) * cos, and a plug amplitude replaces amp_lut * bmax of its element."""
    K, N = 64, 48
    rng = np.random.default_rng(8)
    packed = olay.pack_amp_phase(rng.integers(0, 64, (K, N)), rng.integers(0, 1024, (K, N))).astype(np.int16)
    bmax = (rng.random((K * N + 31) // 32) * 2 + 0.01).astype(np.float16)
    i = np.arange(64, dtype=np.float64)
    amp_lut = ((np.exp(i / 63 * math.log1p(255.0)) - 1) / 255.0).astype(np.float16)
    ph = np.linspace(-math.pi, math.pi, 1025)[:-1]
    cos_lut, sin_lut = np.cos(ph).astype(np.float16), np.sin(ph).astype(np.float16)
    a = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut, dtype=np.float32)
    b = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    for x, y in zip(a, b):
        assert x.dtype == np.float32
        np.testing.assert_allclose(x, y, rtol=2 * 2.0 ** -24, atol=1e-30)
    k, n = 17, 45
    p = int(packed[k, n]) + 32768
    amp = np.float32(np.float32(amp_lut[(p >> 10) & 63]) * np.float32(bmax[(k * N + n) // 32]))
    assert a[0][k, n] == np.float32(amp * np.float32(cos_lut[p & 1023]))
    assert a[1][k, n] == np.float32(amp * np.float32(sin_lut[p & 1023]))
    kk, nn = np.array([3, 17]), np.array([5, 45])
    pa = np.array([0.25, 1.5], np.float16)
    c = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut, plug=(kk, nn, pa))
    ph_q = (packed.astype(np.int32) + 32768) & 1023
    for j in range(2):
        assert c[0][kk[j], nn[j]] == float(pa[j]) * float(cos_lut[ph_q[kk[j], nn[j]]])
        assert c[1][kk[j], nn[j]] == float(pa[j]) * float(sin_lut[ph_q[kk[j], nn[j]]])
    others = np.ones((K, N), bool)
    others[kk, nn] = False
    assert np.array_equal(c[0][others], b[0][others])


def test_dual_layer_dequant_group_index_and_offset():
    K, N = 5, 40
    rng = np.random.default_rng(2)
    amp = rng.integers(0, 64, (K, N))
    ph = rng.integers(0, 1024, (K, N))
    packed = olay.pack_amp_phase(amp, ph).astype(np.int16)
    bmax = (np.arange((K * N + 31) // 32) + 1).astype(np.float16)
    amp_lut = np.arange(64, dtype=np.float16)
    cos_lut = np.ones(1024, np.float16)
    sin_lut = np.arange(1024).astype(np.float16)
    w1, w2 = olay.dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut)
    flat = np.arange(K * N).reshape(K, N)
    np.testing.assert_array_equal(w1, amp * (flat // 32 + 1))
    np.testing.assert_array_equal(w2, amp * (flat // 32 + 1) * ph.astype(np.float16).astype(np.float64))


def test_gemm_f64_brute_force():
    rng = np.random.default_rng(4)
    a = rng.standard_normal((3, 7))
    w = rng.standard_normal((7, 5))
    y = olay.gemm_f64(a, w)
    for m in range(3):
        for n in range(5):
            assert abs(y[m, n] - sum(a[m, k] * w[k, n] for k in range(7))) < 1e-12


def test_pack_quad_layer_luts_closed_form():
    w = [torch.from_numpy(x.reshape(32, 16)) for x in gen.correlated_models(9, [512] * 4)]
    codes, luts, scales = olay.pack_quad_layer(*w)
    assert float(luts[0][0]) == 0.0
    assert float(luts[1][0]) == 1.0 and float(luts[2][0]) == 0.0 and float(luts[5][0]) == 1.0
    np.testing.assert_array_equal(luts[1], luts[3])
    np.testing.assert_array_equal(luts[2], luts[4])
    # norm[255] = r_max (rounded to fp16); r_max = 1.001 * max tuple norm
    wn = [x.double().numpy() / s for x, s in zip(w, scales)]
    rmax = 1.001 * np.sqrt(sum(x ** 2 for x in wn)).max()
    assert abs(float(luts[0][255]) - rmax) <= 2 ** -10 * rmax


def test_dual_layer_packer_scalar_rounding_modes():
    """The oracle's two scalar-rounding modes of quantize_polar_bitpacked: float32 weights
    give the same codes either way but for float32 reciprocal roundings (a few codes, one
    step); fp16 weights under the CPU rule equal an explicit chain with pi rounded to fp16
    for the add; under the GPU rule, an explicit float32 chain rounded to fp16 per op."""
    import math
    import torch
    from oracle import layer as olay
    import gen
    K, N = 64, 96
    ws = gen.correlated_models(21, [K * N] * 2)
    w32 = [torch.from_numpy(w.reshape(K, N)) for w in ws]
    a = olay.quantize_polar_bitpacked(*w32)[0].astype(np.int32)
    b = olay.quantize_polar_bitpacked(*w32, gpu_scalars=True)[0].astype(np.int32)
    d = np.abs((((a & 1023) - (b & 1023)) + 512) % 1024 - 512)
    assert (d > 0).sum() <= 10 and d.max() <= 1 and np.array_equal(a >> 10, b >> 10)
    w16 = [w.half() for w in w32]
    ph = torch.atan2(w16[1].float(), w16[0].float()).half().float()
    pi16 = float(torch.tensor(math.pi, dtype=torch.float16))
    cpu = torch.round((((ph + pi16).half().float() / (2 * math.pi)).half().float() * 1024).half()).long() % 1024
    inv = np.float32(1.0) / np.float32(2 * math.pi)
    gpu = torch.round((((ph + np.float32(math.pi)).half().float() * float(inv)).half().float() * 1024).half()).long() % 1024
    got_cpu = (olay.quantize_polar_bitpacked(*w16)[0].astype(np.int32) + 32768) & 1023
    got_gpu = (olay.quantize_polar_bitpacked(*w16, gpu_scalars=True)[0].astype(np.int32) + 32768) & 1023
    np.testing.assert_array_equal(got_cpu, cpu.numpy())
    np.testing.assert_array_equal(got_gpu, gpu.numpy())
    assert (got_cpu != got_gpu).mean() > 0.05       # the two rules really differ for fp16 weights
