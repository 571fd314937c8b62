"""Tolerance checks shared by the GPU parity tests.

* dequantised weights: within 1 fp16 ulp of the float64 oracle, compared after
  rounding both to fp16 (and the float32 value within 8 float32 ulps);
* GEMM/GEMV outputs (fp32 accumulate, fp16 out): per element
  |y - y_ref| <= 1e-3 * |y_ref| + 1e-5 * max|y_ref| + 2^-25, i.e. rel 1e-3 with a small
  absolute floor for outputs that cancel to near zero, and the fp16 output's own rounding
  below its normal range (half its smallest subnormal); products summed on the matrix
  cores (fp16 operands, fp32 sums: ~1e-6 of sum |w x| measured) add the dot-product
  bound 2^-18 * sum_k |w_k x_k|;
* codes, plug positions: bit-exact (checked by the tests directly).
"""
import numpy as np
import torch

GEMV_RTOL = 1e-3
GEMV_FLOOR = 1e-5
FP16_OUT_FLOOR = 2.0 ** -25    # an fp16 output rounds values below 2^-14 to a multiple of 2^-24


def fp16_ulp_distance(a, b):
    """|a - b| in fp16 ulps after rounding both to fp16 (ordered-integer distance)."""
    ia = np.asarray(a, np.float64).astype(np.float16).view(np.int16).astype(np.int32)
    ib = np.asarray(b, np.float64).astype(np.float16).view(np.int16).astype(np.int32)
    ia = np.where(ia < 0, -32768 - ia, ia)
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


def assert_dequant_close(got_f32, ref_f64, what=""):
    got = np.asarray(got_f32, np.float32)
    ref = np.asarray(ref_f64, np.float64)
    d = fp16_ulp_distance(got, ref)
    assert d.max() <= 1, f"{what}: dequant off by {d.max()} fp16 ulp at {np.unravel_index(d.argmax(), d.shape)}"
    tol = 8 * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) + 1e-30
    bad = np.abs(got.astype(np.float64) - ref) > tol
    assert not bad.any(), f"{what}: float32 dequant error beyond 8 ulp at {np.argwhere(bad)[:5]}"


def assert_gemv_close(got, ref, what="", rtol=GEMV_RTOL, floor=GEMV_FLOOR, bound=None):
    """``bound``: an extra per-element absolute allowance, e.g. the float32 dot-product
    error bound c * sum_k |w_k x_k| for products accumulated on the matrix cores."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max() if ref.size else 0.0
    err = np.abs(got - ref)
    lim = rtol * np.abs(ref) + floor * scale + FP16_OUT_FLOOR
    if bound is not None:
        lim = lim + bound
    worst = (err - lim).argmax() if ref.size else 0
    assert np.all(err <= lim), (f"{what}: |d|={err.flat[worst]:.3e} > {lim.flat[worst]:.3e} "
                                f"(ref {ref.flat[worst]:.4e}, got {got.flat[worst]:.4e}); "
                                f"normwise {err.max() / max(scale, 1e-300):.2e}")


def fp16_weight_bound(a, w):
    """Per-output allowance for weights rounded to fp16 before an fp32-accumulated dot
    product, as the reference kernels do (quad_kernels.py:117-126, polar_kernels.py:78-82)
    and the large-batch path (fp16 decode + library GEMM) does: each weight moves by at
    most 2^-11 of itself (2^-25 absolute below fp16's normal range), and the sum adds the
    float32 dot-product bound 2^-18 * sum_k |w_k x_k|."""
    a = np.abs(np.asarray(a, np.float64))
    w = np.abs(np.asarray(w, np.float64))
    return (2.0 ** -11 + 2.0 ** -18) * (a @ w) + 2.0 ** -25 * a.sum(axis=1, keepdims=True)


def normwise(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-300))


def dual_codes_u16(pack):
    """16-bit codes of a DualPackDevice (either layout) as uint32 numpy."""
    raw = pack.codes.cpu().numpy().view(np.uint16).astype(np.uint32)
    if pack.layout == "u16be":
        return ((raw & 0xFF) << 8) | (raw >> 8)
    return raw ^ 0x8000


def assert_same_dual_pack(pack, dp, max_code_flips=1e-4, min_plug_overlap=0.99):
    """Codes equal but for rare one-step flips at float32 rounding ties; scales
    bit-exact; the same plug count, nearly the same plug set, equal values where
    the positions agree."""
    assert pack.n_codes == dp.n_pairs
    got, ref = dual_codes_u16(pack), dp.codes_u16()
    diff = np.flatnonzero(got != ref)
    assert diff.size <= max(2, max_code_flips * got.size), f"{diff.size} of {got.size} codes differ"
    if diff.size:
        da = np.abs((got[diff] >> 10).astype(np.int64) - (ref[diff] >> 10).astype(np.int64))
        dph = np.abs((got[diff] & 1023).astype(np.int64) - (ref[diff] & 1023).astype(np.int64))
        dph = np.minimum(dph, 1024 - dph)
        assert np.all(da + dph == 1), "a differing code is more than one step away"
    np.testing.assert_array_equal(pack.scales.cpu().numpy().view(np.uint16), dp.scales.view(np.uint16))
    pi = pack.plug_idx.cpu().view(torch.int32).numpy().view(np.uint32)
    pv = pack.plug_val.cpu().numpy()
    assert pi.size == dp.plug_idx.size
    assert np.all(np.diff(pi.astype(np.int64)) > 0)
    common, ia, ib = np.intersect1d(pi, dp.plug_idx, return_indices=True)
    assert common.size >= min_plug_overlap * max(1, pi.size)
    np.testing.assert_array_equal(pv[ia].view(np.uint16), dp.plug_val[ib].view(np.uint16))
