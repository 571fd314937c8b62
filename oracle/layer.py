"""Oracle for the kernel-layout operands (quad_kernels.py, polar_kernels.py).

Test infrastructure only (see :mod:`oracle`).  The two kernel-layout packers
are torch functions in the reference; they are restated here with torch on
the CPU and the same dtype flow, so that they match the reference's CPU
results bit for bit.  The dequant / GEMM references are float64 numpy.
"""
from __future__ import annotations

import math

import numpy as np
import torch

MU = 255.0   # quad_kernels.py:13


def pack_quad_layer(w1, w2, w3, w4, mu=MU):
    """Per-layer quad packer -- quad_kernels.py:16-50.

    Inputs: four (K, N) tensors.  Returns ``(codes uint32 (K,N) numpy,
    luts list of 7 fp16 numpy arrays [norm, cos1, sin1, cos2, sin2, cos3,
    sin3], scales list of 4 Python floats)``.
    """
    ws = [w1, w2, w3, w4]
    s = [torch.sqrt((w.float() ** 2).mean()) for w in ws]
    wn = [w.float() / sk for w, sk in zip(ws, s)]
    r = torch.sqrt(sum(x ** 2 for x in wn))
    r_max = float(r.max()) * 1.001
    log_mu = math.log1p(mu)
    t1 = torch.atan2(torch.sqrt(wn[1] ** 2 + wn[2] ** 2 + wn[3] ** 2), wn[0])
    t2 = torch.atan2(torch.sqrt(wn[2] ** 2 + wn[3] ** 2), wn[1])
    t3 = torch.atan2(wn[3], wn[2]) % (2 * math.pi)
    nq = torch.round(torch.log1p(mu * r / r_max) / log_mu * 255).clip(0, 255)
    q1 = torch.round(t1 / math.pi * 255).clip(0, 255)
    q2 = torch.round(t2 / math.pi * 255).clip(0, 255)
    q3 = torch.round(t3 / (2 * math.pi) * 255).clip(0, 255)
    u = [t.to(torch.int64).cpu().numpy().astype(np.uint32) for t in (nq, q1, q2, q3)]
    codes = ((u[0] << 24) | (u[1] << 16) | (u[2] << 8) | u[3]).astype(np.uint32)
    i = torch.arange(256, dtype=torch.float32)
    luts = [((torch.exp(i / 255 * log_mu) - 1) * r_max / mu),
            torch.cos(i / 255 * math.pi), torch.sin(i / 255 * math.pi),
            torch.cos(i / 255 * math.pi), torch.sin(i / 255 * math.pi),
            torch.cos(i / 255 * 2 * math.pi), torch.sin(i / 255 * 2 * math.pi)]
    luts = [t.to(torch.float16).numpy() for t in luts]
    return codes, luts, [float(sk) for sk in s]


def pack_amp_phase(amp_q, phase_q):
    """int16 code = ((amp & 63) << 10 | (phase & 1023)) - 32768 -- polar_kernels.py:9-11."""
    a = np.asarray(amp_q).astype(np.int32)
    p = np.asarray(phase_q).astype(np.int32)
    return (((a & 0x3F) << 10) | (p & 0x3FF)) - 32768


def _opmath(x, op, c):
    """``x op c`` as torch's GPU elementwise kernels evaluate a tensor-scalar operation: in
    float32 with the scalar as float32 (a division multiplies by the float32 reciprocal),
    rounded once to the tensor's dtype."""
    c32 = torch.tensor(c, dtype=torch.float32)
    y = x.float() + c32 if op == "+" else x.float() * (torch.tensor(1.0, dtype=torch.float32) / c32)
    return y.to(x.dtype)


def quantize_polar_bitpacked(w1, w2, amp_bits=6, num_phases=1024, mu=255, group_size=32, gpu_scalars=False):
    """Per-layer dual packer -- polar_kernels.py:118-151 (torch, CPU).

    Returns ``(packed int16 (K,N), bmax fp16 flat, amp_lut fp16[64],
    cos_lut fp16[1024], sin_lut fp16[1024])`` as numpy arrays.

    The reference function is torch code that runs on whichever device holds the weights,
    and torch rounds Python scalars differently there: on the CPU, ``fp16 + pi`` first
    rounds pi to fp16 (3.140625), while the GPU kernels keep scalars in float32 and
    divide by a scalar through its reciprocal.  ``gpu_scalars=True`` evaluates the
    scalar operations of the phase and amplitude codes the GPU's way (the reference's result for
    weights on a GPU); the default is the CPU's (the golden vectors were written there).
    """
    K, N = w1.shape
    amplitude = torch.sqrt(w1 ** 2 + w2 ** 2)
    phase = torch.atan2(w2, w1)
    if gpu_scalars:
        turns = _opmath(_opmath(phase, "+", math.pi), "/", 2 * math.pi)
    else:
        turns = (phase + math.pi) / (2 * math.pi)
    phase_q = (torch.round(turns * num_phases).long() % num_phases).to(torch.int16)
    total = K * N
    flat = amplitude.flatten()
    pad = (group_size - total % group_size) % group_size
    if pad:
        flat = torch.nn.functional.pad(flat, (0, pad))
    grouped = flat.reshape(-1, group_size)
    bmax = grouped.abs().max(dim=1, keepdim=True).values
    bmax = torch.where(bmax > 1e-10, bmax, torch.ones_like(bmax))
    norm = grouped / bmax
    log_mu = math.log(1 + mu)
    compressed = torch.sign(norm) * torch.log1p(mu * norm.abs())
    compressed = _opmath(compressed, "/", log_mu) if gpu_scalars else compressed / log_mu
    levels = (1 << amp_bits) - 1
    amp_q = torch.round(compressed * levels).clamp(0, levels).to(torch.int8).flatten()[:total].reshape(K, N)
    bmax = bmax.flatten().to(torch.float16)
    packed = pack_amp_phase(amp_q.numpy(), phase_q.numpy()).astype(np.int16)
    phases = torch.linspace(-math.pi, math.pi, num_phases + 1)[:-1]
    i = torch.arange(levels + 1, dtype=torch.float32)
    amp_lut = ((torch.exp(i / levels * log_mu) - 1.0) / mu).to(torch.float16)
    return (packed, bmax.numpy(), amp_lut.numpy(),
            torch.cos(phases).to(torch.float16).numpy(), torch.sin(phases).to(torch.float16).numpy())


def quad_dequant(codes, luts, scales=None, dtype=np.float64):
    """float64 (K,N) weights for kernel-layout codes -- quad_kernels.py:103-121.

    The float64 formula evaluated on the LUT values the caller passes
    (``luts`` = [norm, cos1, sin1, cos2, sin2, cos3, sin3]); multiplied by
    ``scales`` when given (quad_kernels.py:131-134 applies them to the
    accumulator, which is the same product).  ``dtype=np.float32`` evaluates the
    same products in float32 (r*c1, rs = r*s1, rs*c2, rss = rs*s2, rss*c3, rss*s3, each
    rounded once): the weights a kernel that decodes in float32 holds exactly, before
    it rounds them to fp16 operands.
    """
    c = np.asarray(codes, dtype=np.uint32)
    t = [np.asarray(l, dtype=np.float64).astype(dtype) for l in luts]
    nq, q1, q2, q3 = c >> 24, (c >> 16) & 255, (c >> 8) & 255, c & 255
    r = t[0][nq]
    rs = r * t[2][q1]
    rss = rs * t[4][q2]
    w = [r * t[1][q1], rs * t[3][q2], rss * t[5][q3], rss * t[6][q3]]
    if scales is not None:
        w = [wk.astype(np.float64) * float(sk) for wk, sk in zip(w, scales)]
    return w


def dual_dequant(packed, bmax, amp_lut, cos_lut, sin_lut, group_size=32, dtype=np.float64, plug=None):
    """(K,N) weight pair for kernel-layout codes -- polar_kernels.py:64-79.

    ``bmax`` is indexed by ``(k*N + n) // group_size`` over the (K,N)
    row-major flatten, as the reference kernel does (polar_kernels.py:70-71).
    ``dtype=np.float32`` evaluates the reference's products in float32 (amplitude =
    amp_lut * bmax, then amplitude * cos and amplitude * sin, each rounded once,
    polar_kernels.py:72-79): the values it rounds to fp16 before its dot products.
    ``plug=(k, n, amp)`` replaces the amplitude of those elements (polar_bitpack.py:240-243).
    """
    p = np.asarray(packed).astype(np.int32) + 32768
    K, N = p.shape
    amp_q = (p >> 10) & 0x3F
    ph = p & 0x3FF
    g = (np.arange(K)[:, None] * N + np.arange(N)[None, :]) // group_size
    amp = np.asarray(amp_lut, np.float64).astype(dtype)[amp_q] * np.asarray(bmax, np.float64).astype(dtype)[g]
    if plug is not None:
        kk, nn, pa = plug
        amp[kk, nn] = np.asarray(pa, np.float64).astype(dtype)
    return (amp * np.asarray(cos_lut, np.float64).astype(dtype)[ph],
            amp * np.asarray(sin_lut, np.float64).astype(dtype)[ph])


def gemm_f64(a, w):
    """``a @ w`` in float64 (a: (M,K), w: (K,N))."""
    return np.asarray(a, np.float64) @ np.asarray(w, np.float64)
