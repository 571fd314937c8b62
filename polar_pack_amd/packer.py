"""Device-side packer for whole ``.quadpack`` streams (torch ops on the GPU).

Follows the three passes of pack_quad (quaternion_packer.py:52-132) on device
memory: per-model RMS over the common length (float64 accumulation, :59-68),
global ``r_max = 1.001 * max |w/s|`` (:70-77), then codes and plug entries
(:90-113).  Two plug selections:

* ``select="ref"``  -- the reference rule: threshold = percentile of the relative
  reconstruction error over 100 windows of 1,000,000 tuples drawn by
  ``numpy.random.default_rng(42)`` (:79-87), plug = error > threshold;
* ``select="norm"`` -- the top ``plug_cap`` fraction of tuples by norm (threshold
  from a strided sample), as the decode-step benchmark specifies.

Codes are computed in float32 like the reference's numpy pass; device
transcendentals can round differently at exact ties, so a few codes may differ by
one step from a host pack of the same weights (decode parity is unaffected: the
decoder is checked on whatever codes the stream holds).
"""
from __future__ import annotations

import math
from typing import List, Sequence

import numpy as np
import torch

from .container import QuadPackDevice

MU = 255.0


def _f32(x: float) -> float:
    return float(np.float32(x))


def quad_codes_f32(wn: Sequence[torch.Tensor], r_max: float):
    """uint32 words (int64 tensor) and float32 norm of normalised float32 tuples
    (quaternion_packer.py:22-39)."""
    w1, w2, w3, w4 = wn
    log_mu = math.log1p(MU)
    r = torch.sqrt(w1 ** 2 + w2 ** 2 + w3 ** 2 + w4 ** 2)
    t1 = torch.atan2(torch.sqrt(w2 ** 2 + w3 ** 2 + w4 ** 2), w1)
    t2 = torch.atan2(torch.sqrt(w3 ** 2 + w4 ** 2), w2)
    t3 = torch.remainder(torch.atan2(w4, w3), 2 * math.pi)
    nq = torch.round(torch.log1p(MU * r / r_max) / log_mu * 255).clamp(0, 255).to(torch.int64)
    q1 = torch.round(t1 / math.pi * 255).clamp(0, 255).to(torch.int64)
    q2 = torch.round(t2 / math.pi * 255).clamp(0, 255).to(torch.int64)
    q3 = torch.round(t3 / (2 * math.pi) * 255).clamp(0, 255).to(torch.int64)
    return (nq << 24) | (q1 << 16) | (q2 << 8) | q3, r


def _rel_err_f64(wn, words, r, r_max):
    """float64 relative reconstruction error (quaternion_packer.py:41-48)."""
    log_mu = math.log1p(MU)
    nq = (words >> 24).double()
    q1, q2, q3 = ((words >> 16) & 255).double(), ((words >> 8) & 255).double(), (words & 255).double()
    rr = (torch.exp(nq / 255 * log_mu) - 1) * r_max / MU
    s1 = torch.sin(q1 / 255 * math.pi)
    s2 = torch.sin(q2 / 255 * math.pi)
    rw = (rr * torch.cos(q1 / 255 * math.pi), rr * s1 * torch.cos(q2 / 255 * math.pi),
          rr * s1 * s2 * torch.cos(q3 / 255 * 2 * math.pi), rr * s1 * s2 * torch.sin(q3 / 255 * 2 * math.pi))
    e = sum((wn[k].double() - rw[k]) ** 2 for k in range(4))
    return torch.sqrt(e) / torch.clamp(r.double(), min=1e-12)


def pack_quad_device(models: List[List[torch.Tensor]], plug_cap: float = 0.001, select: str = "norm",
                     sample: int = 4_000_000) -> QuadPackDevice:
    """Pack 4 models given as lists of flat fp16/fp32 device tensors (one per projection,
    stream order; all 4 lists have the same lengths) into a device-resident stream."""
    if len(models) != 4 or len({len(m) for m in models}) != 1:
        raise ValueError("need 4 models with the same projection list")
    sizes = [int(t.numel()) for t in models[0]]
    for m in models:
        if [int(t.numel()) for t in m] != sizes:
            raise ValueError("per-model tails are not produced by the device packer; use equal lengths")
    n = sum(sizes)
    if n >= 2 ** 32:
        raise ValueError("a .quadpack stream indexes plug entries with uint32: n must be < 2^32")
    dev = models[0][0].device
    # pass A: RMS per model over the stream (float64 accumulation)
    s = []
    for m in models:
        acc = torch.zeros((), dtype=torch.float64, device=dev)
        for t in m:
            acc += (t.double() ** 2).sum()
        s.append(math.sqrt(float(acc) / n))
    # pass B: r_max, plus a strided norm sample for the 'norm' threshold
    r_max = 0.0
    samples = []
    stride = max(1, n // sample)
    for p in range(len(sizes)):
        wn = [models[k][p].float() / s[k] for k in range(4)]
        r = torch.sqrt(wn[0] ** 2 + wn[1] ** 2 + wn[2] ** 2 + wn[3] ** 2)
        r_max = max(r_max, float(r.max()))
        if select == "norm":
            samples.append(r[::stride].clone())
    r_max *= 1.001
    if select == "norm":
        allr = torch.cat(samples)
        k = max(1, int(round(allr.numel() * (1.0 - plug_cap))))
        thr = float(torch.kthvalue(allr.cpu(), min(k, allr.numel())).values) if plug_cap > 0 else float("inf")
    elif select == "ref":
        thr = _ref_threshold(models, s, sizes, r_max, plug_cap)
    else:
        raise ValueError("select must be 'norm' or 'ref'")
    # pass C: codes + plug
    codes = torch.empty(n, dtype=torch.int32, device=dev)
    pidx, pvals = [], []
    pos = 0
    for p, size in enumerate(sizes):
        wn = [models[k][p].float() / s[k] for k in range(4)]
        words, r = quad_codes_f32(wn, r_max)
        codes[pos:pos + size] = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
        if select == "norm":
            mask = r > thr
        else:
            mask = _rel_err_f64(wn, words, r, r_max) > thr
        nz = torch.nonzero(mask).flatten()
        if nz.numel():
            pidx.append((nz + pos).to(torch.int64))
            pvals.append(torch.stack([w[nz] for w in wn], dim=1).to(torch.float16))
        pos += size
    if pidx:
        pi = torch.cat(pidx)
        pi = torch.where(pi >= 2 ** 31, pi - 2 ** 32, pi).to(torch.int32).view(torch.uint32)
        pv = torch.cat(pvals)
    else:
        pi = torch.zeros(0, dtype=torch.int32, device=dev).view(torch.uint32)
        pv = torch.zeros((0, 4), dtype=torch.float16, device=dev)
    return QuadPackDevice(n=n, s=tuple(_f32(x) for x in s), r_max=_f32(r_max), codes=codes.view(torch.uint32),
                          plug_idx=pi, plug_vals=pv, tails=[torch.zeros(0, dtype=torch.float16, device=dev)] * 4)


def _ref_threshold(models, s, sizes, r_max, plug_cap):
    """Percentile of the relative error over the reference's 100 seeded windows."""
    n = sum(sizes)
    starts = np.random.default_rng(42).integers(0, n - 1_000_000, 100)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    errs = []
    for st in starts:
        parts = []
        for k in range(4):
            seg = []
            lo, hi = int(st), int(st) + 1_000_000
            for p in range(len(sizes)):
                a, b = max(lo, offs[p]), min(hi, offs[p + 1])
                if a < b:
                    seg.append(models[k][p][a - offs[p]:b - offs[p]].float())
            parts.append(torch.cat(seg) / s[k])
        words, r = quad_codes_f32(parts, r_max)
        errs.append(_rel_err_f64(parts, words, r, r_max).cpu().numpy())
    return float(np.percentile(np.concatenate(errs), (1 - plug_cap) * 100))
