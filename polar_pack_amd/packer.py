"""Device-side packers for whole ``.quadpack`` and ``.dualpack`` streams (torch ops on the GPU).

:func:`pack_quad_device` follows the three passes of pack_quad (quaternion_packer.py:52-132) on device
memory: per-model RMS over the common length (float64 accumulation, :59-68),
global ``r_max = 1.001 * max |w/s|`` (:70-77), then codes and plug entries
(:90-113).  Two plug selections:

* ``select="ref"``  -- the reference rule: threshold = percentile of the relative
  reconstruction error over 100 windows of 1,000,000 tuples drawn by
  ``numpy.random.default_rng(42)`` (:79-87), plug = error > threshold;
* ``select="norm"`` -- the top ``plug_cap`` fraction of tuples by norm (threshold
  from a strided sample), as the decode-step benchmark specifies.

Codes are computed in float32 like the reference's numpy pass, with the same
operation order and IEEE divisions (never a multiply by a reciprocal); device
transcendentals can still round differently at exact ties, so a few codes may differ
by one step from a host pack of the same weights (decode parity is unaffected: the
decoder is checked on whatever codes the stream holds).  Models of unequal length
keep their positions past the common length as fp16 tails, as the reference does.

:func:`pack_dual_device` follows pack_dual_models_packed (polar_bitpack.py:93-172)
chunk by chunk.
"""
from __future__ import annotations

import math
from typing import List, Sequence

import numpy as np
import torch

from .container import DualPackDevice, QuadPackDevice

MU = 255.0


def _f32(x: float) -> float:
    return float(np.float32(x))


def _div(x: torch.Tensor, c: float) -> torch.Tensor:
    """x / float32(c), an element-wise IEEE division like numpy's (a Python-scalar divisor
    makes torch on the GPU multiply by its reciprocal instead, which rounds differently)."""
    return x / torch.tensor(c, dtype=torch.float32, device=x.device)


def quad_codes_f32(wn: Sequence[torch.Tensor], r_max: float):
    """uint32 words (int64 tensor) and float32 norm of normalised float32 tuples
    (quaternion_packer.py:22-39)."""
    w1, w2, w3, w4 = wn
    log_mu = math.log1p(MU)
    r = torch.sqrt(w1 ** 2 + w2 ** 2 + w3 ** 2 + w4 ** 2)
    t1 = torch.atan2(torch.sqrt(w2 ** 2 + w3 ** 2 + w4 ** 2), w1)
    t2 = torch.atan2(torch.sqrt(w3 ** 2 + w4 ** 2), w2)
    t3 = torch.remainder(torch.atan2(w4, w3), 2 * math.pi)
    nq = torch.round(_div(torch.log1p(_div(MU * r, r_max)), log_mu) * 255).clamp(0, 255).to(torch.int64)
    q1 = torch.round(_div(t1, math.pi) * 255).clamp(0, 255).to(torch.int64)
    q2 = torch.round(_div(t2, math.pi) * 255).clamp(0, 255).to(torch.int64)
    q3 = torch.round(_div(t3, 2 * math.pi) * 255).clamp(0, 255).to(torch.int64)
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


class _Flat:
    """A model given as a list of flat tensors, read as one stream by position."""

    def __init__(self, parts: Sequence[torch.Tensor]):
        self.parts = [t.reshape(-1) for t in parts]
        self.offs = np.concatenate([[0], np.cumsum([int(t.numel()) for t in self.parts])]).astype(np.int64)

    def __len__(self):
        return int(self.offs[-1])

    def slice(self, a: int, b: int) -> torch.Tensor:
        """Positions [a, b) (one view when they lie in one part)."""
        i = int(np.searchsorted(self.offs, a, side="right")) - 1
        pieces = []
        while a < b:
            lo, hi = int(self.offs[i]), int(self.offs[i + 1])
            take = min(b, hi)
            if take > a:
                pieces.append(self.parts[i][a - lo:take - lo])
                a = take
            i += 1
        return pieces[0] if len(pieces) == 1 else torch.cat(pieces)


def pack_quad_device(models: List[List[torch.Tensor]], plug_cap: float = 0.001, select: str = "norm",
                     sample: int = 4_000_000, threshold=None) -> QuadPackDevice:
    """Pack 4 models, each a list of flat fp16/fp32 device tensors (one per projection, stream
    order), into a device-resident stream.

    As quaternion_packer.py:54-56 and 121-126: ``n`` = the shortest model's length, every
    model's positions past ``n`` are kept as its fp16 tail.  The models' lists may cut the
    stream at different places; the work proceeds over the pieces between all of their
    cuts below ``n``.  ``threshold`` (``select="ref"`` only) replaces the sampled relative-error
    threshold, for streams of at most 1,000,000 tuples where the reference's window sampler
    cannot run."""
    if len(models) != 4:
        raise ValueError("need 4 models")
    flats = [_Flat(m) for m in models]
    lengths = [len(f) for f in flats]
    n = min(lengths)
    if n == 0:
        raise ValueError("every model must hold at least one weight")
    if n >= 2 ** 32:
        raise ValueError("a .quadpack stream indexes plug entries with uint32: n must be < 2^32")
    dev = flats[0].parts[0].device
    cuts = np.unique(np.concatenate([f.offs[(f.offs > 0) & (f.offs < n)] for f in flats] + [[0, n]]))
    pieces = list(zip(cuts[:-1].tolist(), cuts[1:].tolist()))
    # pass A: RMS per model over the common length (float64 accumulation, quaternion_packer.py:59-68)
    s = []
    for f in flats:
        acc = torch.zeros((), dtype=torch.float64, device=dev)
        for a, b in pieces:
            acc += (f.slice(a, b).double() ** 2).sum()
        s.append(math.sqrt(float(acc) / n))
    s32 = [torch.tensor(sk, dtype=torch.float32, device=dev) for sk in s]

    def normalised(a, b):
        return [f.slice(a, b).float() / sk for f, sk in zip(flats, s32)]

    # pass B: r_max (:70-77), plus a strided norm sample for the 'norm' threshold
    r_max = 0.0
    samples = []
    stride = max(1, n // sample)
    for a, b in pieces:
        wn = normalised(a, b)
        r = torch.sqrt(wn[0] ** 2 + wn[1] ** 2 + wn[2] ** 2 + wn[3] ** 2)
        r_max = max(r_max, float(r.max()))
        if select == "norm":
            samples.append(r[(-a) % stride::stride].clone())
    r_max *= 1.001
    if select == "norm":
        allr = torch.cat(samples)
        k = max(1, int(round(allr.numel() * (1.0 - plug_cap))))
        thr = float(torch.kthvalue(allr.cpu(), min(k, allr.numel())).values) if plug_cap > 0 else float("inf")
    elif select == "ref":
        thr = _ref_threshold(normalised, n, r_max, plug_cap) if threshold is None else float(threshold)
    else:
        raise ValueError("select must be 'norm' or 'ref'")
    # pass C: codes + plug (:90-113)
    codes = torch.empty(n, dtype=torch.int32, device=dev)
    pidx, pvals = [], []
    for a, b in pieces:
        wn = normalised(a, b)
        words, r = quad_codes_f32(wn, r_max)
        codes[a:b] = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
        if select == "norm":
            mask = r > thr
        else:
            mask = _rel_err_f64(wn, words, r, r_max) > thr
        nz = torch.nonzero(mask).flatten()
        if nz.numel():
            pidx.append((nz + a).to(torch.int64))
            pvals.append(torch.stack([w[nz] for w in wn], dim=1).to(torch.float16))
    if pidx:
        pi = torch.cat(pidx)
        pi = torch.where(pi >= 2 ** 31, pi - 2 ** 32, pi).to(torch.int32).view(torch.uint32)
        pv = torch.cat(pvals)
    else:
        pi = torch.zeros(0, dtype=torch.int32, device=dev).view(torch.uint32)
        pv = torch.zeros((0, 4), dtype=torch.float16, device=dev)
    # per-model fp16 tails (:121-126)
    tails = [f.slice(n, L).to(torch.float16).contiguous() if L > n else torch.zeros(0, dtype=torch.float16, device=dev)
             for f, L in zip(flats, lengths)]
    return QuadPackDevice(n=n, s=tuple(_f32(x) for x in s), r_max=_f32(r_max), codes=codes.view(torch.uint32),
                          plug_idx=pi, plug_vals=pv, tails=tails)


def _ref_threshold(normalised, n, r_max, plug_cap):
    """Percentile of the relative error over the reference's 100 seeded windows of 1,000,000
    tuples (quaternion_packer.py:79-87; like the reference, needs n > 1,000,000)."""
    if n <= 1_000_000:
        raise ValueError("the reference's plug threshold samples windows of 1,000,000 tuples: n must exceed that")
    starts = np.random.default_rng(42).integers(0, n - 1_000_000, 100)
    errs = []
    for st in starts:
        parts = normalised(int(st), int(st) + 1_000_000)
        words, r = quad_codes_f32(parts, r_max)
        errs.append(_rel_err_f64(parts, words, r, r_max).cpu().numpy())
    return float(np.percentile(np.concatenate(errs), (1 - plug_cap) * 100))


def _dual_chunk(a: torch.Tensor, b: torch.Tensor, amp_bits: int, num_phases: int, mu: float, gs: int,
                plug_cap: float, select: str):
    """One chunk of pack_dual_models_packed (polar_bitpack.py:118-150): float32 polar
    transform, per-group mu-law amplitude codes (quantize_amplitude_codes, :34-76) and
    the chunk's plug entries.  Returns (16-bit codes as int32, fp16 scales, plug
    positions within the chunk, fp16 plug amplitudes)."""
    levels = 2 ** amp_bits - 1
    phase_bits = 16 - amp_bits
    amplitude = torch.sqrt(a * a + b * b)
    phase = torch.atan2(b, a)
    phase_idx = torch.remainder(torch.round((phase + math.pi) / (2 * math.pi) * num_phases).to(torch.int64),
                                num_phases)
    del phase
    ol = amplitude.numel()
    pad = (-ol) % gs
    g = torch.nn.functional.pad(amplitude, (0, pad)).view(-1, gs)
    bmax = g.abs().amax(dim=1, keepdim=True)
    bmax = torch.where(bmax > 1e-10, bmax, torch.ones_like(bmax))
    norm = g / bmax
    log_mu = math.log1p(mu)
    # float32 log1p, then the float64 division by ln(1+mu) (a float64 numpy scalar, :52-53)
    comp = (torch.sign(norm) * torch.log1p(mu * norm.abs())).double() / log_mu
    del norm
    amp_q = torch.round(comp * levels).clamp(0, levels).to(torch.int64)
    del comp
    pidx = pval = None
    n_plug = int(plug_cap * ol)
    if n_plug > 0:
        if select == "ref":       # top n_plug by squared amplitude error (:62-74)
            decoded = torch.expm1(amp_q.double() / levels * log_mu) / mu * bmax.double()
            err = (amplitude.double() - decoded.reshape(-1)[:ol]) ** 2
            del decoded
        elif select == "norm":    # top n_plug by amplitude
            err = amplitude
        else:
            raise ValueError("select must be 'ref' or 'norm'")
        pidx = torch.topk(err, n_plug, sorted=False).indices
        del err
        pidx = torch.sort(pidx).values
        pval = amplitude[pidx].to(torch.float16)
    codes = (amp_q.reshape(-1)[:ol] << phase_bits) | phase_idx
    return codes.to(torch.int32), bmax.reshape(-1).to(torch.float16), pidx, pval


def pack_dual_device(w1: torch.Tensor, w2: torch.Tensor, *, plug_cap: float = 0.03, select: str = "ref",
                     amp_bits: int = 6, num_phases: int = 1024, mu: float = 255.0, group_size: int = 32,
                     chunk_size: int = 50_000_000, tails: bool = False, layout: str = "u16be") -> DualPackDevice:
    """Pack two flat weight streams (any float dtype, on any torch device) as
    pack_dual_models_packed does (polar_bitpack.py:93-172), chunk by chunk.

    ``tails=False`` is the ``.dualpack`` format: ``n_pairs = max(n1, n2)`` and the
    shorter model is zero-padded (:113-117).  ``tails=True`` is this build's
    extension: codes cover the common length rounded down to a multiple of 8
    (``8 * (min(n1, n2) // 8)``, so that tail rows can be read with aligned 16-byte
    loads) and each model's remaining weights are kept as its fp16 tail.

    ``select="ref"`` is the reference's plug rule, the top ``int(plug_cap * L)``
    pairs of each chunk of L pairs by squared amplitude error; ``select="norm"``
    takes the top pairs by amplitude instead.  Codes come from float32 device
    transcendentals: a code can differ by one step from a host pack of the same
    weights at an exact rounding tie, and tied plug candidates may be chosen
    differently (the decode is checked on whatever the stream holds).
    ``layout`` is ``"u16be"`` (the file's big-endian 16-bit words) or ``"i16"``
    (the kernel layout, code - 32768).
    """
    if w1.dim() != 1 or w2.dim() != 1 or w1.device != w2.device:
        raise ValueError("w1 and w2 must be flat tensors on one device")
    if amp_bits > 6 or 16 - amp_bits > 10 or (1 << (16 - amp_bits)) < num_phases:
        raise ValueError("codes are 6-bit amplitude + 10-bit phase")
    if group_size < 1 or chunk_size < 1:
        raise ValueError("group_size and chunk_size must be positive")
    if layout not in ("u16be", "i16"):
        raise ValueError("layout must be 'u16be' or 'i16'")
    n1, n2 = int(w1.numel()), int(w2.numel())
    n = 8 * (min(n1, n2) // 8) if tails else max(n1, n2)
    if n >= 2 ** 32:
        raise ValueError("plug positions are uint32: the stream must hold fewer than 2^32 pairs")
    dev = w1.device
    codes = torch.empty(n, dtype=torch.int16, device=dev)
    scales, pis, pvs = [], [], []
    for start in range(0, n, chunk_size):
        end = min(start + chunk_size, n)
        a = w1[start:min(end, n1)].float()
        b = w2[start:min(end, n2)].float()
        L = end - start
        if a.numel() < L:
            a = torch.nn.functional.pad(a, (0, L - a.numel()))
        if b.numel() < L:
            b = torch.nn.functional.pad(b, (0, L - b.numel()))
        c, sc, pidx, pval = _dual_chunk(a, b, amp_bits, num_phases, mu, group_size, plug_cap, select)
        del a, b
        if layout == "u16be":
            c = ((c & 0xFF) << 8) | (c >> 8)
        else:
            c = c ^ 0x8000
        codes[start:end] = torch.where(c >= 0x8000, c - 0x10000, c).to(torch.int16)
        del c
        scales.append(sc)
        if pidx is not None:
            pis.append(pidx + start)
            pvs.append(pval)
    pi = torch.cat(pis) if pis else torch.zeros(0, dtype=torch.int64, device=dev)
    pv = torch.cat(pvs) if pvs else torch.zeros(0, dtype=torch.float16, device=dev)
    pi = torch.where(pi >= 2 ** 31, pi - 2 ** 32, pi).to(torch.int32).view(torch.uint32)
    tail_list = []
    if tails:
        tail_list = [w1[n:].to(torch.float16).contiguous(), w2[n:].to(torch.float16).contiguous()]
    return DualPackDevice(n_codes=n, n1=n1, n2=n2, codes=codes, layout=layout,
                          scales=torch.cat(scales) if scales else torch.zeros(0, dtype=torch.float16, device=dev),
                          plug_idx=pi, plug_val=pv, amp_bits=amp_bits, phase_bits=16 - amp_bits, mu=float(mu),
                          group_size=group_size, chunk_size=chunk_size, tails=tail_list)
