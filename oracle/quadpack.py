"""Oracle restatement of the ``.quadpack`` v2 container (quaternion_packer.py).

Test infrastructure only (see :mod:`oracle`).  numpy, single threaded, with
the same dtype flow as the reference so that packer outputs are bit-exact on
the same numpy build:

* angles / norm codes are computed in float32 (inputs are float32 and the
  Python-float constants are weak scalars under NEP 50),
  quaternion_packer.py:22-39;
* reconstruction, relative error and unpack run in float64,
  quaternion_packer.py:41-48, 173-196.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = b"QUAD"                       # quaternion_packer.py:13
VERSION = 2                           # quaternion_packer.py:14
N_MODELS = 4                          # quaternion_packer.py:15
MU = 255.0                            # quaternion_packer.py:16
CHUNK = 100_000_000                   # quaternion_packer.py:17
HEADER_FMT = "<4sBBQBBBBfQ4ff4Q"      # quaternion_packer.py:18
HEADER_SIZE = struct.calcsize(HEADER_FMT)   # 82 bytes, quaternion_packer.py:19
PLUG_WINDOW = 1_000_000               # quaternion_packer.py:80,83
PLUG_WINDOWS = 100                    # quaternion_packer.py:80


def to_hyperspherical(w1, w2, w3, w4):
    """quaternion_packer.py:22-27 -- (r, t1, t2, t3); float32 in, float32 out."""
    r = np.sqrt(w1 ** 2 + w2 ** 2 + w3 ** 2 + w4 ** 2)
    t1 = np.arctan2(np.sqrt(w2 ** 2 + w3 ** 2 + w4 ** 2), w1)
    t2 = np.arctan2(np.sqrt(w3 ** 2 + w4 ** 2), w2)
    t3 = np.mod(np.arctan2(w4, w3), 2 * np.pi)
    return r, t1, t2, t3


def decode_fields(codes):
    """Split uint32 words into (nq, q1, q2, q3) -- quaternion_packer.py:173-176."""
    c = np.asarray(codes, dtype=np.uint32)
    return c >> 24, (c >> 16) & 255, (c >> 8) & 255, c & 255


def decode_normalised(codes, r_max, mu=MU):
    """float64 normalised 4-tuples from codes -- quaternion_packer.py:178-185.

    ``r_max`` is the value the unpacker reads from the header (a float32
    widened to float64).  Returns a tuple of 4 float64 arrays.
    """
    nq, q1, q2, q3 = decode_fields(codes)
    log_mu = math.log1p(MU)
    r_rest = (np.exp(nq / 255 * log_mu) - 1) * r_max / mu
    t1 = q1 / 255 * np.pi
    t2 = q2 / 255 * np.pi
    t3 = q3 / 255 * 2 * np.pi
    return (r_rest * np.cos(t1),
            r_rest * np.sin(t1) * np.cos(t2),
            r_rest * np.sin(t1) * np.sin(t2) * np.cos(t3),
            r_rest * np.sin(t1) * np.sin(t2) * np.sin(t3))


def quantize_chunk(wc, r_max, collect_error=False):
    """Codes (and float64 relative error) for one chunk -- quaternion_packer.py:30-49."""
    log_mu = math.log1p(MU)
    r, t1, t2, t3 = to_hyperspherical(*wc)
    nq = np.round(np.log1p(MU * r / r_max) / log_mu * 255).clip(0, 255).astype(np.uint32)
    q1 = np.round(t1 / np.pi * 255).clip(0, 255).astype(np.uint32)
    q2 = np.round(t2 / np.pi * 255).clip(0, 255).astype(np.uint32)
    q3 = np.round(t3 / (2 * np.pi) * 255).clip(0, 255).astype(np.uint32)
    codes = (nq << 24) | (q1 << 16) | (q2 << 8) | q3
    if not collect_error:
        return codes
    r_rest = (np.exp(nq / 255 * log_mu) - 1) * r_max / MU
    s1 = np.sin(q1 / 255 * np.pi)
    s2 = np.sin(q2 / 255 * np.pi)
    rw = (r_rest * np.cos(q1 / 255 * np.pi),
          r_rest * s1 * np.cos(q2 / 255 * np.pi),
          r_rest * s1 * s2 * np.cos(q3 / 255 * 2 * np.pi),
          r_rest * s1 * s2 * np.sin(q3 / 255 * 2 * np.pi))
    err = np.sqrt(sum((wc[k] - rw[k]) ** 2 for k in range(4))) / np.maximum(r, 1e-12)
    return codes, err


@dataclass
class QuadPack:
    """In-memory image of a ``.quadpack`` v2 file (quaternion_packer.py:13-19, 93-132)."""
    n: int
    s: tuple                      # per-model RMS, float32 values as Python floats
    r_max: float                  # float32 value as Python float
    codes: np.ndarray             # uint32 (n,)
    plug_idx: np.ndarray          # uint32 (P,), ascending
    plug_vals: np.ndarray         # float16 (P, 4), normalised (pre-RMS) values
    tails: list = field(default_factory=lambda: [np.zeros(0, np.float16)] * 4)
    mu: float = MU

    @property
    def tail_lengths(self):
        return [int(t.size) for t in self.tails]

    def header_bytes(self) -> bytes:
        return struct.pack(HEADER_FMT, MAGIC, VERSION, N_MODELS, self.n, 8, 8, 8, 8,
                           self.mu, int(self.plug_idx.size), *self.s, self.r_max,
                           *self.tail_lengths)

    def to_bytes(self) -> bytes:
        """File bytes in the order quaternion_packer.py:92-126 writes them."""
        parts = [self.header_bytes(), self.codes.astype("<u4").tobytes(),
                 self.plug_idx.astype("<u4").tobytes(),
                 self.plug_vals.astype("<f2").reshape(-1, 4).tobytes()]
        parts += [t.astype("<f2").tobytes() for t in self.tails if t.size]
        return b"".join(parts)

    @classmethod
    def from_bytes(cls, buf: bytes) -> "QuadPack":
        """Parse a file image -- quaternion_packer.py:146-164, 201-209."""
        hdr = struct.unpack(HEADER_FMT, buf[:HEADER_SIZE])
        magic, ver, nm, n, nb, b1, b2, b3, mu, plug_n = hdr[:10]
        if magic != MAGIC or ver != VERSION:
            raise ValueError("not a .quadpack v2 file")
        s = tuple(hdr[10:14])
        r_max = hdr[14]
        tails_n = hdr[15:19]
        off = HEADER_SIZE
        codes = np.frombuffer(buf, dtype="<u4", count=n, offset=off).copy()
        off += 4 * n
        plug_idx = np.frombuffer(buf, dtype="<u4", count=plug_n, offset=off).copy()
        off += 4 * plug_n
        plug_vals = np.frombuffer(buf, dtype="<f2", count=4 * plug_n, offset=off).reshape(-1, 4).copy()
        off += 8 * plug_n
        tails = []
        for t in tails_n:
            tails.append(np.frombuffer(buf, dtype="<f2", count=t, offset=off).copy())
            off += 2 * t
        return cls(n=n, s=s, r_max=r_max, codes=codes, plug_idx=plug_idx,
                   plug_vals=plug_vals, tails=tails, mu=mu)


def _f32(x: float) -> float:
    """Round a Python float through float32 (what the header stores)."""
    return float(np.float32(x))


def rms_scales(models, n):
    """Pass A: per-model RMS over the common length -- quaternion_packer.py:59-68."""
    s = []
    for m in models:
        acc = 0.0
        for i in range(0, n, CHUNK):
            c = np.asarray(m[i:min(i + CHUNK, n)], dtype=np.float64)
            acc += np.sum(c * c)
        s.append(math.sqrt(acc / n))
    return s


def global_rmax(models, s, n):
    """Pass B, first half: 1.001 * max tuple norm -- quaternion_packer.py:70-77."""
    r_max = 0.0
    for i in range(0, n, CHUNK):
        j = min(i + CHUNK, n)
        wc = [np.asarray(m[i:j], dtype=np.float32) / sk for m, sk in zip(models, s)]
        r_max = max(r_max, float(np.max(np.sqrt(sum(x ** 2 for x in wc)))))
    return r_max * 1.001


def plug_threshold(models, s, n, r_max, plug_cap):
    """Pass B, second half: error percentile over 100 seeded windows -- quaternion_packer.py:79-87.

    Needs ``n > 1_000_000`` exactly as the reference does (``rng.integers``
    raises otherwise).
    """
    rng = np.random.default_rng(42)
    starts = rng.integers(0, n - PLUG_WINDOW, PLUG_WINDOWS)
    errs = []
    for st in starts:
        wc = [np.asarray(m[st:st + PLUG_WINDOW], dtype=np.float32) / sk for m, sk in zip(models, s)]
        errs.append(quantize_chunk(wc, r_max, collect_error=True)[1])
    return float(np.percentile(np.concatenate(errs), (1 - plug_cap) * 100))


def pack_quad(models, plug_cap=0.05, threshold=None) -> QuadPack:
    """Three-pass packer -- quaternion_packer.py:52-132.

    ``threshold`` overrides the sampled plug threshold (used for inputs with
    ``n <= 1_000_000``, where the reference's window sampler cannot run).
    """
    lengths = [len(m) for m in models]
    n = min(lengths)
    s = rms_scales(models, n)
    r_max = global_rmax(models, s, n)
    thr = plug_threshold(models, s, n, r_max, plug_cap) if threshold is None else float(threshold)
    codes = np.empty(n, dtype=np.uint32)
    plug_idx, plug_vals = [], []
    for i in range(0, n, CHUNK):
        j = min(i + CHUNK, n)
        wc = [np.asarray(m[i:j], dtype=np.float32) / sk for m, sk in zip(models, s)]
        c, err = quantize_chunk(wc, r_max, collect_error=True)
        codes[i:j] = c
        mask = err > thr
        if mask.any():
            plug_idx.append((np.nonzero(mask)[0] + i).astype(np.uint32))
            plug_vals.append(np.stack([wc[k][mask] for k in range(4)], axis=1).astype(np.float16))
    pi = np.concatenate(plug_idx) if plug_idx else np.zeros(0, np.uint32)
    pv = np.concatenate(plug_vals) if plug_vals else np.zeros((0, 4), np.float16)
    tails = [np.asarray(m[n:], dtype=np.float16) for m in models]
    # the header stores float32 s and r_max (struct 'f'), quaternion_packer.py:93-94
    return QuadPack(n=n, s=tuple(_f32(x) for x in s), r_max=_f32(r_max), codes=codes,
                    plug_idx=pi, plug_vals=pv, tails=tails)


def unpack_quad(qp: QuadPack):
    """float32 restored models -- quaternion_packer.py:141-214.

    Decodes with the header's float32 ``r_max`` and ``s`` (:148-151), patches
    plug entries with their normalised fp16 values (:187-193), multiplies by
    ``s_k`` (:195-196) and appends the fp16 tails (:201-210).
    """
    n = qp.n
    tl = qp.tail_lengths
    outs = [np.empty(n + tl[k], dtype=np.float32) for k in range(4)]
    for i in range(0, n, CHUNK):
        j = min(i + CHUNK, n)
        rw = [np.array(a) for a in decode_normalised(qp.codes[i:j], qp.r_max)]
        if qp.plug_idx.size:
            lo = np.searchsorted(qp.plug_idx, i)
            hi = np.searchsorted(qp.plug_idx, j)
            if hi > lo:
                pos = qp.plug_idx[lo:hi].astype(np.int64) - i
                for k in range(4):
                    rw[k][pos] = qp.plug_vals[lo:hi, k].astype(np.float32)
        for k in range(4):
            outs[k][i:j] = rw[k] * qp.s[k]
    for k in range(4):
        if tl[k]:
            outs[k][n:] = qp.tails[k].astype(np.float32)
    return outs


def unpack_quad_f64(qp: QuadPack, lo=0, hi=None):
    """float64 restored weights for stream positions [lo, hi) before the float32
    store of quaternion_packer.py:196; positions past ``n`` come from the tails
    (NaN where a model has no weight)."""
    n = qp.n
    hi = max(n + max(qp.tail_lengths), lo) if hi is None else hi
    outs = [np.full(hi - lo, np.nan) for _ in range(4)]
    clo, chi = min(lo, n), min(hi, n)
    if chi > clo:
        rw = [np.array(a) for a in decode_normalised(qp.codes[clo:chi], qp.r_max)]
        if qp.plug_idx.size:
            a = np.searchsorted(qp.plug_idx, clo)
            b = np.searchsorted(qp.plug_idx, chi)
            pos = qp.plug_idx[a:b].astype(np.int64) - clo
            for k in range(4):
                rw[k][pos] = qp.plug_vals[a:b, k].astype(np.float64)
        for k in range(4):
            outs[k][clo - lo:chi - lo] = rw[k] * qp.s[k]
    for k in range(4):
        t = qp.tails[k]
        tlo, thi = max(lo, n), min(hi, n + t.size)
        if thi > tlo:
            outs[k][tlo - lo:thi - lo] = t[tlo - n:thi - n].astype(np.float64)
    return outs
