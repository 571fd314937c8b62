"""Oracle restatement of the ``.dualpack`` v2 container (polar_bitpack.py).

Test infrastructure only (see :mod:`oracle`).  numpy, single threaded, same
dtype flow as the reference (float32 polar transform, float64 mu-law
compression because ``np.log1p(int)`` is a float64 numpy scalar under
NEP 50, float64 unpack), polar_bitpack.py:34-76, 93-189, 194-260.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass

import numpy as np

MAGIC = b"DUALPACK"                         # polar_bitpack.py:26
VERSION = 2                                 # polar_bitpack.py:27
HEADER_FMT = "<8s I Q Q Q B B f I Q Q"      # polar_bitpack.py:28
HEADER_SIZE = struct.calcsize(HEADER_FMT)   # 62 bytes


@dataclass
class DualConfig:
    """Defaults of PackerConfig, polar_packer.py:34-41."""
    amp_bits: int = 6
    num_phases: int = 1024
    mu: int = 255
    plug_cap: float = 0.03
    group_size: int = 32
    chunk_size: int = 50_000_000


def quantize_amplitude_codes(amp_flat, cfg: DualConfig):
    """Per-group mu-law amplitude codes + plug -- polar_bitpack.py:34-76.

    Returns ``(amp_q uint8 flat, bmax fp16, plug_idx uint32, plug_val fp16, decoded f64)``.
    """
    levels = 2 ** cfg.amp_bits - 1
    ol = amp_flat.size
    gs = cfg.group_size
    pad = (gs - ol % gs) % gs
    if pad:
        amp_flat = np.pad(amp_flat, (0, pad))
    b = amp_flat.reshape(-1, gs)
    bmax = np.abs(b).max(axis=1, keepdims=True)
    bmax = np.where(bmax > 1e-10, bmax, 1.0)
    norm = b / bmax
    log_mu = np.log1p(cfg.mu)
    compressed = np.sign(norm) * np.log1p(cfg.mu * np.abs(norm)) / log_mu
    amp_q2d = np.round(compressed * levels).clip(0, levels).astype(np.uint8)
    decoded = (np.expm1(amp_q2d.astype(np.float64) / levels * log_mu) / cfg.mu * bmax).ravel()[:ol].copy()
    amp_q = amp_q2d.ravel()[:ol]
    plug_idx = np.zeros(0, np.uint32)
    plug_val = np.zeros(0, np.float16)
    if cfg.plug_cap > 0:
        core = b.ravel()[:ol]
        err = (core - decoded) ** 2
        n_plug = int(cfg.plug_cap * ol)
        if n_plug > 0:
            sel = np.argpartition(err, -n_plug)[-n_plug:]
            decoded[sel] = core[sel]
            plug_idx = sel.astype(np.uint32)
            plug_val = core[sel].astype(np.float16)
    return amp_q, bmax.astype(np.float16).ravel(), plug_idx, plug_val, decoded


def to_be_bytes(words):
    """uint16 codes as big-endian byte pairs -- polar_bitpack.py:81-85."""
    w = np.asarray(words, dtype=np.uint32)
    out = np.empty(w.size * 2, dtype=np.uint8)
    out[0::2] = ((w >> 8) & 0xFF).astype(np.uint8)
    out[1::2] = (w & 0xFF).astype(np.uint8)
    return out


def from_be_bytes(buf_u8):
    """Inverse of :func:`to_be_bytes` -- polar_bitpack.py:87-88."""
    b = np.asarray(buf_u8, dtype=np.uint8)
    return (b[0::2].astype(np.uint32) << 8) | b[1::2].astype(np.uint32)


def n_groups_for(n_pairs, chunk_size, gs):
    """Scale count; groups restart at every chunk -- polar_bitpack.py:201-203."""
    return sum(math.ceil(min(chunk_size, n_pairs - s) / gs) for s in range(0, n_pairs, chunk_size))


def group_index(pos, chunk_size, gs):
    """Scale index of stream position ``pos`` (groups restart per chunk, polar_bitpack.py:224-238)."""
    pos = np.asarray(pos, dtype=np.int64)
    per_chunk = -(-chunk_size // gs)
    return (pos // chunk_size) * per_chunk + (pos % chunk_size) // gs


@dataclass
class DualPack:
    """In-memory image of a ``.dualpack`` v2 file (polar_bitpack.py:162-172, 195-211)."""
    n_pairs: int
    n1: int
    n2: int
    codes_be: np.ndarray      # uint8 (2 * n_pairs,), big-endian u16 per pair
    scales: np.ndarray        # float16 (n_groups,)
    plug_idx: np.ndarray      # uint32 (P,), ascending
    plug_val: np.ndarray      # float16 (P,), absolute amplitude
    amp_bits: int = 6
    phase_bits: int = 10
    mu: float = 255.0
    group_size: int = 32
    chunk_size: int = 50_000_000

    def header_bytes(self) -> bytes:
        return struct.pack(HEADER_FMT, MAGIC, VERSION, self.n_pairs, self.n1, self.n2,
                           self.amp_bits, self.phase_bits, float(self.mu), self.group_size,
                           self.chunk_size, int(self.plug_idx.size))

    def to_bytes(self) -> bytes:
        return b"".join([self.header_bytes(), self.codes_be.tobytes(),
                         self.scales.astype("<f2").tobytes(),
                         self.plug_idx.astype("<u4").tobytes(),
                         self.plug_val.astype("<f2").tobytes()])

    @classmethod
    def from_bytes(cls, buf: bytes) -> "DualPack":
        (magic, ver, n_pairs, n1, n2, amp_bits, phase_bits, mu, gs, chunk,
         plug_n) = struct.unpack(HEADER_FMT, buf[:HEADER_SIZE])
        if magic != MAGIC or ver != VERSION:
            raise ValueError("wrong .dualpack format")
        ng = n_groups_for(n_pairs, chunk, gs)
        off = HEADER_SIZE
        codes = np.frombuffer(buf, dtype=np.uint8, count=2 * n_pairs, offset=off).copy()
        off += 2 * n_pairs
        scales = np.frombuffer(buf, dtype="<f2", count=ng, offset=off).copy()
        off += 2 * ng
        pi = np.frombuffer(buf, dtype="<u4", count=plug_n, offset=off).copy()
        off += 4 * plug_n
        pv = np.frombuffer(buf, dtype="<f2", count=plug_n, offset=off).copy()
        return cls(n_pairs=n_pairs, n1=n1, n2=n2, codes_be=codes, scales=scales,
                   plug_idx=pi, plug_val=pv, amp_bits=amp_bits, phase_bits=phase_bits,
                   mu=mu, group_size=gs, chunk_size=chunk)

    def codes_u16(self):
        return from_be_bytes(self.codes_be)


def pack_dual(w1, w2, cfg: DualConfig = DualConfig()) -> DualPack:
    """Chunked packer -- polar_bitpack.py:93-172 (statistics omitted).

    ``w1``/``w2`` are float32 flat streams of lengths n1, n2; the shorter one is
    zero-padded per chunk (polar_bitpack.py:113-117).
    """
    n1, n2 = len(w1), len(w2)
    phase_bits = 16 - cfg.amp_bits
    assert 2 ** phase_bits >= cfg.num_phases
    max_n = max(n1, n2)
    codes, scales, pis, pvs = [], [], [], []
    for start in range(0, max_n, cfg.chunk_size):
        end = min(start + cfg.chunk_size, max_n)
        a = np.array(w1[start:min(end, n1)], dtype=np.float32) if start < n1 else np.zeros(0, np.float32)
        b = np.array(w2[start:min(end, n2)], dtype=np.float32) if start < n2 else np.zeros(0, np.float32)
        L = max(len(a), len(b))
        if len(a) < L:
            a = np.pad(a, (0, L - len(a)))
        if len(b) < L:
            b = np.pad(b, (0, L - len(b)))
        amplitude = np.sqrt(a ** 2 + b ** 2)
        phase = np.arctan2(b, a)
        phase_idx = (np.round((phase + np.pi) / (2 * np.pi) * cfg.num_phases)
                     .astype(np.int64) % cfg.num_phases).astype(np.uint32)
        amp_q, bmax16, pidx, pval, _ = quantize_amplitude_codes(amplitude, cfg)
        if pidx.size:
            pis.append(pidx + np.uint32(start))
            pvs.append(pval)
        codes.append(to_be_bytes((amp_q.astype(np.uint32) << phase_bits) | phase_idx))
        scales.append(bmax16)
    pi = np.concatenate(pis) if pis else np.zeros(0, np.uint32)
    pv = np.concatenate(pvs) if pvs else np.zeros(0, np.float16)
    order = np.argsort(pi)
    return DualPack(n_pairs=max_n, n1=n1, n2=n2, codes_be=np.concatenate(codes) if codes else np.zeros(0, np.uint8),
                    scales=np.concatenate(scales) if scales else np.zeros(0, np.float16),
                    plug_idx=pi[order], plug_val=pv[order], amp_bits=cfg.amp_bits,
                    phase_bits=phase_bits, mu=float(cfg.mu), group_size=cfg.group_size,
                    chunk_size=cfg.chunk_size)


def decode_pairs_f64(dp: DualPack, lo=0, hi=None):
    """float64 (w1, w2) for pair positions [lo, hi) -- polar_bitpack.py:228-247.

    Amplitude follows :237-238 (float64 mu-law times fp16 scale, stored as
    float32), plug entries replace the amplitude (:240-243), and the final
    ``amp * cos(ang)`` stays float64 here (the reference then stores float32).
    """
    hi = dp.n_pairs if hi is None else hi
    levels = 2 ** dp.amp_bits - 1
    log_mu = np.log1p(dp.mu)
    phase_mask = (1 << dp.phase_bits) - 1
    codes = from_be_bytes(dp.codes_be[2 * lo:2 * hi])     # = dp.codes_u16()[lo:hi]
    amp_q = (codes >> dp.phase_bits) & levels
    phase_idx = codes & phase_mask
    pos = np.arange(lo, hi, dtype=np.int64)
    scale = dp.scales[group_index(pos, dp.chunk_size, dp.group_size)].astype(np.float32)
    amp_norm = np.expm1(amp_q.astype(np.float64) / levels * log_mu) / dp.mu
    amp = (amp_norm * scale).astype(np.float32)
    a = np.searchsorted(dp.plug_idx, lo)
    b = np.searchsorted(dp.plug_idx, hi)
    if b > a:
        amp[dp.plug_idx[a:b].astype(np.int64) - lo] = dp.plug_val[a:b].astype(np.float32)
    ang = phase_idx.astype(np.float64) / (phase_mask + 1) * 2 * np.pi - np.pi
    return amp * np.cos(ang), amp * np.sin(ang)


def unpack_dual(dp: DualPack):
    """float32 restored models truncated to n1 / n2 -- polar_bitpack.py:194-260."""
    out1 = np.empty(dp.n1, np.float32)
    out2 = np.empty(dp.n2, np.float32)
    for start in range(0, dp.n_pairs, dp.chunk_size):
        end = min(start + dp.chunk_size, dp.n_pairs)
        w1, w2 = decode_pairs_f64(dp, start, end)
        if start < dp.n1:
            out1[start:min(end, dp.n1)] = w1[:min(end, dp.n1) - start]
        if start < dp.n2:
            out2[start:min(end, dp.n2)] = w2[:min(end, dp.n2) - start]
    return out1, out2
