"""``.quadpack`` v2 and ``.dualpack`` v2 containers: byte-exact readers/writers and
device upload.

Layouts are the reference's (quaternion_packer.py:13-19, 93-132, 146-167 and
polar_bitpack.py:26-29, 162-172, 195-211):

* ``.quadpack``: 82-byte little-endian header ``<4sBBQBBBBfQ4ff4Q`` (magic QUAD,
  version 2, 4 models, n, bits 8/8/8/8, mu, plug_n, s[4], r_max, tails[4]), then
  uint32 codes x n (at byte 82, so not 4-byte aligned), plug_idx uint32 x P,
  plug_vals fp16 x 4P (normalised), then each model's fp16 tail in model order.
* ``.dualpack``: 62-byte header ``<8s I Q Q Q B B f I Q Q`` (magic DUALPACK,
  version 2, n_pairs, n1, n2, amp_bits, phase_bits, mu, group_size, chunk_size,
  plug_n), then big-endian uint16 codes x n_pairs, fp16 scales (groups restart
  every chunk), plug_idx uint32 x P, plug amplitude fp16 x P.

Codes are copied into aligned device buffers unchanged (the big-endian dual codes
are decoded in-kernel; no re-layout pass).
"""
from __future__ import annotations

import math
import os
import struct
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch

QUAD_MAGIC, QUAD_VERSION = b"QUAD", 2
QUAD_HEADER = "<4sBBQBBBBfQ4ff4Q"
QUAD_HEADER_SIZE = struct.calcsize(QUAD_HEADER)       # 82
DUAL_MAGIC, DUAL_VERSION = b"DUALPACK", 2
DUAL_HEADER = "<8s I Q Q Q B B f I Q Q"
DUAL_HEADER_SIZE = struct.calcsize(DUAL_HEADER)       # 62


def _u32_tensor(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


def _read_array(f, dtype, count, chunk_bytes=1 << 28) -> np.ndarray:
    """Read `count` items into an aligned array (the file offset may be unaligned)."""
    out = np.empty(count, dtype=dtype)
    raw = out.view(np.uint8)
    pos = 0
    while pos < raw.size:
        n = f.readinto(memoryview(raw[pos:pos + chunk_bytes]))
        if not n:
            raise ValueError("file is shorter than its header implies")
        pos += n
    return out



def check_ascending(idx: np.ndarray) -> None:
    """Raise ValueError unless the plug positions are strictly ascending, as both containers
    store them (quaternion_packer.py:104-113, polar_bitpack.py:154-157)."""
    if idx.size > 1 and not bool(np.all(idx[1:].astype(np.int64) > idx[:-1].astype(np.int64))):
        raise ValueError("plug positions must be strictly ascending (as .quadpack / .dualpack files store them)")

@dataclass
class QuadPackFile:
    """A ``.quadpack`` v2 file's contents (host arrays)."""
    n: int
    s: tuple
    r_max: float
    codes: np.ndarray            # uint32 (n,)
    plug_idx: np.ndarray         # uint32 (P,)
    plug_vals: np.ndarray        # float16 (P, 4)
    tails: List[np.ndarray] = field(default_factory=lambda: [np.zeros(0, np.float16)] * 4)
    mu: float = 255.0

    @classmethod
    def read(cls, path) -> "QuadPackFile":
        size = os.path.getsize(path)
        with open(path, "rb") as f:
            hdr = struct.unpack(QUAD_HEADER, f.read(QUAD_HEADER_SIZE))
            magic, ver, nm, n, nb, b1, b2, b3, mu, plug_n = hdr[:10]
            if magic != QUAD_MAGIC or ver != QUAD_VERSION or nm != 4:
                raise ValueError(f"{path}: not a .quadpack v2 file")
            if (nb, b1, b2, b3) != (8, 8, 8, 8):
                raise ValueError(f"{path}: only 8/8/8/8-bit quad codes are defined")
            tails_n = hdr[15:19]
            need = QUAD_HEADER_SIZE + 4 * n + 12 * plug_n + 2 * sum(tails_n)
            if size < need:
                raise ValueError(f"{path}: {size} bytes, header implies {need}")
            codes = _read_array(f, "<u4", n)
            plug_idx = _read_array(f, "<u4", plug_n)
            plug_vals = _read_array(f, "<f2", 4 * plug_n).reshape(-1, 4)
            tails = [_read_array(f, "<f2", t) for t in tails_n]
        if plug_n and np.any(np.diff(plug_idx.astype(np.int64)) <= 0):
            raise ValueError(f"{path}: plug_idx is not strictly ascending")
        if plug_n and int(plug_idx[-1]) >= n:
            raise ValueError(f"{path}: plug_idx beyond the code stream")
        return cls(n=n, s=tuple(hdr[10:14]), r_max=hdr[14], codes=codes, plug_idx=plug_idx,
                   plug_vals=plug_vals, tails=tails, mu=mu)

    def header_bytes(self) -> bytes:
        return struct.pack(QUAD_HEADER, QUAD_MAGIC, QUAD_VERSION, 4, self.n, 8, 8, 8, 8, self.mu,
                           int(self.plug_idx.size), *self.s, self.r_max, *[int(t.size) for t in self.tails])

    def write(self, path) -> None:
        with open(path, "wb") as f:
            f.write(self.header_bytes())
            f.write(np.ascontiguousarray(self.codes, "<u4").tobytes())
            f.write(np.ascontiguousarray(self.plug_idx, "<u4").tobytes())
            f.write(np.ascontiguousarray(self.plug_vals, "<f2").tobytes())
            for t in self.tails:
                if t.size:
                    f.write(np.ascontiguousarray(t, "<f2").tobytes())

    def to_device(self, device) -> "QuadPackDevice":
        return QuadPackDevice(
            n=self.n, s=tuple(float(x) for x in self.s), r_max=float(self.r_max),
            codes=_u32_tensor(self.codes).to(device), plug_idx=_u32_tensor(self.plug_idx).to(device),
            plug_vals=torch.from_numpy(np.ascontiguousarray(self.plug_vals)).to(device),
            tails=[torch.from_numpy(np.ascontiguousarray(t)).to(device) for t in self.tails],
            plug_idx_host=self.plug_idx.copy())


@dataclass
class QuadPackDevice:
    """A quad stream resident in device memory (what the decode kernels read)."""
    n: int
    s: tuple
    r_max: float
    codes: torch.Tensor          # uint32 (n,)
    plug_idx: torch.Tensor       # uint32 (P,)
    plug_vals: torch.Tensor      # float16 (P, 4)
    tails: List[torch.Tensor]
    plug_idx_host: Optional[np.ndarray] = None
    plug_checked: bool = False

    @property
    def tail_lengths(self):
        return [int(t.numel()) for t in self.tails]

    def plug_host(self) -> np.ndarray:
        """Host copy of the plug positions, checked strictly ascending once (the stream planners
        slice them with searchsorted)."""
        if self.plug_idx_host is None:
            self.plug_idx_host = self.plug_idx.cpu().view(torch.int32).numpy().view(np.uint32)
        if not self.plug_checked:
            check_ascending(self.plug_idx_host)
            self.plug_checked = True
        return self.plug_idx_host

    def to_file(self) -> QuadPackFile:
        return QuadPackFile(n=self.n, s=self.s, r_max=self.r_max,
                            codes=self.codes.cpu().view(torch.int32).numpy().view(np.uint32),
                            plug_idx=self.plug_host(), plug_vals=self.plug_vals.cpu().numpy(),
                            tails=[t.cpu().numpy() for t in self.tails])


def dual_n_groups(n_pairs: int, chunk_size: int, gs: int) -> int:
    """Scale count; groups restart at every chunk (polar_bitpack.py:201-203)."""
    full, rest = divmod(n_pairs, chunk_size)
    return full * math.ceil(chunk_size / gs) + (math.ceil(rest / gs) if rest else 0)


@dataclass
class DualPackFile:
    """A ``.dualpack`` v2 file's contents (host arrays); codes stay big-endian."""
    n_pairs: int
    n1: int
    n2: int
    codes_be: np.ndarray         # uint8 (2 * n_pairs,)
    scales: np.ndarray           # float16 (n_groups,)
    plug_idx: np.ndarray         # uint32 (P,)
    plug_val: np.ndarray         # float16 (P,)
    amp_bits: int = 6
    phase_bits: int = 10
    mu: float = 255.0
    group_size: int = 32
    chunk_size: int = 50_000_000

    @classmethod
    def read(cls, path) -> "DualPackFile":
        size = os.path.getsize(path)
        with open(path, "rb") as f:
            (magic, ver, n_pairs, n1, n2, amp_bits, phase_bits, mu, gs, chunk,
             plug_n) = struct.unpack(DUAL_HEADER, f.read(DUAL_HEADER_SIZE))
            if magic != DUAL_MAGIC or ver != DUAL_VERSION:
                raise ValueError(f"{path}: wrong .dualpack format")
            if amp_bits + phase_bits != 16 or amp_bits > 6 or phase_bits > 10:
                raise ValueError(f"{path}: codes must be 6-bit amplitude + 10-bit phase")
            ng = dual_n_groups(n_pairs, chunk, gs)
            need = DUAL_HEADER_SIZE + 2 * n_pairs + 2 * ng + 6 * plug_n
            if size < need:
                raise ValueError(f"{path}: {size} bytes, header implies {need}")
            codes = _read_array(f, np.uint8, 2 * n_pairs)
            scales = _read_array(f, "<f2", ng)
            pi = _read_array(f, "<u4", plug_n)
            pv = _read_array(f, "<f2", plug_n)
        return cls(n_pairs=n_pairs, n1=n1, n2=n2, codes_be=codes, scales=scales, plug_idx=pi, plug_val=pv,
                   amp_bits=amp_bits, phase_bits=phase_bits, mu=mu, group_size=gs, chunk_size=chunk)

    def header_bytes(self) -> bytes:
        return struct.pack(DUAL_HEADER, DUAL_MAGIC, DUAL_VERSION, self.n_pairs, self.n1, self.n2, self.amp_bits,
                           self.phase_bits, float(self.mu), self.group_size, self.chunk_size, int(self.plug_idx.size))

    def write(self, path) -> None:
        with open(path, "wb") as f:
            f.write(self.header_bytes())
            f.write(np.ascontiguousarray(self.codes_be, np.uint8).tobytes())
            f.write(np.ascontiguousarray(self.scales, "<f2").tobytes())
            f.write(np.ascontiguousarray(self.plug_idx, "<u4").tobytes())
            f.write(np.ascontiguousarray(self.plug_val, "<f2").tobytes())

    def codes_device(self, device) -> torch.Tensor:
        """The big-endian codes as an int16 device tensor (bytes unchanged)."""
        return torch.from_numpy(self.codes_be.view(np.int16).copy()).to(device)

    def to_device(self, device) -> "DualPackDevice":
        """The stream in device memory, codes in the file's big-endian layout."""
        return DualPackDevice(
            n_codes=self.n_pairs, n1=self.n1, n2=self.n2, codes=self.codes_device(device), layout="u16be",
            scales=torch.from_numpy(np.ascontiguousarray(self.scales)).to(device),
            plug_idx=_u32_tensor(self.plug_idx).to(device),
            plug_val=torch.from_numpy(np.ascontiguousarray(self.plug_val)).to(device),
            amp_bits=self.amp_bits, phase_bits=self.phase_bits, mu=float(self.mu), group_size=self.group_size,
            chunk_size=self.chunk_size, plug_idx_host=self.plug_idx.copy())


@dataclass
class DualPackDevice:
    """A dual stream resident in device memory (what the stream decode reads).

    ``codes`` holds ``n_codes`` 16-bit pairs, either as the file stores them
    (``layout="u16be"``) or in the int16 kernel layout (``"i16"``).  ``tails`` is
    this build's extension for models of different lengths: model m's weights at
    positions ``n_codes ..`` as fp16 (the ``.dualpack`` format itself zero-pads the
    shorter model instead, polar_bitpack.py:113-117, and has no tails).
    """
    n_codes: int
    n1: int
    n2: int
    codes: torch.Tensor           # int16 (n_codes,)
    layout: str
    scales: torch.Tensor          # float16 (n_groups,)
    plug_idx: torch.Tensor        # uint32 as int32 (P,), ascending
    plug_val: torch.Tensor        # float16 (P,), absolute amplitude
    amp_bits: int = 6
    phase_bits: int = 10
    mu: float = 255.0
    group_size: int = 32
    chunk_size: int = 50_000_000
    tails: List[torch.Tensor] = field(default_factory=list)
    plug_idx_host: Optional[np.ndarray] = None
    plug_checked: bool = False

    @property
    def tail_lengths(self):
        t = list(self.tails) + [None] * (2 - len(self.tails))
        return [int(x.numel()) if x is not None else 0 for x in t]

    def plug_host(self) -> np.ndarray:
        """Host copy of the plug positions, checked strictly ascending once (the stream planners
        slice them with searchsorted)."""
        if self.plug_idx_host is None:
            self.plug_idx_host = self.plug_idx.cpu().view(torch.int32).numpy().view(np.uint32)
        if not self.plug_checked:
            check_ascending(self.plug_idx_host)
            self.plug_checked = True
        return self.plug_idx_host
