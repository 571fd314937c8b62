"""Whole-stream decode step: every projection of a ``.quadpack`` stream in one launch.

A stream is the reference's flat Linear order (polar_main.py:33-43): projection p
is an (N_p, K_p) row-major block at stream position pos_p = sum of the previous
N*K.  :class:`QuadStream` turns the stream into wavefront tasks once:

* rows fully inside the code stream -> items of up to ``rows_per_item`` full rows
  (a wavefront walks the whole K of its rows, so nothing is combined across waves);
* rows that reach the FP16 tails (positions >= n) -> one-row TAIL items;
* each item carries its plug range (searchsorted of the sorted plug_idx over its
  rows, as quaternion_packer.py:188-189 does per chunk);
* wavefront w runs items [bounds[w], bounds[w+1]), balanced by bytes.

``bind`` fixes the activation / output buffers, ``__call__`` launches
``pp_quad_stream`` on the current torch stream.
"""
from __future__ import annotations

import ctypes as C
from typing import List, Sequence, Tuple

import numpy as np
import torch

from . import _native as nat
from .container import QuadPackDevice
from .quad_kernels import header_luts

ITEM_DTYPE = np.dtype([("proj", "<i4"), ("row0", "<i4"), ("nrows", "<i4"), ("flags", "<i4"),
                       ("plug_lo", "<i8"), ("plug_hi", "<i8")])
PROJ_DTYPE = np.dtype([("codes", "<u8"), ("ldc", "<i8"), ("pos0", "<i8"), ("x", "<u8"), ("x_sm", "<i8"),
                       ("out", "<u8", (4,)), ("o_sm", "<i8"), ("N", "<i4"), ("K", "<i4")])
SEG = 256


def plan_items(shapes, n, plug_host, rows_per_item):
    """Wavefront tasks of a stream (pure host logic).

    Rows fully below the code count ``n`` become items of up to ``rows_per_item``
    full rows; rows that reach position ``n`` become one-row TAIL items.  Each item
    carries the range of sorted plug entries that fall in its rows.
    """
    pos = np.cumsum([0] + [int(a) * int(b) for a, b in shapes])
    parts = []
    for p, ((N, K), pos0) in enumerate(zip(shapes, pos[:-1])):
        N, K, pos0 = int(N), int(K), int(pos0)
        r_full = int(np.clip((n - pos0) // K, 0, N))
        if r_full > 0:
            row0 = np.arange(0, r_full, rows_per_item)
            it = np.zeros(row0.size, ITEM_DTYPE)
            it["proj"] = p
            it["row0"] = row0
            it["nrows"] = np.minimum(rows_per_item, r_full - row0)
            parts.append(it)
        if r_full < N:
            rows = np.arange(r_full, N)
            it = np.zeros(rows.size, ITEM_DTYPE)
            it["proj"] = p
            it["row0"] = rows
            it["nrows"] = 1
            it["flags"] = nat.PP_ITEM_TAIL
            parts.append(it)
    items = np.concatenate(parts) if parts else np.zeros(0, ITEM_DTYPE)
    if items.size:
        K = np.array([k for _, k in shapes], np.int64)[items["proj"]]
        lo = pos[:-1].astype(np.int64)[items["proj"]] + items["row0"].astype(np.int64) * K
        hi = lo + items["nrows"].astype(np.int64) * K
        items["plug_lo"] = np.searchsorted(plug_host, lo, side="left")
        items["plug_hi"] = np.searchsorted(plug_host, hi, side="left")
    return items


def item_bytes(items, shapes, M=1):
    """Bytes each item reads (codes, activations, plug entries); TAIL rows run on a scalar
    path and are weighted 4x."""
    klen = np.array([k for _, k in shapes], np.int64)[items["proj"]]
    b = 4 * items["nrows"].astype(np.int64) * klen + 2 * M * klen
    b += 12 * (items["plug_hi"] - items["plug_lo"])
    tail = (items["flags"] & nat.PP_ITEM_TAIL) != 0
    b[tail] = 16 * klen[tail]
    return b


def wave_bounds(item_bytes_, n_waves):
    """Item ranges per wavefront so that each gets ~1/n_waves of the bytes."""
    starts = np.concatenate([[0], np.cumsum(item_bytes_)[:-1]]) if item_bytes_.size else np.zeros(0, np.int64)
    total = int(item_bytes_.sum())
    targets = np.arange(n_waves + 1, dtype=np.float64) * total / max(n_waves, 1)
    bounds = np.searchsorted(starts, targets, side="left").astype(np.int64)
    bounds[0] = 0
    bounds[-1] = item_bytes_.size
    return np.maximum.accumulate(bounds)


class QuadStream:
    def __init__(self, pack: QuadPackDevice, shapes: Sequence[Tuple[int, int]], M: int = 1,
                 schedule: str = "bytes"):
        L = nat.lib()
        self.pack = pack
        self.shapes = [(int(n), int(k)) for n, k in shapes]
        self.M = int(M)
        self.device = pack.codes.device
        self.rows_per_item = int(L.pp_quad_stream_rows(self.M))
        nat.check(0 if self.rows_per_item > 0 else nat.PP_EINVAL, "pp_quad_stream_rows")
        pos = np.cumsum([0] + [n * k for n, k in self.shapes])
        self.pos0 = pos[:-1]
        total = int(pos[-1])
        longest = pack.n + max(pack.tail_lengths)
        if total > longest:
            raise ValueError(f"projections cover {total} positions, the stream holds {longest}")
        for n, k in self.shapes:
            if k % 4 or k >= 2 ** 31 or n >= 2 ** 31:
                raise ValueError(f"stream decode needs K % 4 == 0 (got N={n}, K={k})")
        items = plan_items(self.shapes, pack.n, pack.plug_host(), self.rows_per_item)
        is_tail = (items["flags"] & nat.PP_ITEM_TAIL) != 0
        self.tail_items_np = items[is_tail]
        items = items[~is_tail]
        self.items_np = items
        self.n_items = items.size
        self.n_tail = self.tail_items_np.size
        self.item_bytes = item_bytes(items, self.shapes, self.M)
        self.n_waves = int(L.pp_quad_stream_waves(self.M))
        if schedule not in ("interleave", "bytes"):
            raise ValueError("schedule must be 'interleave' or 'bytes'")
        self.schedule = schedule
        self.bounds_np = wave_bounds(self.item_bytes, self.n_waves)
        dev = self.device
        self.items = torch.from_numpy(items.view(np.uint8).copy()).to(dev)
        self.tail_items = torch.from_numpy(self.tail_items_np.view(np.uint8).copy()).to(dev)
        self.bounds = torch.from_numpy(self.bounds_np).to(dev)
        self.luts = header_luts(pack.r_max, device=dev)
        self._lut_ptrs = nat.ptr_array([t.data_ptr() for t in self.luts])
        self._scales = nat.float_array(pack.s)
        self._tail_ptrs = nat.ptr_array([t.data_ptr() if t.numel() else 0 for t in pack.tails])
        self._tail_len = (C.c_int64 * 4)(*pack.tail_lengths)
        self.projs = None

    # ---------------------------------------------------------------- buffers
    def make_buffers(self):
        """One activation buffer (M, K_p) and 4 output buffers (M, N_p) per projection."""
        xs, outs = [], []
        for N, K in self.shapes:
            xs.append(torch.empty((self.M, K), dtype=torch.float16, device=self.device))
            outs.append([torch.empty((self.M, N), dtype=torch.float16, device=self.device) for _ in range(4)])
        return xs, outs

    def bind(self, xs: List[torch.Tensor], outs: List[List[torch.Tensor]]):
        if len(xs) != len(self.shapes) or len(outs) != len(self.shapes):
            raise ValueError("one activation and 4 outputs per projection")
        tab = np.zeros(len(self.shapes), PROJ_DTYPE)
        base = self.pack.codes.data_ptr()
        for p, ((N, K), pos0) in enumerate(zip(self.shapes, self.pos0)):
            x, o = xs[p], outs[p]
            if x.shape != (self.M, K) or x.dtype != torch.float16 or x.stride(1) != 1 or x.data_ptr() % 8 \
                    or (self.M > 1 and x.stride(0) % 4):
                raise ValueError(f"projection {p}: activations must be fp16 ({self.M}, {K}), unit stride, 8-byte aligned")
            for t in o:
                if t.shape != (self.M, N) or t.dtype != torch.float16 or t.stride(1) != 1:
                    raise ValueError(f"projection {p}: outputs must be fp16 ({self.M}, {N}), unit stride")
            if o[0].stride(0) != o[1].stride(0) or o[0].stride(0) != o[2].stride(0) or o[0].stride(0) != o[3].stride(0):
                raise ValueError(f"projection {p}: the 4 outputs must share a row stride")
            tab[p]["codes"] = base + 4 * int(pos0)
            tab[p]["ldc"] = K
            tab[p]["pos0"] = int(pos0)
            tab[p]["x"] = x.data_ptr()
            tab[p]["x_sm"] = x.stride(0)
            tab[p]["out"] = [t.data_ptr() for t in o]
            tab[p]["o_sm"] = o[0].stride(0)
            tab[p]["N"] = N
            tab[p]["K"] = K
        self.projs = torch.from_numpy(tab.view(np.uint8).copy()).to(self.device)
        self._bound = (xs, outs)          # keep the buffers alive while bound

    def __call__(self):
        if self.projs is None:
            raise RuntimeError("QuadStream.bind() must be called before launching")
        pk = self.pack
        stream = torch.cuda.current_stream(self.device).cuda_stream
        rc = nat.lib().pp_quad_stream(self.projs.data_ptr(), len(self.shapes),
                                      self.items.data_ptr() if self.n_items else None, self.n_items,
                                      self.tail_items.data_ptr() if self.n_tail else None, self.n_tail,
                                      self.bounds.data_ptr() if self.schedule == "bytes" else None, self.n_waves,
                                      self._lut_ptrs, self._scales,
                                      pk.plug_idx.data_ptr() if pk.plug_idx.numel() else None,
                                      pk.plug_vals.data_ptr() if pk.plug_vals.numel() else None,
                                      pk.n, self._tail_ptrs, self._tail_len, self.M, stream)
        nat.check(rc, "pp_quad_stream")

    # ---------------------------------------------------------------- accounting
    def algorithmic_bytes(self) -> int:
        """4*N*K codes + 12 B per plug entry + 2*M*K x + 8*M*N outputs + 2 B per tail weight read."""
        plug = self.pack.plug_host()
        total = 0
        for (N, K), pos0 in zip(self.shapes, self.pos0):
            lo, hi = int(pos0), int(pos0) + N * K
            in_codes = max(0, min(hi, self.pack.n) - lo)
            P = int(np.searchsorted(plug, hi) - np.searchsorted(plug, lo))
            tail_w = sum(max(0, min(hi, self.pack.n + t) - max(lo, self.pack.n)) for t in self.pack.tail_lengths)
            total += 4 * in_codes + 12 * P + 2 * self.M * K + 8 * self.M * N + 2 * tail_w
        return total
