"""Whole-stream decode step: every projection of a ``.quadpack`` stream in one launch.

A stream is the reference's flat Linear order (polar_main.py:33-43): projection p
is an (N_p, K_p) row-major block at stream position pos_p = sum of the previous
N*K.  :class:`QuadStream` plans the launch once:

* rows fully inside the code stream are cut into tasks of ``rows_per_task`` rows
  (the kernel's row group); the tasks, in stream order, are dealt to the
  wavefronts in contiguous runs of equal bytes;
* each wavefront's run is split at projection boundaries into segments
  (``pp_quad_seg``: projection, row range, first plug entry at or after the
  segment start, found with searchsorted as quaternion_packer.py:188-189 does per
  chunk); inside a segment the kernel finds each task's plug entries itself;
* rows that reach the FP16 tails (positions >= n) become one-row TAIL items with
  their plug range, decoded by a second small kernel.

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
SEG_DTYPE = np.dtype([("proj", "<i4"), ("row0", "<i4"), ("row1", "<i4"), ("task0", "<i4"), ("plug_lo", "<i8"),
                      ("k0", "<i4"), ("k1", "<i4"), ("parts", "<i4"), ("reserved", "<i4"), ("acc_off", "<i8")])
PROJ_DTYPE = np.dtype([("codes", "<u8"), ("ldc", "<i8"), ("pos0", "<i8"), ("x", "<u8"), ("x_sm", "<i8"),
                       ("out", "<u8", (4,)), ("o_sm", "<i8"), ("N", "<i4"), ("K", "<i4")])
DUAL_PROJ_DTYPE = np.dtype([("codes", "<u8"), ("ldc", "<i8"), ("pos0", "<i8"), ("x", "<u8"), ("x_sm", "<i8"),
                            ("out", "<u8", (2,)), ("o_sm", "<i8"), ("N", "<i4"), ("K", "<i4")])


def stream_positions(shapes, positions=None):
    """Stream position of each projection: ``positions`` when given (ascending, the
    projections not overlapping), else back to back from 0."""
    sizes = np.array([int(a) * int(b) for a, b in shapes], np.int64)
    if positions is None:
        return np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64) if sizes.size else np.zeros(0, np.int64)
    pos = np.asarray(positions, np.int64).reshape(-1)
    if pos.size != sizes.size or (pos.size and (pos[0] < 0 or np.any(pos[1:] < pos[:-1] + sizes[:-1]))):
        raise ValueError("projection positions must be >= 0, ascending and not overlapping")
    return pos


def full_rows(shapes, n, positions=None):
    """Stream position of each projection and how many of its rows lie fully below ``n``."""
    pos = stream_positions(shapes, positions)
    N = np.array([int(a) for a, _ in shapes], np.int64)
    K = np.array([int(b) for _, b in shapes], np.int64)
    r_full = np.clip((int(n) - pos) // np.maximum(K, 1), 0, N)
    return pos, N, K, r_full


def plan_tasks(shapes, n, rows_per_task, positions=None):
    """Tasks (proj, row0, nrows) over the full rows of every projection, in stream order."""
    pos0, N, K, r_full = full_rows(shapes, n, positions)
    counts = (r_full + rows_per_task - 1) // rows_per_task
    proj = np.repeat(np.arange(len(shapes), dtype=np.int64), counts)
    first = np.concatenate([[0], np.cumsum(counts)[:-1]]) if counts.size else np.zeros(0, np.int64)
    local = np.arange(proj.size, dtype=np.int64) - np.repeat(first, counts)
    row0 = local * rows_per_task
    nrows = np.minimum(rows_per_task, r_full[proj] - row0) if proj.size else np.zeros(0, np.int64)
    return proj, row0, nrows


def task_bytes(proj, nrows, shapes, M=1, code_bytes=4):
    """Bytes each task reads: its codes and its activation vector(s)."""
    K = np.array([int(b) for _, b in shapes], np.int64)[proj]
    return code_bytes * nrows * K + 2 * M * K


def wave_bounds(bytes_, n_waves, weights=None):
    """Contiguous ranges of tasks per wavefront so that each gets ~1/n_waves of the bytes, or
    a share proportional to ``weights`` (n_waves values) when given."""
    starts = np.concatenate([[0], np.cumsum(bytes_)[:-1]]) if bytes_.size else np.zeros(0, np.int64)
    total = int(bytes_.sum())
    if weights is None:
        targets = np.arange(n_waves + 1, dtype=np.float64) * total / max(n_waves, 1)
    else:
        w = np.asarray(weights, np.float64)
        targets = np.concatenate([[0.0], np.cumsum(w)]) * (total / max(w.sum(), 1e-300))
    bounds = np.searchsorted(starts, targets, side="left").astype(np.int64)
    bounds[0] = 0
    bounds[-1] = bytes_.size
    return np.maximum.accumulate(bounds)


# Waves w and w + 4 of a workgroup of 8 share a SIMD and the older one wins instruction
# issue: measured on the quad 3B stream, waves 4-7 of every workgroup take 7.4% longer for
# the same bytes, so equal shares leave the first four idle at the end (8.6-9.9% of the
# wave-time idle; 5.2% with these weights, and the launch 2.7% shorter).
SLOT_FACTOR = 1.074
DUAL_SLOT_FACTOR = 1.10


def slot_weights(n_waves, waves_per_group, factor=SLOT_FACTOR):
    """Planner weights of the launch's wavefronts (numbered workgroup by workgroup): the
    younger half of each workgroup's waves gets 1/factor of the older half's share."""
    w = np.ones(int(n_waves))
    if waves_per_group >= 2:
        w[(np.arange(int(n_waves)) % waves_per_group) >= waves_per_group // 2] /= factor
    return w


def _waves_per_group(n_waves, device):
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    return max(1, int(n_waves) // max(1, cus))


def split_factors(shapes, n, rows_per_task, n_waves, block=512, positions=None):
    """(slices, column blocks per slice, at most) per projection, slices being whole blocks
    of ``block`` columns (the kernel's chunk width), from r = wavefronts / tasks:
      * r < 1.5: 1 slice (the tasks fill the launch; measured on 11008x2048 at 1 token,
        1,376 tasks: 26.7 us whole, 31 us in 2 or 4 slices);
      * 1.5 <= r < 4: 2 slices for projections of at least 8 blocks (2048x11008 at 2
        tokens: 35.6 us against 37.2 us whole), else 1;
      * r >= 4: ceil(r / 2) slices, at most one per block (2048x11008 at 1 token: 31.3 us
        in 4 slices, 32.6 us in 8, 65 us whole; the dual 2048x2048 Linear: 11.0 us in 4,
        14.0 us whole): about one item per two wavefronts, since every item adds a
        reduction, partial-sum atomics and a pipeline restart.
    :func:`slice_bounds` deals the blocks to the slices."""
    proj, _, _ = plan_tasks(shapes, n, rows_per_task, positions)
    K = np.array([int(b) for _, b in shapes], np.int64)
    blocks = np.maximum(1, (K + block - 1) // block)
    ones = np.ones(len(shapes), np.int64)
    if proj.size == 0:
        return ones, blocks
    r = n_waves / proj.size
    if r >= 4:
        want = np.full(len(shapes), -(-n_waves // (2 * proj.size)), np.int64)
    elif r >= 1.5:
        want = np.where(blocks >= 8, 2, 1)
    else:
        return ones, blocks
    parts = np.maximum(1, np.minimum(want, blocks))
    per = -(-blocks // parts)                              # blocks per slice, at most
    return parts, per


# Planner cost of each item of a split projection, in bytes, on top of the bytes it reads:
# its reduction, partial-sum atomics and pipeline restart (measured on 2048x11008 at 1-2
# tokens: 64 KiB balances the waves best, 2-9 % faster than 0).
SPLIT_ITEM_COST = 65536


def slice_bounds(K, parts, block):
    """Column ranges of the ``parts`` slices of a K-column projection: the ceil(K / block)
    blocks dealt as evenly as possible (slice s takes blocks [s*B // parts, (s+1)*B //
    parts)), so that no slice is left with a sliver of the columns (one 256-column slice
    among 1536-column ones made the planner give its waves six tasks each: 2.2x the
    time of the others for the same bytes, from the per-task reduction and restart)."""
    B = max(1, -(-int(K) // block))
    return [((sl * B // parts) * block, min(int(K), ((sl + 1) * B // parts) * block)) for sl in range(int(parts))]


def plan_segments(shapes, n, plug_host, n_waves, rows_per_task, M=1, code_bytes=4, split=False, block=512,
                  positions=None, wave_weights=None, task_cost=0):
    """Per-wave segments (SEG_DTYPE), seg_bounds (n_waves + 1) and the workspace bytes
    for the rows below ``n``.

    Tasks (:func:`plan_tasks`) are the units; with ``split`` and few tasks per wavefront
    (a single Linear with few rows) every task of a projection is cut into column slices of whole ``block``-column
    chunks (:func:`split_factors`), the
    slices of a projection ordered slice by slice.  The items are dealt to the wavefronts
    in contiguous runs of equal cost (bytes read, plus ``task_cost`` bytes for each item's
    reduction and stores, plus SPLIT_ITEM_COST for an item of a split projection), or of
    cost proportional to ``wave_weights``, and each
    wavefront's run is cut into segments of one projection and one slice.  The workspace of split launches holds one uint32
    counter per task, then 4*M*N float32 accumulators per split projection.
    """
    proj, row0, nrows = plan_tasks(shapes, n, rows_per_task, positions)
    if proj.size == 0:
        return np.zeros(0, SEG_DTYPE), np.zeros(n_waves + 1, np.int64), 0
    pos0, N, K, _ = full_rows(shapes, n, positions)
    tid = np.arange(proj.size, dtype=np.int64)
    parts = np.ones(len(shapes), np.int64)
    per = np.zeros(len(shapes), np.int64)
    if split:
        parts, per = split_factors(shapes, n, rows_per_task, n_waves, block, positions)
    if np.all(parts == 1):
        it_task, it_k0, it_k1 = tid, np.zeros(proj.size, np.int64), K[proj]
    else:
        chunks = []
        for p in range(len(shapes)):
            ts = tid[proj == p]
            if ts.size == 0:
                continue
            for k0, k1 in slice_bounds(K[p], parts[p], block):
                chunks.append((ts, np.full(ts.size, k0, np.int64), np.full(ts.size, k1, np.int64)))
        it_task = np.concatenate([c[0] for c in chunks])
        it_k0 = np.concatenate([c[1] for c in chunks])
        it_k1 = np.concatenate([c[2] for c in chunks])
    it_proj = proj[it_task]
    width = it_k1 - it_k0
    ib = code_bytes * nrows[it_task] * width + 2 * M * width + int(task_cost) \
        + np.where(parts[it_proj] > 1, SPLIT_ITEM_COST, 0)
    tb = wave_bounds(ib, n_waves, wave_weights)
    wave = np.searchsorted(tb, np.arange(it_task.size), side="right") - 1
    brk = np.ones(it_task.size, bool)
    brk[1:] = (wave[1:] != wave[:-1]) | (it_proj[1:] != it_proj[:-1]) | (it_k0[1:] != it_k0[:-1])
    first = np.flatnonzero(brk)
    last = np.concatenate([first[1:], [it_task.size]]) - 1
    segs = np.zeros(first.size, SEG_DTYPE)
    fp = it_proj[first]
    segs["proj"] = fp
    segs["row0"] = row0[it_task[first]]
    segs["row1"] = row0[it_task[last]] + nrows[it_task[last]]
    segs["task0"] = it_task[first]
    segs["plug_lo"] = np.searchsorted(plug_host, pos0[fp] + segs["row0"] * K[fp], side="left")
    segs["k0"] = it_k0[first]
    segs["k1"] = it_k1[first]
    segs["parts"] = parts[fp]
    ws_bytes = 0
    if np.any(parts > 1):
        base = (4 * proj.size + 255) // 256 * 64              # floats: after the counters, 256-byte aligned
        acc_off = np.zeros(len(shapes), np.int64)
        off = base
        for p in np.flatnonzero(parts > 1):
            acc_off[p] = off
            off += 4 * M * int(N[p])
        segs["acc_off"] = np.where(parts[fp] > 1, acc_off[fp], 0)
        ws_bytes = 4 * off
    seg_wave = wave[first]
    bounds = np.searchsorted(seg_wave, np.arange(n_waves + 1), side="left").astype(np.int64)
    return segs, bounds, ws_bytes


def plan_task_plug(shapes, n, plug_host, rows_per_task, positions=None):
    """Per task (in the order of :func:`plan_tasks`): the first plug entry at or after its
    first position and the first entry past its last position, as an (n_tasks, 2) int64
    table, and the number of chunks (512-pair steps) of each task."""
    proj, row0, nrows = plan_tasks(shapes, n, rows_per_task, positions)
    pos0, _, K, _ = full_rows(shapes, n, positions)
    start = pos0[proj] + row0 * K[proj]
    tab = np.empty((proj.size, 2), np.int64)
    tab[:, 0] = np.searchsorted(plug_host, start, side="left")
    tab[:, 1] = np.searchsorted(plug_host, start + nrows * K[proj], side="left")
    return tab, (K[proj] + 511) // 512


def plan_tail_items(shapes, n, plug_host, tail_lengths=None, fp16_rows=0, positions=None):
    """Items for the rows that reach position ``n``.

    By default one TAIL item per row, with its plug range.  With ``fp16_rows`` > 0 and
    the models' ``tail_lengths``, rows that start at or past ``n`` and, for every model,
    lie wholly inside or wholly past its tail become FP16 items of up to ``fp16_rows``
    consecutive rows with the same status; the rest stay one-row TAIL items.
    """
    pos0, N, K, r_full = full_rows(shapes, n, positions)
    parts = []
    for p in np.flatnonzero(r_full < N):
        rows = np.arange(r_full[p], N[p], dtype=np.int64)
        lo = pos0[p] + rows * K[p]
        hi = lo + K[p]
        key = np.full(rows.size, -1, np.int64)              # -1: element by element
        if fp16_rows > 0 and tail_lengths is not None:
            clean = lo >= n
            status = np.zeros(rows.size, np.int64)
            for m, L in enumerate(tail_lengths):
                inside = hi <= n + L
                clean &= inside | (lo >= n + L)
                status |= inside.astype(np.int64) << m
            key = np.where(clean, status, -1)
        start = np.ones(rows.size, bool)
        start[1:] = (key[1:] != key[:-1]) | (key[1:] < 0)
        run_id = np.cumsum(start) - 1
        run_first = np.flatnonzero(start)
        in_run = np.arange(rows.size) - run_first[run_id]
        if fp16_rows > 0:
            start |= (in_run % fp16_rows) == 0
        first = np.flatnonzero(start)
        count = np.diff(np.concatenate([first, [rows.size]]))
        it = np.zeros(first.size, ITEM_DTYPE)
        it["proj"] = p
        it["row0"] = rows[first]
        it["nrows"] = count
        fp16 = key[first] >= 0
        it["flags"] = np.where(fp16, nat.PP_ITEM_FP16, nat.PP_ITEM_TAIL)
        plo = np.searchsorted(plug_host, lo[first], side="left")
        phi = np.searchsorted(plug_host, hi[first], side="left")
        it["plug_lo"] = np.where(fp16, 0, plo)
        it["plug_hi"] = np.where(fp16, 0, phi)
        parts.append(it)
    return np.concatenate(parts) if parts else np.zeros(0, ITEM_DTYPE)


def layer_map_projections(layer_info, model=None):
    """The projections of the reference's layer map (collect_weights, polar_main.py:33-46:
    dicts with ``name``, ``shape`` = [N, K] and ``numel``, in stream order) as
    ``(names, shapes, positions)``.  Each entry advances the stream position by its
    ``numel``; entries that are not an (N, K) Linear -- a shape that is not 2-D or does not
    hold ``numel`` weights, or, with ``model`` given, a name that is not an ``nn.Linear``
    of that size there -- are skipped, as replace_model_weights does
    (polar_packer.py:297-305)."""
    names, shapes, positions = [], [], []
    pos = 0
    for info in layer_info:
        numel = int(info["numel"])
        shape = [int(v) for v in info["shape"]]
        ok = len(shape) == 2 and shape[0] * shape[1] == numel and numel > 0
        if ok and model is not None:
            from .linear import _module_at
            _, module = _module_at(model, info["name"])
            ok = isinstance(module, torch.nn.Linear) and module.weight.numel() == numel
        if ok:
            names.append(info["name"])
            shapes.append((shape[0], shape[1]))
            positions.append(pos)
        pos += numel
    return names, shapes, positions


class QuadStream:
    """One-launch decode of many projections of a quad stream (``pp_quad_stream``).

    ``split`` lets a launch with fewer row tasks than half its wavefronts (a single
    Linear with few rows) cut its tasks into column slices whose sums meet in a
    workspace owned by this object (so two launches of one QuadStream must not overlap).
    ``wave_weights``: per-wave shares of the work ("slots": :func:`slot_weights`; None:
    equal bytes); ``task_cost``: bytes charged per task for its reduction and stores.
    ``one_linear``: a single projection wholly inside the codes runs the row kernel's
    one-Linear launch (``pp_quad_rows``: the waves find their rows and column slice from the
    launch shape, with no segment table to read), except at one token with column slices,
    where the segment plan measured faster; False keeps the segment plan.
    """

    def __init__(self, pack: QuadPackDevice, shapes: Sequence[Tuple[int, int]], M: int = 1, split: bool = True,
                 positions=None, wave_weights="slots", task_cost=0, one_linear: bool = True):
        L = nat.lib()
        self.pack = pack
        self.shapes = [(int(n), int(k)) for n, k in shapes]
        self.M = int(M)
        self.device = pack.codes.device
        self.rows_per_item = int(L.pp_quad_stream_rows(self.M))
        nat.check(0 if self.rows_per_item > 0 else nat.PP_EINVAL, "pp_quad_stream_rows")
        self.pos0 = stream_positions(self.shapes, positions)
        self.positions = self.pos0 if positions is not None else None
        total = int(self.pos0[-1]) + self.shapes[-1][0] * self.shapes[-1][1] if self.shapes else 0
        longest = pack.n + max(pack.tail_lengths)
        if total > longest:
            raise ValueError(f"projections cover {total} positions, the stream holds {longest}")
        for n, k in self.shapes:
            if k % 4 or k >= 2 ** 31 or n >= 2 ** 31:
                raise ValueError(f"stream decode needs K % 4 == 0 (got N={n}, K={k})")
        plug = pack.plug_host()
        self.n_waves = int(L.pp_quad_stream_waves(self.M))
        # one Linear wholly inside the codes: the row kernel's one-Linear launch (pp_quad_rows),
        # which needs no segment table (its waves find their rows from the launch shape).  At one
        # token with column slices the segment plan is kept: measured interleaved, down_proj
        # 2048x11008 at one token 30.3 us on the segment plan against 34-35 us on the one-Linear
        # launch, whatever its deal; gate_proj (whole rows) 22.9 against 25.3 us, and down at 2 / 4
        # tokens 28.3 / 31.7 against 34.3 / 39.9 us, go to the one-Linear launch
        sliced_one_token = self.M == 1 and self.shapes and \
            int(L.pp_quad_rows_workspace_size(self.M, *self.shapes[0])) > 0
        self.direct = one_linear and len(self.shapes) == 1 and total <= pack.n and split and not sliced_one_token
        if self.direct:
            self._plan_direct(plug)
            return
        if isinstance(wave_weights, str) and wave_weights == "slots":
            wave_weights = slot_weights(self.n_waves, _waves_per_group(self.n_waves, self.device))
        self.segs_np, self.bounds_np, ws_bytes = plan_segments(
            self.shapes, pack.n, plug, self.n_waves, self.rows_per_item, self.M, split=split,
            block=int(L.pp_quad_stream_chunk(self.M)), positions=self.positions, wave_weights=wave_weights,
            task_cost=task_cost)
        self.tail_items_np = plan_tail_items(self.shapes, pack.n, plug, positions=self.positions)
        self.n_segs = self.segs_np.size
        self.n_tail = self.tail_items_np.size
        self.split = bool(np.any(self.segs_np["parts"] > 1))
        dev = self.device
        # split launches: counters + accumulators, zero once here, left zero by every launch
        self.workspace = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None
        self.segs = torch.from_numpy(self.segs_np.view(np.uint8).copy()).to(dev)
        self.tail_items = torch.from_numpy(self.tail_items_np.view(np.uint8).copy()).to(dev)
        self.bounds = torch.from_numpy(self.bounds_np).to(dev)
        self.luts = header_luts(pack.r_max, device=dev)
        self._lut_ptrs = nat.ptr_array([t.data_ptr() for t in self.luts])
        self._scales = nat.float_array(pack.s)
        self._tail_ptrs = nat.ptr_array([t.data_ptr() if t.numel() else 0 for t in pack.tails])
        self._tail_len = (C.c_int64 * 4)(*pack.tail_lengths)
        # each plug entry's code word, gathered once here (pp_quad_plug_codes)
        P = int(pack.plug_idx.numel())
        self.plug_code = torch.empty(max(P, 1), dtype=torch.int32, device=dev)
        if P:
            rc = L.pp_quad_plug_codes(pack.codes.data_ptr(), pack.n, pack.plug_idx.data_ptr(), P,
                                      self.plug_code.data_ptr(), nat.raw_stream(dev))
            nat.check(rc, "pp_quad_plug_codes")
        self.projs = None

    def _plan_direct(self, plug):
        """The plan of a one-Linear launch: the Linear's slice of the plug table, each
        wavefront's first entry in it (pp_quad_rows_plan), the entries' code words
        (pp_quad_plug_codes) and the zeroed column-slice workspace."""
        L = nat.lib()
        pk, dev = self.pack, self.device
        (N, K), pos0 = self.shapes[0], int(self.pos0[0])
        self.plug_lo = int(np.searchsorted(plug, pos0, side="left"))
        self.plug_hi = int(np.searchsorted(plug, pos0 + N * K, side="left"))
        n = self.plug_hi - self.plug_lo
        stream = nat.raw_stream(dev)
        self.wave_plug = torch.zeros(int(L.pp_quad_rows_plan_size(self.M)), dtype=torch.int64, device=dev)
        self.plug_code = torch.zeros(max(n, 1), dtype=torch.int32, device=dev)
        if n:
            idx = pk.plug_idx.data_ptr() + 4 * self.plug_lo
            nat.check(L.pp_quad_rows_plan(idx, n, pos0, K, self.M, N, K, self.wave_plug.data_ptr(), stream),
                      "pp_quad_rows_plan")
            nat.check(L.pp_quad_plug_codes(pk.codes.data_ptr(), pk.n, idx, n, self.plug_code.data_ptr(), stream),
                      "pp_quad_plug_codes")
        ws_bytes = int(L.pp_quad_rows_workspace_size(self.M, N, K))
        self.workspace = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None
        self._ws_bytes = ws_bytes
        self.split = int(L.pp_quad_rows_parts(self.M, N, K)) > 1
        self.n_segs = self.n_tail = 0
        self.luts = header_luts(pk.r_max, device=dev)
        self._lut_ptrs = nat.ptr_array([t.data_ptr() for t in self.luts])
        self._scales = nat.float_array(pk.s)
        self.projs = None

    @classmethod
    def from_layer_map(cls, pack: QuadPackDevice, layer_info, M: int = 1, model=None, split: bool = True):
        """The stream of every Linear of a reference layer map (:func:`layer_map_projections`);
        ``names`` lists them in projection order."""
        names, shapes, positions = layer_map_projections(layer_info, model)
        st = cls(pack, shapes, M=M, split=split, positions=positions)
        st.names = names
        return st

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
        if self.direct:
            self._out_ptrs = nat.ptr_array([t.data_ptr() for t in outs[0]])

    def _call_direct(self):
        pk = self.pack
        (N, K), pos0 = self.shapes[0], int(self.pos0[0])
        xs, outs = self._bound
        n = self.plug_hi - self.plug_lo
        rc = nat.lib().pp_quad_rows(xs[0].data_ptr(), xs[0].stride(0), pk.codes.data_ptr() + 4 * pos0, K,
                                    self._lut_ptrs, nat.PP_F32, self._scales,
                                    pk.plug_idx.data_ptr() + 4 * self.plug_lo if n else None,
                                    pk.plug_vals.data_ptr() + 8 * self.plug_lo if n else None,
                                    self.plug_code.data_ptr() if n else None, n,
                                    self.wave_plug.data_ptr() if n else None, pos0, self._out_ptrs,
                                    outs[0][0].stride(0), 1, self.M, N, K,
                                    self.workspace.data_ptr() if self.workspace is not None else None,
                                    self._ws_bytes, nat.raw_stream(self.device))
        nat.check(rc, "pp_quad_rows")

    def __call__(self):
        if self.projs is None:
            raise RuntimeError("QuadStream.bind() must be called before launching")
        if self.direct:
            return self._call_direct()
        pk = self.pack
        stream = nat.raw_stream(self.device)
        rc = nat.lib().pp_quad_stream(self.projs.data_ptr(), len(self.shapes),
                                      self.segs.data_ptr() if self.n_segs else None, self.n_segs,
                                      self.bounds.data_ptr(), self.n_waves,
                                      self.workspace.data_ptr() if self.workspace is not None else None,
                                      self.tail_items.data_ptr() if self.n_tail else None, self.n_tail,
                                      self._lut_ptrs, self._scales,
                                      pk.plug_idx.data_ptr() if pk.plug_idx.numel() else None,
                                      pk.plug_vals.data_ptr() if pk.plug_vals.numel() else None,
                                      self.plug_code.data_ptr(),
                                      int(pk.plug_idx.numel()), pk.n, self._tail_ptrs, self._tail_len, self.M, stream)
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


class DualStream:
    """One-launch decode of every projection of a dual stream (``pp_dual_stream``).

    Same planning as :class:`QuadStream`, plus each task's plug range (the kernel
    spreads a task's plug entries over its steps, 64 or 128 per step: ``plug_windows``,
    chosen from the table's density unless given); positions past ``pack.n_codes`` come
    from the per-model fp16 tails.  Projection rows and positions must be multiples of
    8 pairs (a lane reads 8 pairs that share one group scale).  ``split`` as for
    :class:`QuadStream` (column slices for launches with few row tasks, summed in a
    workspace owned by this object: two launches of one DualStream must not overlap).
    ``scale_table`` (default: where it applies) gives the decode the group scales regrouped
    per task of R = ``rows_per_item`` rows (``pp_dual_scale_table``: one load per step for
    all R rows); it applies when chunk_size % group_size == 0 and every projection has
    K % group_size == 0, N % R == 0 and a position that is a multiple of R * group_size.
    ``one_linear``: a single projection wholly inside the codes runs the stream kernel's
    one-Linear launch (``pp_dual_rows``: no segment table; its column slices meet in a
    workspace sized by ``pp_dual_rows_workspace_size``); False keeps the segment plan.
    """

    def __init__(self, pack, shapes: Sequence[Tuple[int, int]], M: int = 1, plug_windows=None, split: bool = True,
                 positions=None, wave_weights="slots", task_cost=0, scale_table=None, one_linear: bool = True):
        L = nat.lib()
        self.pack = pack
        self.shapes = [(int(n), int(k)) for n, k in shapes]
        self.M = int(M)
        self.device = pack.codes.device
        self.rows_per_item = int(L.pp_dual_stream_rows(self.M))
        nat.check(0 if self.rows_per_item > 0 else nat.PP_EINVAL, "pp_dual_stream_rows")
        self.pos0 = stream_positions(self.shapes, positions)
        self.positions = self.pos0 if positions is not None else None
        total = int(self.pos0[-1]) + self.shapes[-1][0] * self.shapes[-1][1] if self.shapes else 0
        longest = pack.n_codes + max(pack.tail_lengths)
        if total > longest:
            raise ValueError(f"projections cover {total} positions, the stream holds {longest}")
        for n, k in self.shapes:
            if k % 8 or k >= 2 ** 19 or n >= 2 ** 31:
                raise ValueError(f"dual stream decode needs K % 8 == 0 and K < 2^19 (got N={n}, K={k})")
        if pack.group_size < 8 or pack.group_size & (pack.group_size - 1) or pack.chunk_size % 8:
            raise ValueError("dual stream decode needs a power-of-two group_size >= 8 and chunk_size % 8 == 0")
        plug = pack.plug_host()
        self.n_waves = int(L.pp_dual_stream_waves(self.M))
        if isinstance(wave_weights, str) and wave_weights == "slots":
            wave_weights = slot_weights(self.n_waves, _waves_per_group(self.n_waves, self.device), DUAL_SLOT_FACTOR)
        self.segs_np, self.bounds_np, ws_bytes = plan_segments(
            self.shapes, pack.n_codes, plug, self.n_waves, self.rows_per_item, self.M, code_bytes=2, split=split,
            block=int(L.pp_dual_stream_chunk(self.M)), positions=self.positions, wave_weights=wave_weights,
            task_cost=task_cost)
        self.split = bool(np.any(self.segs_np["parts"] > 1))
        self.direct = one_linear and len(self.shapes) == 1 and total <= pack.n_codes and split
        if self.direct:
            # K parts meet in LDS when a workgroup holds a task's parts, else in the workspace
            ws_bytes = int(L.pp_dual_rows_workspace_size(self.M, *self.shapes[0]))
            self.split = int(L.pp_dual_rows_parts(self.M, *self.shapes[0])) > 1
        # split launches: counters + accumulators, zero once here, left zero by every launch
        self.workspace = torch.zeros(ws_bytes, dtype=torch.uint8, device=self.device) if ws_bytes else None
        self._ws_bytes = ws_bytes
        tails = list(pack.tails) + [None] * (2 - len(pack.tails))
        aligned = pack.n_codes % 8 == 0 and all(t is None or t.numel() == 0 or t.data_ptr() % 16 == 0
                                                for t in tails)
        self.tail_items_np = plan_tail_items(self.shapes, pack.n_codes, plug, pack.tail_lengths,
                                             fp16_rows=8 if aligned else 0, positions=self.positions)
        self.n_segs = self.segs_np.size
        self.n_tail = self.tail_items_np.size
        self.task_plug_np, nck = plan_task_plug(self.shapes, pack.n_codes, plug, self.rows_per_item, self.positions)
        self.n_tasks = self.task_plug_np.shape[0]
        if plug_windows is None:
            # one 64-entry window per step, two when more than 2% of the tasks would
            # otherwise have entries left after their last step
            left = (self.task_plug_np[:, 1] - self.task_plug_np[:, 0]) > 64 * nck
            plug_windows = 2 if left.size and left.mean() > 0.02 else 1
        if plug_windows not in (1, 2):
            raise ValueError("plug_windows must be 1 or 2")
        self.plug_windows = int(plug_windows)
        dev = self.device
        self.task_plug = torch.from_numpy(np.ascontiguousarray(self.task_plug_np).reshape(-1)).to(dev)
        self.segs = torch.from_numpy(self.segs_np.view(np.uint8).copy()).to(dev)
        self.tail_items = torch.from_numpy(self.tail_items_np.view(np.uint8).copy()).to(dev)
        self.bounds = torch.from_numpy(self.bounds_np).to(dev)
        from .polar_kernels import header_luts as dual_header_luts
        self.luts = dual_header_luts(pack.amp_bits, pack.phase_bits, pack.mu, device=dev)
        tails = list(pack.tails) + [None] * (2 - len(pack.tails))
        self._tail_ptrs = nat.ptr_array([t.data_ptr() if t is not None and t.numel() else 0 for t in tails])
        self._tail_len = (C.c_int64 * 2)(*pack.tail_lengths)
        self.code_layout = nat.PP_DUAL_U16_BE if pack.layout == "u16be" else nat.PP_DUAL_I16_OFFSET
        # each plug entry's 8-byte record (column, row in its task and phase of its pair; its
        # amplitude correction), built once here (pp_dual_plug_table)
        P = int(pack.plug_idx.numel())
        self.plug_ent = torch.zeros(max(2 * P, 1), dtype=torch.int32, device=dev)
        if P:
            self._proj_pos0 = torch.tensor(list(self.pos0) + [total], dtype=torch.int64, device=dev)
            self._proj_k = torch.tensor([k for _, k in self.shapes], dtype=torch.int32, device=dev)
            rc = L.pp_dual_plug_table(pack.codes.data_ptr(), pack.n_codes, self.code_layout, pack.scales.data_ptr(),
                                      int(pack.scales.numel()), pack.group_size, pack.chunk_size,
                                      self.luts[0].data_ptr(), pack.plug_idx.data_ptr(), pack.plug_val.data_ptr(), P,
                                      self._proj_pos0.data_ptr(), self._proj_k.data_ptr(), len(self.shapes),
                                      self.rows_per_item, self.plug_ent.data_ptr(),
                                      nat.raw_stream(dev))
            nat.check(rc, "pp_dual_plug_table")
        # one-Linear launch: each task's records in a block of the same size (the largest
        # task's count; pp_dual_task_entries), so that a wave loads its records without first
        # loading their range.  Kept while the blocks hold at most 4x the records (or 64K);
        # a projection without entries passes none (task_cap 1, every window empty).
        self.task_cap, self.task_ent = 0, None
        if self.direct:
            cnt = self.task_plug_np[:, 1] - self.task_plug_np[:, 0]
            cap = int(cnt.max()) if cnt.size else 0
            if cap == 0:
                self.task_cap = 1
            elif self.n_tasks * cap <= max(4 * P, 1 << 16):
                self.task_ent = torch.empty(2 * self.n_tasks * cap, dtype=torch.int32, device=dev)
                rc = L.pp_dual_task_entries(self.plug_ent.data_ptr(), P, self.task_plug.data_ptr(), self.n_tasks, cap,
                                            self.task_ent.data_ptr(), nat.raw_stream(dev))
                nat.check(rc, "pp_dual_task_entries")
                self.task_cap = cap
        gs, R = pack.group_size, self.rows_per_item
        fits = (pack.chunk_size % gs == 0 and len(self.shapes) > 0
                and all(k % gs == 0 and n % R == 0 and int(p) % (R * gs) == 0
                        for (n, k), p in zip(self.shapes, self.pos0)))
        if scale_table and not fits:
            raise ValueError(f"the scale table needs chunk_size % group_size == 0 and, for every projection, "
                             f"K % group_size == 0, N % {R} == 0 and a position that is a multiple of "
                             f"{R} * group_size")
        self.scale_tab = None
        if fits and scale_table is not False:
            n_tab = max(int(pack.scales.numel()), -(-total // gs))
            self.scale_tab = torch.empty(n_tab, dtype=torch.float16, device=dev)
            self._tab_pos0 = torch.tensor(self.pos0, dtype=torch.int64, device=dev)
            self._tab_n = torch.tensor([n for n, _ in self.shapes], dtype=torch.int32, device=dev)
            self._tab_k = torch.tensor([k for _, k in self.shapes], dtype=torch.int32, device=dev)
            rc = L.pp_dual_scale_table(pack.scales.data_ptr(), int(pack.scales.numel()), gs,
                                       self._tab_pos0.data_ptr(), self._tab_n.data_ptr(), self._tab_k.data_ptr(),
                                       len(self.shapes), R, self.scale_tab.data_ptr(), n_tab,
                                       nat.raw_stream(dev))
            nat.check(rc, "pp_dual_scale_table")
        self.projs = None

    @classmethod
    def from_layer_map(cls, pack, layer_info, M: int = 1, model=None, split: bool = True, plug_windows=None):
        """The stream of every Linear of a reference layer map (:func:`layer_map_projections`);
        ``names`` lists them in projection order."""
        names, shapes, positions = layer_map_projections(layer_info, model)
        st = cls(pack, shapes, M=M, split=split, positions=positions, plug_windows=plug_windows)
        st.names = names
        return st

    def make_buffers(self):
        """One activation buffer (M, K_p) and 2 output buffers (M, N_p) per projection."""
        xs, outs = [], []
        for N, K in self.shapes:
            xs.append(torch.empty((self.M, K), dtype=torch.float16, device=self.device))
            outs.append([torch.empty((self.M, N), dtype=torch.float16, device=self.device) for _ in range(2)])
        return xs, outs

    def bind(self, xs: List[torch.Tensor], outs: List[List[torch.Tensor]]):
        if len(xs) != len(self.shapes) or len(outs) != len(self.shapes):
            raise ValueError("one activation and 2 outputs per projection")
        tab = np.zeros(len(self.shapes), DUAL_PROJ_DTYPE)
        base = self.pack.codes.data_ptr()
        for p, ((N, K), pos0) in enumerate(zip(self.shapes, self.pos0)):
            x, o = xs[p], outs[p]
            if x.shape != (self.M, K) or x.dtype != torch.float16 or x.stride(1) != 1 or x.data_ptr() % 16 \
                    or (self.M > 1 and x.stride(0) % 8):
                raise ValueError(f"projection {p}: activations must be fp16 ({self.M}, {K}), unit stride, "
                                 "16-byte aligned")
            for t in o:
                if t.shape != (self.M, N) or t.dtype != torch.float16 or t.stride(1) != 1:
                    raise ValueError(f"projection {p}: outputs must be fp16 ({self.M}, {N}), unit stride")
            if o[0].stride(0) != o[1].stride(0):
                raise ValueError(f"projection {p}: the 2 outputs must share a row stride")
            tab[p]["codes"] = base + 2 * int(pos0)
            tab[p]["ldc"] = K
            tab[p]["pos0"] = int(pos0)
            tab[p]["x"] = x.data_ptr()
            tab[p]["x_sm"] = x.stride(0)
            tab[p]["out"] = [t.data_ptr() for t in o]
            tab[p]["o_sm"] = o[0].stride(0)
            tab[p]["N"] = N
            tab[p]["K"] = K
        self.projs = torch.from_numpy(tab.view(np.uint8).copy()).to(self.device)
        self._bound = (xs, outs)
        if self.direct:
            self._proj = nat.DualProj.from_buffer_copy(tab[0].tobytes())

    def _call_direct(self):
        pk = self.pack
        amp, cos, sin = self.luts
        P = int(pk.plug_idx.numel())
        if self.task_cap > 0:
            ent, P = (self.task_ent, P) if self.task_ent is not None else (None, 0)
        else:
            ent = self.plug_ent
        rc = nat.lib().pp_dual_rows(C.byref(self._proj), self.task_plug.data_ptr(), self.task_cap, self.plug_windows,
                                    self.code_layout, pk.scales.data_ptr(), int(pk.scales.numel()), pk.group_size,
                                    pk.chunk_size, self.scale_tab.data_ptr() if self.scale_tab is not None else None,
                                    int(self.scale_tab.numel()) if self.scale_tab is not None else 0,
                                    amp.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                    pk.plug_idx.data_ptr() if P else None, pk.plug_val.data_ptr() if P else None,
                                    ent.data_ptr() if P else None, P, self.M,
                                    self.workspace.data_ptr() if self.workspace is not None else None,
                                    self._ws_bytes, nat.raw_stream(self.device))
        nat.check(rc, "pp_dual_rows")

    def __call__(self):
        if self.projs is None:
            raise RuntimeError("DualStream.bind() must be called before launching")
        if self.direct:
            return self._call_direct()
        pk = self.pack
        stream = nat.raw_stream(self.device)
        amp, cos, sin = self.luts
        rc = nat.lib().pp_dual_stream(self.projs.data_ptr(), len(self.shapes),
                                      self.segs.data_ptr() if self.n_segs else None, self.n_segs,
                                      self.bounds.data_ptr(), self.n_waves,
                                      self.workspace.data_ptr() if self.workspace is not None else None,
                                      self.task_plug.data_ptr() if self.n_tasks else None, self.n_tasks,
                                      self.plug_windows,
                                      self.tail_items.data_ptr() if self.n_tail else None, self.n_tail,
                                      self.code_layout, pk.scales.data_ptr(), int(pk.scales.numel()),
                                      pk.group_size, pk.chunk_size,
                                      self.scale_tab.data_ptr() if self.scale_tab is not None else None,
                                      int(self.scale_tab.numel()) if self.scale_tab is not None else 0,
                                      amp.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                      pk.plug_idx.data_ptr() if pk.plug_idx.numel() else None,
                                      pk.plug_val.data_ptr() if pk.plug_val.numel() else None,
                                      self.plug_ent.data_ptr(),
                                      int(pk.plug_idx.numel()), pk.n_codes, self._tail_ptrs, self._tail_len,
                                      self.M, stream)
        nat.check(rc, "pp_dual_stream")

    def algorithmic_bytes(self) -> int:
        """2*N*K codes + 2 B per group scale + 6 B per plug entry + 2*M*K x + 4*M*N outputs
        + 2 B per tail weight read."""
        plug = self.pack.plug_host()
        gs = self.pack.group_size
        n = self.pack.n_codes
        total = 0
        for (N, K), pos0 in zip(self.shapes, self.pos0):
            lo, hi = int(pos0), int(pos0) + N * K
            in_codes = max(0, min(hi, n) - lo)
            P = int(np.searchsorted(plug, hi) - np.searchsorted(plug, lo))
            tail_w = sum(max(0, min(hi, n + t) - max(lo, n)) for t in self.pack.tail_lengths)
            total += 2 * in_codes + 2 * (-(-in_codes // gs)) + 6 * P + 2 * self.M * K + 4 * self.M * N + 2 * tail_w
        return total


def mfma_slices(N, K, waves):
    """(slices, slice_cols) for the batch decode of an (N, K) projection: as many K slices
    of whole 32-column steps as keep the 16-row x slice items within one per wavefront
    (one item more than the wavefronts would double the launch for the waves that take
    two)."""
    tiles = -(-int(N) // 16)
    s = max(1, min(int(K) // 32, int(waves) // tiles))
    cols = -(-int(K) // s)
    cols = -(-cols // 32) * 32
    return -(-int(K) // cols), cols


def mfma_row_plug(plug_host, pos0, N, K, ldc, slices, cols):
    """First plug entry at or after each (row, slice) start, then the end of the projection."""
    keys = (int(pos0) + np.arange(int(N), dtype=np.int64)[:, None] * int(ldc)
            + np.arange(int(slices), dtype=np.int64)[None, :] * int(cols)).reshape(-1)
    keys = np.concatenate([keys, [int(pos0) + int(N) * int(ldc)]])
    return np.searchsorted(plug_host, keys, side="left").astype(np.int64)


class QuadBatch:
    """Batch decode of one projection of a quad stream on the matrix cores
    (``pp_quad_mfma``, 1..64 tokens): the (N, K) block at stream position ``pos0``.

    The K slices and their plug starts are planned once; with several slices the float32
    accumulators live in a workspace owned by this object (two launches of one QuadBatch
    must not overlap).
    """

    def __init__(self, pack: QuadPackDevice, N: int, K: int, pos0: int = 0, M: int = 16, slices=None):
        L = nat.lib()
        self.pack = pack
        self.N, self.K, self.pos0, self.M = int(N), int(K), int(pos0), int(M)
        if not 1 <= self.M <= 64:
            raise ValueError("the batch decode takes 1..64 tokens")
        if self.K % 32 or self.pos0 + self.N * self.K > pack.n:
            raise ValueError("needs K % 32 == 0 and the projection inside the coded stream")
        self.device = pack.codes.device
        if slices is None:
            self.slices, self.cols = mfma_slices(self.N, self.K, int(L.pp_quad_mfma_waves(self.M)))
        else:
            self.slices = int(slices)
            cols = -(-self.K // self.slices)
            self.cols = -(-cols // 32) * 32
            self.slices = -(-self.K // self.cols)
        plug = pack.plug_host()
        self.row_plug = torch.from_numpy(mfma_row_plug(plug, self.pos0, self.N, self.K, self.K, self.slices,
                                                       self.cols)).to(self.device)
        lo, hi = np.searchsorted(plug, [self.pos0, self.pos0 + self.N * self.K])
        self.n_plug = int(hi - lo)
        ws = int(L.pp_quad_mfma_workspace_size(self.M, self.N, self.slices))
        self.workspace = torch.zeros(ws, dtype=torch.uint8, device=self.device) if ws else None
        self.luts = header_luts(pack.r_max, device=self.device)
        self._lut_ptrs = nat.ptr_array([t.data_ptr() for t in self.luts])
        self._scales = nat.float_array(pack.s)
        self.x = self.outs = None

    def make_buffers(self):
        x = torch.empty((self.M, self.K), dtype=torch.float16, device=self.device)
        return x, [torch.empty((self.M, self.N), dtype=torch.float16, device=self.device) for _ in range(4)]

    def bind(self, x: torch.Tensor, outs: List[torch.Tensor]):
        if x.shape != (self.M, self.K) or x.dtype != torch.float16 or x.stride(1) != 1 or x.data_ptr() % 16 \
                or (self.M > 1 and x.stride(0) % 8):
            raise ValueError(f"activations must be fp16 ({self.M}, {self.K}), unit stride, 16-byte aligned rows")
        if len(outs) != 4 or any(o.shape != (self.M, self.N) or o.dtype != torch.float16 or o.stride(1) != 1
                                 or o.stride(0) != outs[0].stride(0) for o in outs):
            raise ValueError(f"4 fp16 outputs ({self.M}, {self.N}) with one row stride")
        self.x, self.outs = x, outs
        self._out_ptrs = nat.ptr_array([o.data_ptr() for o in outs])

    def __call__(self):
        if self.x is None:
            raise RuntimeError("QuadBatch.bind() must be called before launching")
        pk = self.pack
        stream = nat.raw_stream(self.device)
        rc = nat.lib().pp_quad_mfma(pk.codes.data_ptr() + 4 * self.pos0, self.K, self.pos0, self.x.data_ptr(),
                                    self.x.stride(0), self._lut_ptrs, nat.PP_F32, self._scales,
                                    pk.plug_idx.data_ptr() if pk.plug_idx.numel() else None,
                                    pk.plug_vals.data_ptr() if pk.plug_vals.numel() else None,
                                    int(pk.plug_idx.numel()), self.row_plug.data_ptr(), self.slices, self.cols,
                                    self._out_ptrs, self.outs[0].stride(0), self.M, self.N, self.K,
                                    self.workspace.data_ptr() if self.workspace is not None else None,
                                    int(self.workspace.numel()) if self.workspace is not None else 0, stream)
        nat.check(rc, "pp_quad_mfma")

    def algorithmic_bytes(self) -> int:
        """4*N*K codes + 12 B per plug entry + 2*M*K x + 8*M*N outputs."""
        return 4 * self.N * self.K + 12 * self.n_plug + 2 * self.M * self.K + 8 * self.M * self.N
