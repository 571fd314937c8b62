"""Plug tables in the order the kernels read them.

A ``.quadpack`` / ``.dualpack`` plug table is strictly ascending by construction
(quaternion_packer.py:104-113 takes ``np.where`` of a mask; polar_bitpack.py:154-157 sorts the
entries of all chunks), and the kernels rely on it: the row kernels consume a task's entries
in order and the matrix-core routes binary-search them.  A caller of a drop-in operator may
pass a table of its own, so every operator call goes through :func:`ascending`, which returns
the table with its entries sorted by position and, where one position appears more than once,
only the last of its entries kept in place (the others are moved to position 0xFFFFFFFF, past
every stream; the reference's unpackers assign the plug values with one fancy-indexed store,
quaternion_packer.py:187-193, polar_bitpack.py:240-243, so the last duplicate wins).

The sorted copy is made on the device once per table and cached, keyed on the two tensor
objects and their version counters (an in-place change of either makes a new copy); the
entry goes when the index tensor is freed.  Under stream capture a table that is not cached
yet is sorted inside the captured work and not cached (its memory belongs to the graph).
"""
from __future__ import annotations

import threading
import weakref

import torch

_lock = threading.Lock()
_cache = {}          # (id(idx), id(vals)) -> (weakref idx, weakref vals, idx version, vals version, result)

NO_POSITION = 0xFFFFFFFF


def _sorted(idx: torch.Tensor, vals: torch.Tensor):
    P = idx.numel()
    pos = idx.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    s, order = torch.sort(pos, stable=True)
    last = torch.ones(P, dtype=torch.bool, device=idx.device)
    if P > 1:
        last[:-1] = s[:-1] != s[1:]
    s2, order2 = torch.sort(torch.where(last, s, NO_POSITION), stable=True)
    perm = order[order2]
    out_idx = torch.where(s2 >= 1 << 31, s2 - (1 << 32), s2).to(torch.int32)
    if idx.dtype == torch.uint32:
        out_idx = out_idx.view(torch.uint32)
    width = vals.numel() // P
    out_vals = vals.reshape(P, width)[perm].reshape(vals.shape).contiguous()
    return out_idx.contiguous(), out_vals


def ascending(idx: torch.Tensor, vals: torch.Tensor):
    """``(idx, vals)`` as the kernels need them: positions strictly ascending (duplicates
    resolved as described above), values permuted alike.  ``idx`` uint32 or int32 holding
    uint32 bits, ``vals`` (P, w) or (P,) with the entries along the first axis."""
    if idx.numel() <= 1:
        return idx, vals
    key = (id(idx), id(vals))
    with _lock:
        hit = _cache.get(key)
    if hit is not None:
        ri, rv, vi, vv, res = hit
        if ri() is idx and rv() is vals and idx._version == vi and vals._version == vv:
            return res
    res = _sorted(idx, vals)
    if torch.cuda.is_available() and idx.is_cuda and torch.cuda.is_current_stream_capturing():
        return res
    with _lock:
        _cache[key] = (weakref.ref(idx), weakref.ref(vals), idx._version, vals._version, res)
    weakref.finalize(idx, _forget, key)
    return res


def _forget(key) -> None:
    with _lock:
        _cache.pop(key, None)


def clear() -> None:
    """Drop every cached sorted table."""
    with _lock:
        _cache.clear()
