"""Host logic of the one-launch stream decode: task coverage, plug ranges, wave balance."""
import numpy as np
import pytest

from polar_pack_amd import _native as nat
from polar_pack_amd.stream import ITEM_DTYPE, item_bytes, plan_items, wave_bounds

SHAPES = [(2048, 2048), (256, 2048), (256, 2048), (2048, 2048), (11008, 2048), (11008, 2048), (2048, 11008)]


def coverage(items, shapes):
    """Count how often each (projection, row) is covered."""
    cov = [np.zeros(N, np.int8) for N, _ in shapes]
    for it in items:
        p, r0, nr = int(it["proj"]), int(it["row0"]), int(it["nrows"])
        cov[p][r0:r0 + nr] += 1
    return cov


@pytest.mark.parametrize("rpi", [4, 2, 1])
def test_items_cover_every_row_once(rpi):
    shapes = [(37, 2048), (5, 11008), (8, 256), (3, 4100)]
    n = sum(a * b for a, b in shapes)
    items = plan_items(shapes, n, np.zeros(0, np.uint32), rpi)
    for c in coverage(items, shapes):
        assert c.min() == 1 and c.max() == 1
    assert np.all(items["nrows"] <= rpi) and not np.any(items["flags"])


def test_tail_rows_and_plug_ranges():
    shapes = [(4, 100), (6, 64)]
    n = 4 * 100 + 2 * 64 + 10           # projection 1: rows 0-1 in codes, row 2 straddles, rows 3-5 tail
    plug = np.array([5, 99, 100, 399, 400, 463, 464, 527, 528, 537], np.uint32)
    items = plan_items(shapes, n, plug, 4)
    tail = items[(items["flags"] & nat.PP_ITEM_TAIL) != 0]
    assert list(tail["proj"]) == [1, 1, 1, 1] and list(tail["row0"]) == [2, 3, 4, 5]
    for it in items:
        pos0 = 0 if it["proj"] == 0 else 400
        K = shapes[int(it["proj"])][1]
        lo = pos0 + int(it["row0"]) * K
        hi = lo + int(it["nrows"]) * K
        expect = np.nonzero((plug >= lo) & (plug < hi))[0]
        got = np.arange(int(it["plug_lo"]), int(it["plug_hi"]))
        np.testing.assert_array_equal(got, expect)


def test_wave_bounds_balance_bytes():
    shapes = SHAPES * 3
    n = sum(a * b for a, b in shapes)
    items = plan_items(shapes, n, np.zeros(0, np.uint32), 2)
    b = item_bytes(items, shapes)
    W = 4096
    bounds = wave_bounds(b, W)
    assert bounds[0] == 0 and bounds[-1] == items.size and np.all(np.diff(bounds) >= 0)
    per = np.add.reduceat(np.concatenate([b, [0]]), bounds[:-1])[:W]
    per[np.diff(bounds) == 0] = 0
    assert per.sum() == b.sum()
    assert per.max() <= b.sum() / W + b.max()          # at most one item over the even share


def test_item_struct_layout_matches_abi():
    assert ITEM_DTYPE.itemsize == 32
    import ctypes
    assert ctypes.sizeof(nat.QuadItem) == 32
    for name, _ in nat.QuadItem._fields_:
        assert getattr(nat.QuadItem, name).offset == ITEM_DTYPE.fields[name][1]
