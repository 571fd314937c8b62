"""Host logic of the one-launch stream decode: task coverage, segments, plug starts, wave balance."""
import ctypes

import numpy as np
import pytest

from polar_pack_amd import _native as nat
from polar_pack_amd.stream import (DUAL_PROJ_DTYPE, ITEM_DTYPE, SEG_DTYPE, plan_segments, plan_tail_items, plan_tasks, task_bytes,
                                   wave_bounds)

SHAPES = [(2048, 2048), (256, 2048), (256, 2048), (2048, 2048), (11008, 2048), (11008, 2048), (2048, 11008)]


def seg_coverage(segs, shapes):
    cov = [np.zeros(N, np.int8) for N, _ in shapes]
    for s in segs:
        cov[int(s["proj"])][int(s["row0"]):int(s["row1"])] += 1
    return cov


@pytest.mark.parametrize("rpt", [4, 2, 1])
@pytest.mark.parametrize("waves", [1, 7, 64, 4096])
def test_segments_cover_every_row_once(rpt, waves):
    shapes = [(37, 2048), (5, 11008), (8, 256), (3, 4100)]
    n = sum(a * b for a, b in shapes)
    segs, bounds, _ = plan_segments(shapes, n, np.zeros(0, np.uint32), waves, rpt)
    for c in seg_coverage(segs, shapes):
        assert c.min() == 1 and c.max() == 1
    assert bounds.size == waves + 1 and bounds[0] == 0 and bounds[-1] == segs.size
    assert np.all(np.diff(bounds) >= 0)
    # each wave's segments are in stream order and no segment spans projections
    assert np.all(segs["row1"] > segs["row0"])
    # segments start on task boundaries of their projection
    assert np.all(segs["row0"] % rpt == 0)


def test_tail_rows_and_plug_ranges():
    shapes = [(4, 100), (6, 64)]
    n = 4 * 100 + 2 * 64 + 10           # projection 1: rows 0-1 in codes, row 2 straddles, rows 3-5 tail
    plug = np.array([5, 99, 100, 399, 400, 463, 464, 527, 528, 537], np.uint32)
    segs, bounds, _ = plan_segments(shapes, n, plug, 3, 4)
    tail = plan_tail_items(shapes, n, plug)
    assert list(tail["proj"]) == [1, 1, 1, 1] and list(tail["row0"]) == [2, 3, 4, 5]
    assert np.all(tail["flags"] == nat.PP_ITEM_TAIL) and np.all(tail["nrows"] == 1)
    cov = seg_coverage(segs, shapes)
    assert cov[0].tolist() == [1, 1, 1, 1] and cov[1].tolist() == [1, 1, 0, 0, 0, 0]
    pos0 = [0, 400]
    for s in segs:
        start = pos0[int(s["proj"])] + int(s["row0"]) * shapes[int(s["proj"])][1]
        assert int(s["plug_lo"]) == int(np.searchsorted(plug, start))      # first entry >= start
    for it in tail:
        lo = 400 + int(it["row0"]) * 64
        expect = np.nonzero((plug >= lo) & (plug < lo + 64))[0]
        np.testing.assert_array_equal(np.arange(int(it["plug_lo"]), int(it["plug_hi"])), expect)


def test_wave_bounds_balance_bytes():
    shapes = SHAPES * 3
    n = sum(a * b for a, b in shapes)
    proj, row0, nrows = plan_tasks(shapes, n, 4)
    b = task_bytes(proj, nrows, shapes)
    W = 4096
    bounds = wave_bounds(b, W)
    assert bounds[0] == 0 and bounds[-1] == b.size and np.all(np.diff(bounds) >= 0)
    per = np.add.reduceat(np.concatenate([b, [0]]), bounds[:-1])[:W]
    per[np.diff(bounds) == 0] = 0
    assert per.sum() == b.sum()
    assert per.max() <= b.sum() / W + b.max()          # at most one task over the even share


def test_struct_layouts_match_abi():
    assert ITEM_DTYPE.itemsize == ctypes.sizeof(nat.QuadItem) == 32
    for name, _ in nat.QuadItem._fields_:
        assert getattr(nat.QuadItem, name).offset == ITEM_DTYPE.fields[name][1]
    assert SEG_DTYPE.itemsize == ctypes.sizeof(nat.QuadSeg) == 48
    for name, _ in nat.QuadSeg._fields_:
        assert getattr(nat.QuadSeg, name).offset == SEG_DTYPE.fields[name][1]
    assert DUAL_PROJ_DTYPE.itemsize == ctypes.sizeof(nat.DualProj) == 72
    for name, _ in nat.DualProj._fields_:
        assert getattr(nat.DualProj, name).offset == DUAL_PROJ_DTYPE.fields[name][1]


def test_task_plug_ranges_partition_the_plug_table():
    from polar_pack_amd.stream import plan_task_plug
    shapes = [(24, 1024), (8, 2048), (3, 16), (9, 520)]
    total = sum(n * k for n, k in shapes)
    n = total - 700                      # the last projection's last rows reach the tails
    plug = np.sort(np.random.default_rng(3).choice(n, 900, replace=False)).astype(np.uint32)
    for rg in (2, 4, 8):
        tab, nck = plan_task_plug(shapes, n, plug, rg)
        proj, row0, nrows = plan_tasks(shapes, n, rg)
        assert tab.shape == (proj.size, 2) and nck.shape == (proj.size,)
        pos = np.cumsum([0] + [a * b for a, b in shapes])
        K = np.array([b for _, b in shapes])
        for t in range(proj.size):
            lo = pos[proj[t]] + row0[t] * K[proj[t]]
            hi = lo + nrows[t] * K[proj[t]]
            sel = plug[tab[t, 0]:tab[t, 1]].astype(np.int64)
            assert np.all((sel >= lo) & (sel < hi))
            assert np.count_nonzero((plug >= lo) & (plug < hi)) == sel.size
        assert np.all(nck == (K[proj] + 511) // 512)
    segs, _, _ = plan_segments(shapes, n, plug, 16, 4, code_bytes=2)
    proj, row0, _ = plan_tasks(shapes, n, 4)
    assert np.all(proj[segs["task0"]] == segs["proj"]) and np.all(row0[segs["task0"]] == segs["row0"])


def test_tail_items_fp16_runs():
    from polar_pack_amd.stream import plan_tail_items
    shapes = [(10, 64), (20, 32), (5, 16)]
    n = 3 * 64 + 16                    # row 3 of projection 0 straddles n
    tails = [10 * 64 + 20 * 32 + 5 * 16 - n, 6 * 64 + 4 * 32 + 8]   # model 2's tail ends inside a row
    plug = np.array([1, 50, 200, 205], np.uint32)
    it = plan_tail_items(shapes, n, plug, tails, fp16_rows=4)
    pos = np.cumsum([0] + [a * b for a, b in shapes])
    covered = []
    for x in it:
        p, r0, nr, fl = int(x["proj"]), int(x["row0"]), int(x["nrows"]), int(x["flags"])
        K = shapes[p][1]
        lo, hi = pos[p] + r0 * K, pos[p] + (r0 + nr) * K
        covered += [(p, r) for r in range(r0, r0 + nr)]
        if fl == 2:
            assert 1 <= nr <= 4 and lo >= n and x["plug_lo"] == x["plug_hi"] == 0
            for L in tails:            # every row wholly inside or wholly past each tail
                for r in range(nr):
                    a, b = lo + r * K, lo + (r + 1) * K
                    assert b <= n + L or a >= n + L
        else:
            assert fl == 1 and nr == 1
            assert x["plug_lo"] == np.searchsorted(plug, lo) and x["plug_hi"] == np.searchsorted(plug, hi)
    expect = [(p, r) for p, (N, K) in enumerate(shapes) for r in range(N) if pos[p] + (r + 1) * K > n]
    assert covered == expect
    assert int((it["flags"] == 1).sum()) == 2            # the row across n, the row across model 2's tail end
    plain = plan_tail_items(shapes, n, plug)
    assert np.all(plain["flags"] == 1) and np.all(plain["nrows"] == 1) and plain.size == len(expect)


@pytest.mark.parametrize("shape,waves", [((11008, 2048), 8192), ((2048, 11008), 2048), ((256, 2048), 2048),
                                         ((40, 1000), 64)])
def test_split_segments_cover_every_task_slice_once(shape, waves):
    N, K = shape
    shapes = [shape]
    n = N * K
    plug = np.sort(np.random.default_rng(1).choice(n, 500, replace=False)).astype(np.uint32)
    rpt = 8
    segs, bounds, ws = plan_segments(shapes, n, plug, waves, rpt, split=True)
    parts = int(segs["parts"][0])
    assert np.all(segs["parts"] == parts) and parts > 1
    ntask = -(-N // rpt)
    assert ws >= 4 * ntask + 4 * 4 * N
    # every (task, column) pair covered exactly once, slices on 512-column boundaries
    cover = np.zeros((ntask, K), np.int32)
    for g in segs:
        assert g["k0"] % 512 == 0 and (g["k1"] % 512 == 0 or g["k1"] == K) and g["k0"] < g["k1"] <= K
        t0 = g["row0"] // rpt
        assert g["task0"] == t0 and g["plug_lo"] == np.searchsorted(plug, g["row0"] * K)
        for t in range(t0, -(-g["row1"] // rpt)):
            cover[t, g["k0"]:g["k1"]] += 1
        assert g["acc_off"] * 4 >= 4 * ntask and g["acc_off"] % 64 == 0
        assert (g["acc_off"] + 4 * N) * 4 <= ws
    assert np.all(cover == 1)
    # each task is cut into exactly `parts` slices
    slices = {}
    for g in segs:
        for t in range(g["row0"] // rpt, -(-g["row1"] // rpt)):
            slices.setdefault(t, set()).add(int(g["k0"]))
    assert all(len(v) == parts for v in slices.values())
    assert np.all(np.diff(bounds) >= 0) and bounds[-1] == segs.size


def test_large_streams_are_not_split():
    shapes = [(2048, 2048), (11008, 2048)] * 20
    n = sum(a * b for a, b in shapes)
    segs, _, ws = plan_segments(shapes, n, np.zeros(0, np.uint32), 2048, 8, split=True)
    assert np.all(segs["parts"] == 1) and ws == 0
    assert np.all(segs["k0"] == 0) and np.all(segs["k1"] == np.array([b for _, b in shapes])[segs["proj"]])


def test_layer_map_projections_skip_non_linear_entries():
    """Every entry advances the stream position by its numel; entries that are not an
    (N, K) Linear are skipped (polar_packer.py:297-305)."""
    from polar_pack_amd.stream import layer_map_projections
    info = [{"name": "model.layers.0.q", "shape": [8, 16], "numel": 128},
            {"name": "model.norm", "shape": [16], "numel": 16},
            {"name": "model.layers.0.k", "shape": [4, 16], "numel": 64},
            {"name": "bad", "shape": [4, 4], "numel": 20},
            {"name": "lm_head", "shape": [12, 16], "numel": 192}]
    names, shapes, pos = layer_map_projections(info)
    assert names == ["model.layers.0.q", "model.layers.0.k", "lm_head"]
    assert shapes == [(8, 16), (4, 16), (12, 16)]
    assert pos == [0, 144, 228]


def test_layer_map_projections_with_a_model():
    import torch
    from polar_pack_amd.stream import layer_map_projections
    m = torch.nn.Sequential(torch.nn.Linear(16, 8), torch.nn.SiLU(), torch.nn.Embedding(4, 16), torch.nn.Linear(16, 6))
    info = [{"name": "0", "shape": [8, 16], "numel": 128}, {"name": "2", "shape": [4, 16], "numel": 64},
            {"name": "3", "shape": [5, 16], "numel": 80}]        # a size that does not match the module
    names, shapes, pos = layer_map_projections(info, model=m)
    assert names == ["0"] and pos == [0]


def test_positioned_plans_match_back_to_back_plans_shifted():
    """Projections at explicit positions (gaps between them, as skipped layer-map entries
    leave) plan the same segments as back-to-back ones, with plug starts and tail items
    found at the real positions."""
    shapes = [(37, 2048), (5, 1024), (8, 256)]
    gaps = [0, 300, 17]
    pos = np.cumsum([g + (shapes[i - 1][0] * shapes[i - 1][1] if i else 0) for i, g in enumerate(gaps)])
    end = int(pos[-1]) + 8 * 256
    n = end - 3 * 256 - 5                 # the last projection's last rows reach the tails
    rng = np.random.default_rng(0)
    plug = np.sort(rng.choice(end, 400, replace=False)).astype(np.uint32)
    segs, bounds, _ = plan_segments(shapes, n, plug, 16, 4, positions=pos)
    cov = seg_coverage(segs, shapes)
    assert [c.tolist() for c in cov[:2]] == [[1] * 37, [1] * 5]
    assert cov[2].tolist() == [1] * 4 + [0] * 4
    for s in segs:
        start = int(pos[int(s["proj"])]) + int(s["row0"]) * shapes[int(s["proj"])][1]
        assert int(s["plug_lo"]) == int(np.searchsorted(plug, start))
    tail = plan_tail_items(shapes, n, plug, positions=pos)
    assert list(tail["proj"]) == [2] * 4 and list(tail["row0"]) == [4, 5, 6, 7]
    for it in tail:
        lo = int(pos[2]) + int(it["row0"]) * 256
        expect = np.nonzero((plug >= lo) & (plug < lo + 256))[0]
        np.testing.assert_array_equal(np.arange(int(it["plug_lo"]), int(it["plug_hi"])), expect)
    with pytest.raises(ValueError):
        plan_segments(shapes, n, plug, 16, 4, positions=[0, 10, 20])       # overlapping
