"""The product's container readers and writers on the reference-written files (CPU only).

``DualPackFile.read`` restates polar_bitpack.py:194-211 (62-byte header, big-endian codes,
per-chunk group scales, plug positions and amplitudes); the committed ``dp_*`` fixtures
are files written by the reference's own ``pack_dual_models_packed`` (chunk restarts,
n1 != n2, plug caps 0.001 and 0.03).  The oracle's reader is pinned against the same
bytes in test_oracle_golden.py.
"""
import os

import numpy as np
import pytest

import make_golden as mg
from oracle import dualpack as odp
from polar_pack_amd.container import DualPackFile, QuadPackFile, dual_n_groups

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("case", mg.DUALPACK_CASES, ids=[c[0] for c in mg.DUALPACK_CASES])
def test_dualpack_reader_on_reference_files(tmp_path, case):
    name, n1, n2, seed, cap, chunk = case
    raw = np.load(os.path.join(HERE, name + ".npz"))["packed"].tobytes()
    path = tmp_path / "g.dualpack"
    path.write_bytes(raw)
    f = DualPackFile.read(path)
    ref = odp.DualPack.from_bytes(raw)
    assert (f.n_pairs, f.n1, f.n2) == (max(n1, n2), n1, n2)
    assert (f.amp_bits, f.phase_bits, f.group_size, f.chunk_size) == (6, 10, 32, chunk)
    assert f.mu == ref.mu == 255.0
    np.testing.assert_array_equal(f.codes_be, ref.codes_be)
    assert f.scales.size == dual_n_groups(f.n_pairs, chunk, 32) == odp.n_groups_for(f.n_pairs, chunk, 32)
    np.testing.assert_array_equal(f.scales.view(np.uint16), ref.scales.view(np.uint16))
    np.testing.assert_array_equal(f.plug_idx, ref.plug_idx)
    np.testing.assert_array_equal(f.plug_val.view(np.uint16), ref.plug_val.view(np.uint16))
    assert f.plug_idx.size == sum(int(cap * min(chunk, f.n_pairs - s)) for s in range(0, f.n_pairs, chunk))
    # writing it back gives the reference's bytes
    out = tmp_path / "w.dualpack"
    f.write(out)
    assert out.read_bytes() == raw


def test_dualpack_reader_rejects_truncated_and_foreign_files(tmp_path):
    raw = np.load(os.path.join(HERE, "dp_small.npz"))["packed"].tobytes()
    short = tmp_path / "short.dualpack"
    short.write_bytes(raw[:-3])
    with pytest.raises(ValueError, match="header implies"):
        DualPackFile.read(short)
    bad = tmp_path / "bad.dualpack"
    bad.write_bytes(b"DUALPAKK" + raw[8:])
    with pytest.raises(ValueError):
        DualPackFile.read(bad)
    quad = tmp_path / "x.quadpack"
    quad.write_bytes(raw)
    with pytest.raises(ValueError):
        QuadPackFile.read(quad)
