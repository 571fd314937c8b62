"""The device dual packer (pack_dual_device) run on CPU torch tensors, against the
reference's own .dualpack files (tests/golden) and the oracle packer."""
import os

import numpy as np
import pytest
import torch

import make_golden as mg
from oracle import dualpack as odp
from parity import assert_same_dual_pack, dual_codes_u16
from polar_pack_amd.packer import pack_dual_device

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("case", mg.DUALPACK_CASES, ids=[c[0] for c in mg.DUALPACK_CASES])
def test_device_packer_matches_reference_file(case):
    name, n1, n2, seed, cap, chunk = case
    dp = odp.DualPack.from_bytes(np.load(os.path.join(HERE, name + ".npz"))["packed"].tobytes())
    w1, w2 = mg.dualpack_inputs(n1, n2, seed)
    pack = pack_dual_device(torch.from_numpy(w1), torch.from_numpy(w2), plug_cap=cap, chunk_size=chunk)
    assert (pack.n1, pack.n2, pack.chunk_size, pack.group_size) == (dp.n1, dp.n2, dp.chunk_size, dp.group_size)
    assert pack.tails == []
    assert_same_dual_pack(pack, dp)


def test_device_packer_i16_layout_is_the_kernel_layout():
    w1, w2 = mg.dualpack_inputs(6000, 6000, 5)
    a = pack_dual_device(torch.from_numpy(w1), torch.from_numpy(w2), plug_cap=0.01, layout="u16be")
    b = pack_dual_device(torch.from_numpy(w1), torch.from_numpy(w2), plug_cap=0.01, layout="i16")
    be = a.codes.numpy().view(np.uint16)
    swapped = ((be.astype(np.uint32) & 0xFF) << 8) | (be >> 8)
    np.testing.assert_array_equal(b.codes.numpy().view(np.uint16), (swapped ^ 0x8000).astype(np.uint16))


@pytest.mark.parametrize("longer", [1, 2])
def test_device_packer_tail_mode(longer):
    """Tail mode = the format's pack of the common length + the longer model's rest in fp16."""
    n_long, n_short = 9000, 8123
    n = 8120                                     # the common length rounded down to a multiple of 8
    lens = [n_long, n_short] if longer == 1 else [n_short, n_long]
    w1, w2 = mg.dualpack_inputs(lens[0], lens[1], 77)
    pack = pack_dual_device(torch.from_numpy(w1), torch.from_numpy(w2), plug_cap=0.03, chunk_size=1000, tails=True)
    dp = odp.pack_dual(w1[:n], w2[:n], odp.DualConfig(plug_cap=0.03, chunk_size=1000))
    assert_same_dual_pack(pack, dp)
    assert pack.tail_lengths == [lens[0] - n, lens[1] - n]
    for m, src in enumerate((w1, w2)):
        np.testing.assert_array_equal(pack.tails[m].numpy(), src[n:].astype(np.float16))


def test_device_packer_norm_selection_takes_the_largest_amplitudes():
    w1, w2 = mg.dualpack_inputs(4000, 4000, 9)
    pack = pack_dual_device(torch.from_numpy(w1), torch.from_numpy(w2), plug_cap=0.01, select="norm",
                            chunk_size=1000)
    amp = np.sqrt(w1.astype(np.float32) ** 2 + w2.astype(np.float32) ** 2)
    pi = pack.plug_idx.view(torch.int32).numpy()
    assert pi.size == 40
    for c in range(4):
        sel = pi[(pi >= 1000 * c) & (pi < 1000 * (c + 1))]
        assert sel.size == 10
        assert amp[sel].min() >= np.sort(amp[1000 * c:1000 * (c + 1)])[-10]
    np.testing.assert_array_equal(pack.plug_val.numpy(), amp[pi].astype(np.float16))


def test_device_packer_rejects_bad_arguments():
    w = torch.zeros(100)
    with pytest.raises(ValueError):
        pack_dual_device(w, w, layout="le")
    with pytest.raises(ValueError):
        pack_dual_device(w.view(10, 10), w)
    with pytest.raises(ValueError):
        pack_dual_device(w, w, amp_bits=7)
