"""Write the golden vectors under tests/golden/ by running the reference's packers.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py [--ref /root/reference]

Only the packer functions are imported and run -- their float32 rounding
ties, ``default_rng(42)`` window sampling and ``np.argpartition`` order can
be pinned no other way.  Decoders are pinned by closed forms in the tests and
are not imported here.  Inputs are regenerated from :mod:`tests.golden.gen`
(bit-stable integer-hash draws), so only outputs are stored.
"""
from __future__ import annotations

import argparse
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import gen  # noqa: E402

# Golden-case tables (shared with the tests through the .npz metadata).
QUAD_LAYER_CASES = [  # (name, K, N, seed, correlated)
    ("ql_64x48_corr", 64, 48, 11, True),
    ("ql_96x130_corr", 96, 130, 12, True),
    ("ql_256x96_rand", 256, 96, 13, False),
]
DUAL_LAYER_CASES = [  # (name, K, N, seed, dtype)
    ("dl_64x96_f16", 64, 96, 21, "float16"),
    ("dl_128x64_f32", 128, 64, 22, "float32"),
    ("dl_33x40_f16", 33, 40, 23, "float16"),   # K*N not a multiple of 32
]
QUADPACK_CASES = [  # (name, n, tails, seed, plug_cap)
    ("qp_cap0001", 1_004_093, (0, 517, 0, 1031), 31, 0.001),
    ("qp_cap005", 1_004_093, (0, 517, 0, 1031), 32, 0.05),
]
DUALPACK_CASES = [  # (name, n1, n2, seed, plug_cap, chunk_size)
    ("dp_small", 5000, 4321, 41, 0.001, 1000),
    ("dp_cap003", 70_000, 66_500, 42, 0.03, 10_001),
    ("dp_longer2", 20_000, 23_456, 43, 0.03, 50_000_000),
]


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def quad_layer_inputs(K, N, seed, correlated):
    if correlated:
        ws = gen.correlated_models(seed, [K * N] * 4)
    else:
        ws = [gen.normal(seed, 50 + i, K * N) for i in range(4)]
    return [w.reshape(K, N).astype(np.float16) for w in ws]


def dual_layer_inputs(K, N, seed, dtype):
    ws = gen.correlated_models(seed, [K * N] * 2)
    return [w.reshape(K, N).astype(dtype) for w in ws]


def quadpack_inputs(n, tails, seed):
    return gen.correlated_models(seed, [n + t for t in tails])


def dualpack_inputs(n1, n2, seed):
    return gen.correlated_models(seed, [n1, n2], delta_growth=False)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()
    sys.dont_write_bytecode = True
    sys.path.insert(0, args.ref)
    import torch
    import quad_kernels as rq          # imports triton; CPU-only functions are used
    import polar_kernels as rp
    import quaternion_packer as rqp
    import polar_bitpack as rdb
    import polar_packer as rpk

    for name, K, N, seed, corr in QUAD_LAYER_CASES:
        ws = [torch.from_numpy(w) for w in quad_layer_inputs(K, N, seed, corr)]
        codes, luts, scales = rq.pack_quad_layer(*ws)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), K=K, N=N, seed=seed, correlated=corr,
                            codes=codes.numpy().view(np.uint32) if hasattr(codes, "numpy") else codes,
                            luts=np.stack([l.numpy() for l in luts]), scales=np.array(scales, np.float64))
        print("wrote", name)

    for name, K, N, seed, dt in DUAL_LAYER_CASES:
        w1, w2 = [torch.from_numpy(w) for w in dual_layer_inputs(K, N, seed, dt)]
        packed, bmax, amp_lut, cos_lut, sin_lut = rp.quantize_polar_bitpacked(w1, w2)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), K=K, N=N, seed=seed, dtype=dt,
                            packed=packed.numpy(), bmax=bmax.numpy(), amp_lut=amp_lut.numpy(),
                            cos_lut=cos_lut.numpy(), sin_lut=sin_lut.numpy())
        print("wrote", name)

    with tempfile.TemporaryDirectory() as td:
        for name, n, tails, seed, cap in QUADPACK_CASES:
            models = quadpack_inputs(n, tails, seed)
            path = os.path.join(td, "g.quadpack")
            rqp.pack_quad(models, path, plug_cap=cap)
            buf = open(path, "rb").read()
            hs = rqp.HEADER_SIZE
            codes = np.frombuffer(buf, dtype="<u4", count=n, offset=hs)
            hdr = np.frombuffer(buf, dtype=np.uint8, count=hs)
            import struct
            plug_n = struct.unpack(rqp.HEADER_FMT, buf[:hs])[9]
            pidx = np.frombuffer(buf, dtype="<u4", count=plug_n, offset=hs + 4 * n)
            pval = np.frombuffer(buf, dtype="<f2", count=4 * plug_n, offset=hs + 4 * n + 4 * plug_n)
            keep = min(plug_n, 2000)
            np.savez_compressed(os.path.join(HERE, f"{name}.npz"), n=n, tails=np.array(tails), seed=seed,
                                plug_cap=cap, header=hdr, file_sha=hashlib.sha256(buf).hexdigest(),
                                file_size=len(buf), codes_sha=sha(codes), codes_head=codes[:4096].copy(),
                                codes_tail=codes[-4096:].copy(), plug_n=plug_n, plug_idx_sha=sha(pidx),
                                plug_vals_sha=sha(pval), plug_idx_head=pidx[:keep].copy(),
                                plug_vals_head=pval[:4 * keep].copy())
            print("wrote", name, "plug_n", plug_n)

        for name, n1, n2, seed, cap, chunk in DUALPACK_CASES:
            w1, w2 = dualpack_inputs(n1, n2, seed)
            f1, f2 = os.path.join(td, "m1.dat"), os.path.join(td, "m2.dat")
            w1.tofile(f1)
            w2.tofile(f2)
            cfg = rpk.PackerConfig(plug_cap=cap, chunk_size=chunk)
            out = os.path.join(td, "g.dualpack")
            rdb.pack_dual_models_packed(f1, f2, n1, n2, out, cfg)
            buf = open(out, "rb").read()
            np.savez_compressed(os.path.join(HERE, f"{name}.npz"), n1=n1, n2=n2, seed=seed, plug_cap=cap,
                                chunk_size=chunk, packed=np.frombuffer(buf, dtype=np.uint8))
            print("wrote", name, "bytes", len(buf))


if __name__ == "__main__":
    main()
