"""CPU oracle for the polar_pack decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or, for the CPU baseline, as the timed reference CPU path).

Contents (each function cites the reference file:line it restates):

* :mod:`oracle.quadpack` -- ``.quadpack`` v2 container: header, packer,
  float64 unpacker (quaternion_packer.py).
* :mod:`oracle.dualpack` -- ``.dualpack`` v2 container: header, packer,
  float64 unpacker (polar_bitpack.py).
* :mod:`oracle.layer`    -- the kernel-layout packers ``pack_quad_layer``
  (quad_kernels.py:16-50) and ``quantize_polar_bitpacked``
  (polar_kernels.py:9-11, 118-151), plus float64 dequant / GEMM references
  for the kernel-layout operands (quad_kernels.py:103-134,
  polar_kernels.py:64-95).

How each part is pinned (tests/test_oracle_*.py):

* packers: bit-exact against golden vectors written by importing the
  reference's own packer functions (tests/golden/make_golden.py);
* decoders: closed forms and special cases (zero tuple, single-axis tuples,
  (1,1,1,1) angles, exact LUT end points), byte-exact header sizes and
  offsets, exhaustive code-field round trips, plug/tail substitution
  invariants, and re-decoding of the reference-written golden containers;
* GEMV: brute force float64 on tiny shapes.
"""
