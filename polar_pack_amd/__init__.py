"""polar_pack_amd: MI355X-native (gfx950) fused dequant-matmul decode for polar_pack.

Modules mirror the reference's operator files:

* :mod:`polar_pack_amd.quad_kernels`  -- drop-in for quad_kernels.py
* :mod:`polar_pack_amd.polar_kernels` -- drop-in for polar_kernels.py
* :mod:`polar_pack_amd.container`     -- .quadpack / .dualpack v2 readers and writers
* :mod:`polar_pack_amd.stream`        -- whole-stream batch-1 decode step (one launch)

All compute runs in the HIP library ``lib/libpolar_pack.so`` (C ABI in
include/polar_pack.h); there is no CPU or eager fallback.
"""
__version__ = "0.1.0"
