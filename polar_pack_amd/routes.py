"""Which kernel a drop-in operator call runs: one table per operator.

A call is described by

* the kernels its code tensor's storage admits (:func:`quad_storage`, :func:`dual_storage`:
  the layout, alignment and 32-bit offset limits each kernel's entry point checks),
* the token count M,
* whether it carries plug entries,
* the ``fused`` switch of the operator (None = by size, True = the fused matrix-core kernel
  wherever it can run, False = never it above the row kernels' sizes).

The route is the first row of the operator's table whose kernel the storage admits, whose
token range holds M and whose ``plug`` / ``fused`` columns match.  ``quad_bitpacked`` and
``polar_dual_bitpacked`` read nothing else to choose a kernel; tests list every cell.

Quad kernels (the reference's one fused kernel, quad_kernels.py:53-159, at every M):

* ``rows``     fused row decode of (N,K) rows seen as (K,N) (the container stream layout),
               1-8 tokens (``pp_quad_gemm`` -> ``quad_rows_kernel``)
* ``kn``       fused row decode of (K,N) codes with unit column stride (``pack_quad_layer``),
               8 tokens per pass (``pp_quad_gemm`` -> ``quad_kn_kernel``)
* ``mfma``     matrix-core batch decode of (N,K) rows, 1-64 tokens per launch (``pp_quad_mfma``)
* ``big_nk``   fused matrix-core kernel on (N,K) rows, blocks of 16-256 tokens (``pp_quad_big``)
* ``big_kn``   the same kernel on (K,N) codes as stored
* ``kn_mfma``  (K,N) codes transposed into (N,K) rows, then ``mfma`` (``fused=False`` only)
* ``prefill``  fp16 decode + one batched library GEMM (hipBLASLt through ``torch.matmul``)
* ``generic``  any strides: decode into a float32 workspace, then a plain GEMV kernel

Dual kernels (polar_kernels.py:14-115):

* ``dual_mfma``  matrix-core decode of the int16 (K,N) kernel layout (``pp_dual_mfma``)
* ``dual_kn``    fused row decode of (K,N) codes, 8 tokens per pass (``pp_dual_gemm``)
* ``dual_rows``  fused row decode of container (N,K) rows, 1-4 tokens (``pp_dual_gemm``)
* ``dual_nk_mfma`` matrix-core decode of container (N,K) rows (``pp_dual_nk_mfma``)
* ``prefill`` / ``generic`` as for quad.

The token boundaries are measured crossovers (graph-replayed GPU times on the reference's
4096x4096 layer and the gate / down shapes; the numbers are in the comments of each row).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, FrozenSet, Optional, Tuple, Union

INF = 1 << 62
ANY_FUSED = (None, True, False)
ANY_PLUG = (False, True)

QB_ROWS = 16          # weight rows per work item of the fused matrix-core kernel (quad_big.hip)


@dataclass(frozen=True)
class Route:
    kernel: str
    m_lo: Union[int, Callable[[int, int, bool], int]]    # int, or f(K, N, has_plug)
    m_hi: int                                             # inclusive
    plug: Tuple[bool, ...] = ANY_PLUG
    fused: Tuple[Optional[bool], ...] = ANY_FUSED
    cap: Optional[str] = None                             # a further capability the storage must have

    def lo(self, K: int, N: int, has_plug: bool) -> int:
        return self.m_lo(K, N, has_plug) if callable(self.m_lo) else self.m_lo

    def matches(self, caps: FrozenSet[str], M: int, K: int, N: int, has_plug: bool, fused) -> bool:
        return (self.kernel in caps and (self.cap is None or self.cap in caps) and has_plug in self.plug
                and fused in self.fused and self.lo(K, N, has_plug) <= M <= self.m_hi)


def kn_big_min_m(K: int, N: int, has_plug: bool) -> int:
    """(K,N) codes without plug entries: the fused matrix-core kernel from 2 tokens when N <= K,
    from 3 when N > K; the (K,N) row kernel below (graph-replayed, row kernel against fused
    kernel at 1 / 2 / 4 / 8 tokens: 4096x4096 23.3 / 29.6 / 36.6 / 45.5 against 27.6 / 27.4 /
    27.4 / 27.4 us; K x N = 11008x2048 27.7 / 34.4 / 42.2 / 53.9 against 32.2 / 32.4 / 32.5 /
    32.3; 2048x11008 25.6 / 33.9 / 41.9 / 56.3 against 38.4 / 38.4 / 40.6 / 40.7, 3 tokens 41.3
    against 39.5)."""
    return 2 if N <= K else 3


def dual_mfma_min_m(K: int, N: int, has_plug: bool) -> int:
    """int16 (K,N) codes: the matrix-core decode from 2 tokens when N <= K without plug entries
    (4096x4096 at 2 / 3 / 4 tokens 26.0 / 26.7 / 28.3 against 29.6 / 32.8 / 36.6 us for the
    row kernel, K x N = 11008x2048 30.2 / 31.5 / 32.1 against 33.8 / 37.9 / 40.6; at 1 token
    the row kernel wins, 21.8 against 25.2 us), else from 5 (2048x11008: 38.0 / 38.4 / 38.5
    against 29.6 / 34.6 / 38.1 us; with plug entries the matrix-core route moves them to its
    frame on every call)."""
    return 2 if N <= K and not has_plug else 5


# ------------------------------------------------------------------------------- quad
QUAD_ROUTES = (
    # (N,K) rows: the row kernel to 4 tokens; from 5 the matrix cores (gate 11008x2048 / down
    # 2048x11008, 0.1 % plug: 5 tokens 45.4 / 43.9 us against 66.1 / 80.0 us on the row
    # kernel, 4 tokens 43.6 / 44.7 against 40.9 / 43.9)
    Route("rows", 1, 4),
    Route("mfma", 5, 64),
    Route("rows", 5, 8),                                   # K % 32 != 0: no matrix cores
    # 65-128 tokens: the fused kernel (11008x2048 / 2048x11008, 0.1 % plug: 106-108 / 87-90
    # us against 113-115 / 114-121 us for the fp16 decode + one batched GEMM at 65-128
    # tokens; 150 / 156 against 116 / 149 at 192); above, the decode + GEMM unless fused=True
    Route("big_nk", 65, 128, fused=(None,)),
    Route("big_nk", 65, INF, fused=(True,)),
    # (K,N) codes (pack_quad_layer): the fused kernel at any size when asked for
    Route("big_kn", 1, INF, fused=(True,)),
    # the (K,N) row kernel at 1 token, and with plug entries to 8 (the fused kernel would
    # move the entries to its (N,K) frame on every call)
    Route("kn", 1, 1),
    Route("kn", 1, 8, plug=(True,)),
    # to 256 tokens (4096x4096 at 65 / 128 / 192 / 256: 55 / 58 / 63 / 68 us against 64 / 64
    # / 73 / 80 us for the fp16 decode + one batched GEMM; at 320 96 against 81)
    Route("big_kn", kn_big_min_m, 256, plug=(False,), fused=(None,)),
    Route("big_kn", 9, 256, plug=(True,), fused=(None,)),
    # fused=False on (K,N): transposed copy + batch decode (4096x4096 16 / 32 / 64 tokens 59
    # / 65 / 84 us, against 33 / 40 / 58 us on the fused kernel)
    Route("kn_mfma", 9, 64, fused=(False,)),
    Route("kn", 1, 16),                                    # two 8-token passes (K % 32 != 0)
    Route("generic", 1, 8),
    Route("prefill", 1, INF),
)


def _aligned(ptr: int, n: int) -> bool:
    return ptr % n == 0


def quad_storage(c_sk: int, c_sn: int, ptr: int, K: int, N: int, plug_n: int = 0) -> FrozenSet[str]:
    """Kernels that can read quad codes of the (K,N) view with strides (c_sk, c_sn) at device
    address ``ptr``: each kernel's layout, alignment and 32-bit offset limits, as its entry
    point checks them (quad_rows.hip quad_rows_ok, quad_kn.hip quad_kn_ok, quad_mfma.hip
    pp_quad_mfma, quad_big.hip pp_quad_big)."""
    caps = {"prefill", "generic"}
    a16 = _aligned(ptr, 16)
    nk = c_sk == 1 and c_sn >= K and c_sn % 4 == 0 and a16
    if nk and K % 4 == 0 and K > 0 and N * c_sn < (1 << 29):
        caps.add("rows")
    if nk and K % 32 == 0 and K > 0 and QB_ROWS * c_sn * 4 < (1 << 31):
        caps.add("mfma")
        if plug_n < (1 << 28):
            caps.add("big_nk")
    kn = c_sn == 1 and c_sk >= N and c_sk % 4 == 0 and N % 4 == 0 and N > 0 and K > 0 and K % 8 == 0 and a16 \
        and K < (1 << 30) and c_sk * K < (1 << 30)
    if kn:
        caps.add("kn")
        if K % 32 == 0:
            caps.add("kn_mfma")
    if c_sn == 1 and c_sk >= N and K % 32 == 0 and K > 0 and _aligned(ptr, 4) and K * c_sk * 4 < (1 << 31) \
            and plug_n < (1 << 28):
        caps.add("big_kn")
    return frozenset(caps)


def quad_route(M: int, K: int, N: int, caps: FrozenSet[str], has_plug: bool, fused=None) -> str:
    """The kernel ``quad_bitpacked`` runs (the first matching row of QUAD_ROUTES)."""
    for r in QUAD_ROUTES:
        if r.matches(caps, M, K, N, has_plug, fused):
            return r.kernel
    raise AssertionError("the prefill row matches every call")


# ------------------------------------------------------------------------------- dual
def dual_nk_mfma_min_m(K: int, N: int, has_plug: bool) -> int:
    """First token count of the container-row matrix-core decode by default: 1, or 3 when
    N > K (there the row kernel is faster at 1-2 tokens)."""
    return 3 if N > K else 1


DUAL_ROUTES = (
    Route("dual_mfma", 1, INF, fused=(True,)),
    # from 96 tokens the fp16 decode + one batched GEMM is faster (4096x4096: 52 against 66 us)
    Route("dual_mfma", dual_mfma_min_m, 64, fused=(None,)),
    # 65-128 tokens on the rows its producer/consumer form reads (no plug table, N a multiple
    # of 16 and of the group size, 16-byte rows): 4096x4096 at 65 / 128 / 192 tokens 46 / 43 /
    # 60 us against 53 / 53 / 54 us for the fp16 decode + one batched GEMM
    Route("dual_mfma", 65, 128, plug=(False,), fused=(None,), cap="dual_pc"),
    Route("dual_nk_mfma", 1, INF, fused=(True,)),
    Route("dual_kn", 1, 8),
    # container rows, no plug table, graph-replayed per Linear: 2048x2048 at 1 token 12.8
    # against 16.1 us on the row kernel, 2048x11008 25.6 against 80.2; 11008x2048 (N > K) at
    # 1-2 tokens 33.1 / 31.3 against 22.7 / 27.4 us, at 3 tokens 32.0 against 51.7; above 64
    # tokens the fp16 decode + GEMM wins on 2048x2048 (32.7 against 61.5 us at 65)
    Route("dual_nk_mfma", dual_nk_mfma_min_m, 64, fused=(None,)),
    Route("dual_rows", 1, 4),
    Route("generic", 1, 4),
    Route("prefill", 1, INF),
)


def dual_storage(c_sk: int, c_sn: int, ptr: int, K: int, N: int, layout: str, group_size: int, chunk_size: int,
                 elem_base: int, plug_n: int = 0) -> FrozenSet[str]:
    """Kernels that can read dual codes of the (K,N) view with strides (c_sk, c_sn) at device
    address ``ptr`` (dual_kn.hip dual_kn_ok, dual.hip dual_fast_ok, dual_mfma.hip
    pp_dual_mfma and pp_dual_nk_mfma)."""
    caps = {"prefill", "generic"}
    a16 = _aligned(ptr, 16)
    gs_ok = group_size >= 8 and group_size & (group_size - 1) == 0
    kn = c_sn == 1 and c_sk >= N and c_sk % 8 == 0 and N % 8 == 0 and N > 0 and K > 0 and K % 8 == 0 and a16 \
        and chunk_size == 0 and gs_ok
    if kn and K * N < (1 << 32) and 2 * c_sk * K < (1 << 31):
        caps.add("dual_kn")
    n_groups = (K * N + group_size - 1) // max(group_size, 1)
    if kn and layout == "i16" and K % 32 == 0 and K * c_sk * 2 < (1 << 31) and n_groups * 2 < (1 << 31) \
            and plug_n < (1 << 29):
        caps.add("dual_mfma")
        # rows of 8 codes per 16-byte load (pp_dual_mfma's transposing loads and its
        # producer/consumer form): dual_mfma.hip's gcols condition
        if plug_n == 0 and N % 16 == 0 and N % group_size == 0 and c_sk % 8 == 0 and a16:
            caps.add("dual_pc")
    if c_sk == 1 and c_sn % 8 == 0 and c_sn >= K and K % 8 == 0 and K > 0 and a16 and chunk_size > 0 \
            and chunk_size % 8 == 0 and gs_ok and elem_base % 8 == 0:
        caps.add("dual_rows")
        if K % 32 == 0 and 32 <= chunk_size < (1 << 30) and 32 * c_sn < (1 << 31) and N < (1 << 30) \
                and plug_n < (1 << 29):
            caps.add("dual_nk_mfma")
    return frozenset(caps)


def dual_route(M: int, K: int, N: int, caps: FrozenSet[str], has_plug: bool, fused=None) -> str:
    """The kernel ``polar_dual_bitpacked`` runs (the first matching row of DUAL_ROUTES)."""
    for r in DUAL_ROUTES:
        if r.matches(caps, M, K, N, has_plug, fused):
            return r.kernel
    raise AssertionError("the prefill row matches every call")
