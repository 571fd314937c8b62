"""Packed Linear layers: a model's Linear weights served straight from a quad / dual
stream instead of restored to dense fp16.

The reference restores every Linear of a model from its unpacked float32 dump
(``replace_model_weights``, polar_packer.py:285-316: walk the layer map of
``collect_weights``, polar_main.py:25-50, in stream order and overwrite
``module.weight``).  Here the same walk swaps each ``nn.Linear`` for a
:class:`QuadPackedLinear` / :class:`DualPackedLinear` that keeps the codes in HBM
and decodes them inside the matmul (``quad_bitpacked`` / ``polar_dual_bitpacked``
with the stream's plug table), so one pass over a Linear's codes serves all packed
models at once, and a model's forward is a real dependent decode step.

Projections must lie inside the coded stream (positions < n); rows that reach a
model's FP16 tails are served by the whole-step streams (:mod:`.stream`).
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import polar_kernels as pk
from . import quad_kernels as qk
from .container import DualPackDevice, QuadPackDevice


class _PackedLinear(torch.nn.Module):
    models = 0

    def __init__(self, N: int, K: int, pos0: int, n: int, model: Optional[int], bias: Optional[torch.Tensor]):
        super().__init__()
        if pos0 < 0 or pos0 + N * K > n:
            raise ValueError(f"projection [{pos0}, {pos0 + N * K}) is not inside the coded stream (n = {n})")
        if model is not None and not 0 <= model < self.models:
            raise ValueError(f"model index must be in 0..{self.models - 1}")
        self.in_features, self.out_features, self.pos0, self.model = int(K), int(N), int(pos0), model
        self.bias = torch.nn.Parameter(bias.detach().to(torch.float16), requires_grad=False) if bias is not None \
            else None

    def _all(self, x2: torch.Tensor):
        raise NotImplementedError

    def forward(self, x: torch.Tensor):
        """``x`` (..., K) fp16.  With ``model`` set: that model's (..., N) output, like the
        ``nn.Linear`` it replaces; otherwise a tuple with every model's output."""
        lead = x.shape[:-1]
        if x.shape[-1] != self.in_features:
            raise ValueError(f"expected (..., {self.in_features}) input, got {tuple(x.shape)}")
        outs = self._all(x.reshape(-1, self.in_features).to(torch.float16))
        outs = [o.reshape(*lead, self.out_features) for o in outs]
        if self.bias is not None:
            outs = [o + self.bias for o in outs]
        return outs[self.model] if self.model is not None else tuple(outs)


class QuadPackedLinear(_PackedLinear):
    """The (N, K) block at stream position ``pos0`` of a quad stream, 4 models."""
    models = 4

    def __init__(self, pack: QuadPackDevice, N: int, K: int, pos0: int, model: Optional[int] = None,
                 bias: Optional[torch.Tensor] = None):
        super().__init__(N, K, pos0, pack.n, model, bias)
        self.pack = pack
        self.codes = pack.codes[pos0:pos0 + N * K].reshape(N, K).t()     # (K, N) view of the (N, K) rows
        self.luts = qk.header_luts(pack.r_max, device=pack.codes.device)
        self.scales = list(pack.s)

    def _all(self, x2):
        return qk.quad_bitpacked(x2, self.codes, self.luts, self.scales,
                                 plug=(self.pack.plug_idx, self.pack.plug_vals), elem_base=self.pos0)


class DualPackedLinear(_PackedLinear):
    """The (N, K) block at stream position ``pos0`` of a dual stream, 2 models."""
    models = 2

    def __init__(self, pack: DualPackDevice, N: int, K: int, pos0: int, model: Optional[int] = None,
                 bias: Optional[torch.Tensor] = None):
        super().__init__(N, K, pos0, pack.n_codes, model, bias)
        self.pack = pack
        self.codes = pack.codes[pos0:pos0 + N * K].reshape(N, K).t()
        self.luts = pk.header_luts(pack.amp_bits, pack.phase_bits, pack.mu, device=pack.codes.device)

    def _all(self, x2):
        p = self.pack
        plug = (p.plug_idx, p.plug_val)
        return pk.polar_dual_bitpacked(x2, self.codes, p.scales, *self.luts, num_phases=1 << p.phase_bits,
                                       group_size=p.group_size, plug=plug, elem_base=self.pos0, layout=p.layout,
                                       chunk_size=p.chunk_size)


def _module_at(model: torch.nn.Module, name: str):
    parent, leaf = None, model
    for part in name.split("."):
        parent = leaf
        leaf = leaf[int(part)] if part.isdigit() else getattr(leaf, part)
    return parent, leaf


def replace_model_weights(model: torch.nn.Module, pack, layer_info: Sequence[dict], model_index: int = 0) -> int:
    """Swap the Linear layers named in ``layer_info`` (the reference's layer map: dicts with
    ``name``, ``shape`` = [N, K], ``numel``, in stream order) for packed layers serving
    model ``model_index`` of ``pack``.  Entries that are not an ``nn.Linear`` of that size
    are skipped but still advance the stream position, as polar_packer.py:297-305 does.
    Returns the number of layers replaced."""
    cls = QuadPackedLinear if isinstance(pack, QuadPackDevice) else DualPackedLinear
    pos = 0
    replaced = 0
    for info in layer_info:
        numel = int(info["numel"])
        parent, module = _module_at(model, info["name"])
        if isinstance(module, torch.nn.Linear) and module.weight.numel() == numel:
            N, K = (int(v) for v in info["shape"])
            new = cls(pack, N, K, pos, model=model_index, bias=module.bias)
            leaf = info["name"].split(".")[-1]
            if leaf.isdigit():
                parent[int(leaf)] = new
            else:
                setattr(parent, leaf, new)
            replaced += 1
        pos += numel
    return replaced
