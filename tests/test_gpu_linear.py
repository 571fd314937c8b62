"""GPU parity of the packed Linear layers (a model's Linears served from a quad / dual
stream, polar_packer.py:285-316's walk) on a dependent two-layer step."""
import copy

import numpy as np
import pytest
import torch

import gen
from oracle import dualpack as odp
from oracle import quadpack as oqp
from parity import assert_gemv_close, fp16_weight_bound
from polar_pack_amd.container import DualPackFile, QuadPackFile
from polar_pack_amd import polar_kernels as pk
from polar_pack_amd.linear import DualPackedLinear, QuadPackedLinear, replace_model_weights
from refs import route_class

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# the reference's layer map (polar_main.py:33-43): a Linear, an activation, a Linear with bias
LAYERS = [{"name": "0", "shape": [96, 256], "numel": 96 * 256},
          {"name": "2", "shape": [40, 96], "numel": 40 * 96}]


def mlp():
    torch.manual_seed(0)
    m = torch.nn.Sequential(torch.nn.Linear(256, 96, bias=False), torch.nn.SiLU(), torch.nn.Linear(96, 40))
    return m.to(DEV).to(torch.float16)


def run_and_check(model, weights, x_np, fp16):
    """Layer by layer: each packed layer against the oracle's float64 product on the
    input it actually received (the previous layer's fp16 output).  The routes that feed
    fp16 weights to the dot product, as the reference's kernels do (``fp16``: one flag per
    layer, from the operator's routing table), are held to the fp16-weight bound."""
    flags = iter(fp16)

    def bound(a, w):
        return fp16_weight_bound(a, w.T) if next(flags) else None
    x = torch.from_numpy(x_np).to(DEV)
    h1 = model[0](x)
    assert_gemv_close(h1.float().cpu().numpy(), x_np.astype(np.float64) @ weights[0].T, "layer 0",
                      bound=bound(x_np, weights[0]))
    a1 = model[1](h1)
    y = model[2](a1)
    a1_np = a1.float().cpu().numpy().astype(np.float64)
    prod = a1_np @ weights[1].T
    ref = prod + model[2].bias.float().cpu().numpy()
    # the product is rounded to fp16 before the bias add, which rounds once more: half an
    # fp16 ulp of each (the product can exceed |y| where the bias cancels it)
    extra = 2.0 ** -11 * (np.abs(prod) + np.abs(ref))
    b = bound(a1_np, weights[1])
    assert_gemv_close(y.float().cpu().numpy(), ref, "layer 2", bound=extra if b is None else extra + b)
    assert y.shape == (x_np.shape[0], 40) and y.dtype == torch.float16


@pytest.mark.parametrize("M", [1, 3, 20])
def test_quad_packed_mlp_every_model(M):
    n = sum(l["numel"] for l in LAYERS)
    qp = oqp.pack_quad(gen.correlated_models(4, [n] * 4), threshold=0.01)
    pack = QuadPackFile(n=qp.n, s=qp.s, r_max=qp.r_max, codes=qp.codes, plug_idx=qp.plug_idx,
                        plug_vals=qp.plug_vals).to_device(DEV)
    W = oqp.unpack_quad_f64(qp, 0, n)
    x_np = np.random.default_rng(M).standard_normal((M, 256)).astype(np.float16)
    base = mlp()
    for k in range(4):
        model = copy.deepcopy(base)
        assert replace_model_weights(model, pack, LAYERS, model_index=k) == 2
        assert isinstance(model[0], QuadPackedLinear) and isinstance(model[2], QuadPackedLinear)
        weights = [W[k][:96 * 256].reshape(96, 256), W[k][96 * 256:].reshape(40, 96)]
        run_and_check(model, weights, x_np, (M > 8, M > 8))
    # all four models from one pass: the per-model layers' outputs (split-K sums may
    # meet in another order between launches, so equal to the GEMV tolerance, not bitwise)
    both = QuadPackedLinear(pack, 96, 256, 0)
    x = torch.from_numpy(x_np).to(DEV)
    outs = both(x)
    assert len(outs) == 4
    for k in range(4):
        single = QuadPackedLinear(pack, 96, 256, 0, model=k)(x)
        assert_gemv_close(outs[k].float().cpu().numpy(), single.float().cpu().numpy(), f"model {k}")


@pytest.mark.parametrize("layout", ["u16be", "i16"])
@pytest.mark.parametrize("M", [1, 4, 9])
def test_dual_packed_mlp(layout, M):
    n = sum(l["numel"] for l in LAYERS)
    w1, w2 = gen.correlated_models(6, [n, n], delta_growth=False)
    dp = odp.pack_dual(w1, w2, odp.DualConfig(plug_cap=0.02, chunk_size=10_000))
    f = DualPackFile(n_pairs=dp.n_pairs, n1=dp.n1, n2=dp.n2, codes_be=dp.codes_be, scales=dp.scales,
                     plug_idx=dp.plug_idx, plug_val=dp.plug_val, amp_bits=dp.amp_bits, phase_bits=dp.phase_bits,
                     mu=dp.mu, group_size=dp.group_size, chunk_size=dp.chunk_size)
    pack = f.to_device(DEV)
    if layout == "i16":
        code = odp.from_be_bytes(dp.codes_be).astype(np.uint16)
        pack.codes = torch.from_numpy((code ^ np.uint16(0x8000)).view(np.int16)).to(DEV)
        pack.layout = "i16"
    d = odp.decode_pairs_f64(dp, 0, n)
    x_np = np.random.default_rng(M).standard_normal((M, 256)).astype(np.float16)
    base = mlp()
    for k in range(2):
        model = copy.deepcopy(base)
        assert replace_model_weights(model, pack, LAYERS, model_index=k) == 2
        assert isinstance(model[0], DualPackedLinear)
        weights = [d[k][:96 * 256].reshape(96, 256), d[k][96 * 256:].reshape(40, 96)]
        fp16 = [route_class(pk.dual_call_route(layer.codes, M, layout=pack.layout, group_size=pack.group_size,
                                               chunk_size=pack.chunk_size, elem_base=layer.pos0,
                                               plug_n=pack.plug_idx.numel())) != "fused"
                for layer in (model[0], model[2])]
        run_and_check(model, weights, x_np, fp16)


def test_projection_outside_the_coded_stream_is_rejected():
    qp = oqp.pack_quad(gen.correlated_models(4, [4096] * 4), threshold=0.01)
    pack = QuadPackFile(n=qp.n, s=qp.s, r_max=qp.r_max, codes=qp.codes, plug_idx=qp.plug_idx,
                        plug_vals=qp.plug_vals).to_device(DEV)
    with pytest.raises(ValueError, match="inside the coded stream"):
        QuadPackedLinear(pack, 64, 64, 1)
