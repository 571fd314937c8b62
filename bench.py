#!/usr/bin/env python3
"""Batch-1 decode step over a quad-pack Qwen2.5-3B-shaped Linear stream on one MI355X.

Default workload (one "step"): 36 layers x {q, o 2048x2048; k, v 256x2048; gate,
up 11008x2048; down 2048x11008} projections, 4 models packed in one .quadpack v2
stream (2,774,532,096 uint32 tuples, top 0.1% of tuples by norm in the plug table),
one fp16 N(0,1) activation vector per projection, 4 fp16 outputs per projection,
decoded by one pp_quad_stream launch.  Weights are synthetic: per layer-seeded
Student-t(df=5) base scaled to std 0.02, model i = base + N(0, 0.002 i), fp16.

Prints ONE JSON line: achieved GB/s of algorithmic bytes (value), ms per step,
roofline (HIP-event kernel time vs 8 TB/s HBM) and the CPU baseline (the CPU
oracle's numpy unpack + torch CPU matmul on a bounded sample, extrapolated).

    python bench.py [--steps 30] [--warmup 10] [--layers 36] [--no-cpu]

Other workloads (``--workload``), one JSON line each:

* ``dual3b``     -- dual-pack 3B-shaped stream, Student-t(df=3) base, model 2 = base +
                    N(0, 0.004) truncated to 95% of the stream, top 1% of pairs in the plug
                    table (largest squared amplitude error per 50M-pair chunk); model 1's
                    last 5% are fp16 tails; one pp_dual_stream launch per step;
* ``dual3b-pad`` -- the same weights in the .dualpack format itself (model 2 zero-padded);
* ``dual2048``   -- one dual 2048x2048 Linear, 2 models, plug 0.1% by norm;
* ``quadgate``   -- one quad 11008x2048 Linear (gate_proj), 4 models, plug 0.1% by norm;
* ``sweep``      -- quad gate_proj 11008x2048 and down_proj 2048x11008 at 1, 4, 16, 64
                    tokens per model (one line per shape and batch);
* ``refbench``   -- the reference's own kernel benchmarks (quad_kernels.py:160-200,
                    polar_kernels.py:153-184): 4096x4096 N(0,1) weights packed by the drop-in
                    pack_quad_layer / quantize_polar_bitpacked, the drop-in operators called
                    as the reference calls them at M = 1, 8, 32, 128, 1024 tokens, beside
                    torch's fp16 matmul of the unpacked weights (one line per operator);
* ``quadbig``    -- the fused large-batch quad kernel (quad_bitpacked(fused=True)) on the
                    refbench layer at ``--big-tokens`` tokens, against the matrix cores'
                    fp16 roofline (one line per batch size);
* ``dualmfma``   -- the dual matrix-core decode (polar_dual_bitpacked(fused=True)) on the
                    refbench dual layer at ``--dual-tokens`` tokens, the same roofline;
* ``dualrows``   -- polar_dual_bitpacked on .dualpack (N,K) rows (2048x2048, gate, down) at
                    ``--rows-tokens`` tokens: the default route against fused=False.

Single-Linear workloads rotate enough copies of the packed weights (>= 512 MB in total)
that no launch finds its codes in the 256 MB last-level cache, and time a HIP graph of
one launch per copy, so the figure is device time without host launch gaps.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from polar_pack_amd import polar_kernels as pk  # noqa: E402
from polar_pack_amd import quad_kernels as qk  # noqa: E402
from polar_pack_amd import routes  # noqa: E402
from polar_pack_amd.packer import pack_dual_device, pack_quad_device  # noqa: E402
from polar_pack_amd.stream import DualStream, QuadBatch, QuadStream  # noqa: E402

METRIC = "achieved HBM GB/s (% of peak) + ms per quad-pack 3B decode step, batch 1"
PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2500.0
LAYER = [("q_proj", 2048, 2048), ("k_proj", 256, 2048), ("v_proj", 256, 2048), ("o_proj", 2048, 2048),
         ("gate_proj", 11008, 2048), ("up_proj", 11008, 2048), ("down_proj", 2048, 11008)]
PMC_SUMMARY = {"quad3b": os.path.join(ROOT, "profiles", "quad_stream_3b_pmc.md"),
               "dual3b": os.path.join(ROOT, "profiles", "dual_stream_3b_pmc.md"),
               "dual2048": os.path.join(ROOT, "profiles", "dual_linear_2048_direct.md"),
               "quadgate": os.path.join(ROOT, "profiles", "quad_linear_gate_direct.md")}
# The sources of the kernels each summary measured: a summary's traffic is used only while
# their digest equals the one it records (kernel_sources_sha256), so a kernel changed after
# its profile reports traffic null until the profile is taken again.
_QUAD_ROWS_SRC = ["quad_rows.hip", "quad_rows.h", "quad_lds.h", "rows_common.h", "pp_common.h"]
_DUAL_ROWS_SRC = ["dual_rows.hip", "dual_lds.h", "rows_common.h", "pp_common.h"]
PMC_SOURCES = {"quad3b": _QUAD_ROWS_SRC, "quadgate": _QUAD_ROWS_SRC, "dual3b": _DUAL_ROWS_SRC,
               "dual2048": _DUAL_ROWS_SRC}
MALL_BYTES = 512 << 20


def seed_of(config, layer, proj):
    return 20260000 + 1000 * config + 10 * layer + proj


def student_t(n, df, std, g, dev):
    """Student-t(df) scaled to standard deviation ``std`` (variance of t_df is df/(df-2))."""
    z = torch.randn(n, generator=g, device=dev)
    chi = torch.zeros_like(z)
    for _ in range(df):
        chi += torch.randn(n, generator=g, device=dev) ** 2
    return z / torch.sqrt(chi / df) * (std / math.sqrt(df / (df - 2.0)))


def synth_models(n_layers, dev):
    """4 correlated fp16 models, flat (N,K) row-major per projection, stream order."""
    models = [[], [], [], []]
    for layer in range(n_layers):
        for p, (_, n, k) in enumerate(LAYER):
            g = torch.Generator(device=dev).manual_seed(seed_of(3, layer, p))
            w0 = student_t(n * k, 5, 0.02, g, dev)
            for m in range(4):
                d = torch.randn(n * k, generator=g, device=dev) * (0.002 * (m + 1))
                models[m].append((w0 + d).to(torch.float16))
                del d
            del w0
    return models


def synth_dual_stream(shapes, dev, truncate=0.05):
    """Flat fp16 model streams: model 1 = Student-t(3) base (std 0.02), model 2 = base +
    N(0, 0.004), model 2 truncated to floor((1 - truncate) * n1) weights."""
    n1 = sum(n * k for n, k in shapes)
    n2 = int(math.floor((1.0 - truncate) * n1))
    w1 = torch.empty(n1, dtype=torch.float16, device=dev)
    w2 = torch.empty(n2, dtype=torch.float16, device=dev)
    pos = 0
    for i, (n, k) in enumerate(shapes):
        layer, p = divmod(i, len(LAYER))
        g = torch.Generator(device=dev).manual_seed(seed_of(5, layer, p))
        w0 = student_t(n * k, 3, 0.02, g, dev)
        w1[pos:pos + n * k] = w0.to(torch.float16)
        d = torch.randn(n * k, generator=g, device=dev) * 0.004
        hi = min(pos + n * k, n2)
        if hi > pos:
            w2[pos:hi] = (w0 + d)[:hi - pos].to(torch.float16)
        del w0, d
        pos += n * k
    return w1, w2


def stream_shapes(layers):
    """(N, K) of every projection of the 3B-shaped stream, in stream order."""
    return [(n, k) for _ in range(layers) for (_, n, k) in LAYER]


def quad3b_pack(layers, dev):
    """The quad 3B-shaped workload's stream: synthesized weights packed on the device, plug
    table = top 0.1% of tuples by norm."""
    models = synth_models(layers, dev)
    pack = pack_quad_device(models, plug_cap=0.001, select="norm")
    del models
    torch.cuda.empty_cache()
    return pack


def dual3b_pack(layers, dev, tails):
    """The dual 3B-shaped heavy-tail workload's stream (model 2 truncated by 5%): top 1% of
    pairs by squared amplitude error per chunk in the plug table; ``tails`` keeps model 1's
    last weights as fp16 tails, otherwise the shorter model is zero-padded."""
    w1, w2 = synth_dual_stream(stream_shapes(layers), dev)
    pack = pack_dual_device(w1, w2, plug_cap=0.01, select="ref", tails=tails)
    del w1, w2
    torch.cuda.empty_cache()
    return pack


def dual2048_pack(dev):
    """The dual 2048x2048 Linear: Student-t(5) base with std 0.02, each model base + N(0,
    0.002), plug table = top 0.1% of pairs by amplitude."""
    N = K = 2048
    g = torch.Generator(device=dev).manual_seed(seed_of(1, 0, 0))
    w0 = student_t(N * K, 5, 0.02, g, dev)
    w1 = (w0 + torch.randn(N * K, generator=g, device=dev) * 0.002).to(torch.float16)
    w2 = (w0 + torch.randn(N * K, generator=g, device=dev) * 0.002).to(torch.float16)
    return pack_dual_device(w1, w2, plug_cap=0.001, select="norm")


def check_close(got, ref, what, rtol=1e-3, floor=1e-5):
    """|got - ref| <= rtol |ref| + floor max|ref| + 2^-25 per element (fp16 outputs)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    lim = rtol * np.abs(ref) + floor * np.abs(ref).max() + 2.0 ** -25
    if not np.all(err <= lim):
        raise SystemExit(f"parity check failed on {what}: max |d| {err.max():.3e}, max |ref| {np.abs(ref).max():.3e}")
    return float(err.max() / max(np.abs(ref).max(), 1e-300))


def cpu_baseline(pack, shapes, sample_tuples, xs=None, outs=None):
    """The CPU oracle's unpack (numpy float64, single thread) + torch CPU float32 matmul,
    on the first projections of the stream up to ~sample_tuples, extrapolated to the step.
    With the GPU run's activations ``xs`` and outputs ``outs``, the CPU products are also
    the check of those projections' GPU outputs (rel 1e-3)."""
    from oracle import quadpack as oqp
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    take, tuples = [], 0
    for n, k in shapes:
        if tuples + n * k > sample_tuples and take:
            break
        take.append((n, k))
        tuples += n * k
    codes = pack.codes[:tuples].cpu().view(torch.int32).numpy().view(np.uint32)
    plug = pack.plug_host()
    hi = int(np.searchsorted(plug, tuples))
    qp = oqp.QuadPack(n=tuples, s=pack.s, r_max=pack.r_max, codes=codes, plug_idx=plug[:hi].copy(),
                      plug_vals=pack.plug_vals[:hi].cpu().numpy())
    rng = np.random.default_rng(0)
    t_unpack = t_mm = 0.0
    pos = 0
    worst = 0.0
    for p, (n, k) in enumerate(take):
        sub = oqp.QuadPack(n=n * k, s=qp.s, r_max=qp.r_max, codes=qp.codes[pos:pos + n * k],
                           plug_idx=(qp.plug_idx[(qp.plug_idx >= pos) & (qp.plug_idx < pos + n * k)] - pos).astype(np.uint32),
                           plug_vals=qp.plug_vals[(qp.plug_idx >= pos) & (qp.plug_idx < pos + n * k)])
        t0 = time.perf_counter()
        ws = oqp.unpack_quad(sub)
        t1 = time.perf_counter()
        x = xs[p].float() if xs is not None else torch.from_numpy(rng.standard_normal((1, k)).astype(np.float32))
        ys = [x @ torch.from_numpy(w.reshape(n, k)).t() for w in ws]
        t2 = time.perf_counter()
        t_unpack += t1 - t0
        t_mm += t2 - t1
        if outs is not None:
            for m in range(4):
                worst = max(worst, check_close(outs[p][m].float().numpy(), ys[m].numpy(), f"projection {p} model {m}"))
        pos += n * k
        del ws, ys
    total_tuples = sum(n * k for n, k in shapes)
    scale = total_tuples / tuples
    return {"unpack_s": t_unpack, "matmul_s": t_mm, "sample_tuples": tuples, "scale": scale,
            "step_s": (t_unpack + t_mm) * scale, "threads": threads, "checked": len(take) if outs else 0,
            "worst_normwise": worst}


def cpu_baseline_dual(pack, shapes, sample_pairs, xs=None, outs=None):
    """The CPU oracle's dual unpack (numpy float64, single thread) + torch CPU float32 matmul
    on the first projections of the stream up to ~sample_pairs, extrapolated to the step;
    with the GPU run's activations and outputs, also the check of those projections."""
    from oracle import dualpack as odp
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    take, pairs = [], 0
    for n, k in shapes:
        if pairs + n * k > sample_pairs and take:
            break
        take.append((n, k))
        pairs += n * k
    pairs = min(pairs, pack.n_codes)
    be = pack.codes[:pairs].cpu().numpy().view(np.uint16)
    if pack.layout == "i16":
        be = (be ^ np.uint16(0x8000)).byteswap()
    plug = pack.plug_host()
    hi = int(np.searchsorted(plug, pairs))
    ng = odp.n_groups_for(pairs, pack.chunk_size, pack.group_size)
    dp = odp.DualPack(n_pairs=pairs, n1=pairs, n2=pairs, codes_be=be.view(np.uint8).copy(),
                      scales=pack.scales[:ng].cpu().numpy(), plug_idx=plug[:hi].copy(),
                      plug_val=pack.plug_val[:hi].cpu().numpy(), amp_bits=pack.amp_bits,
                      phase_bits=pack.phase_bits, mu=pack.mu, group_size=pack.group_size,
                      chunk_size=pack.chunk_size)
    rng = np.random.default_rng(0)
    t_unpack = t_mm = 0.0
    pos = 0
    worst = 0.0
    for p, (n, k) in enumerate(take):
        t0 = time.perf_counter()
        w1, w2 = odp.decode_pairs_f64(dp, pos, pos + n * k)
        w1, w2 = w1.astype(np.float32), w2.astype(np.float32)
        t1 = time.perf_counter()
        x = xs[p].float() if xs is not None else torch.from_numpy(rng.standard_normal((1, k)).astype(np.float32))
        ys = [x @ torch.from_numpy(w.reshape(n, k)).t() for w in (w1, w2)]
        t2 = time.perf_counter()
        t_unpack += t1 - t0
        t_mm += t2 - t1
        if outs is not None:
            for m in range(2):
                worst = max(worst, check_close(outs[p][m].float().numpy(), ys[m].numpy(), f"projection {p} model {m}"))
        pos += n * k
        del w1, w2, ys
    total = sum(n * k for n, k in shapes)
    scale = total / pairs
    return {"unpack_s": t_unpack, "matmul_s": t_mm, "sample": pairs, "scale": scale,
            "step_s": (t_unpack + t_mm) * scale, "threads": threads, "checked": len(take) if outs else 0,
            "worst_normwise": worst}


def kernel_sources_sha256(names):
    """sha256 over the named files of polar_pack_amd/csrc, in the order given."""
    import hashlib
    h = hashlib.sha256()
    for n in names:
        with open(os.path.join(ROOT, "polar_pack_amd", "csrc", n), "rb") as f:
            h.update(n.encode() + b"\0" + f.read())
    return h.hexdigest()


def read_pmc_traffic(path, sources=None):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE), if
    committed and, when ``sources`` names the kernel's files, taken of those sources as they
    are now (the summary's kernel_sources_sha256); None otherwise."""
    try:
        text = open(path).read()
    except (OSError, TypeError):
        return None
    m = re.search(r"traffic_bytes_per_launch\s*[=:]\s*([0-9.eE+]+)", text)
    if not m:
        return None
    if sources is not None:
        h = re.search(r"kernel_sources_sha256\s*[=:]\s*([0-9a-f]{64})", text)
        if not h or h.group(1) != kernel_sources_sha256(sources):
            return None
    return float(m.group(1))


def pmc_traffic(workload):
    return read_pmc_traffic(PMC_SUMMARY[workload], PMC_SOURCES[workload])


def time_events(launch, steps, warmup):
    """HIP-event duration of each of ``steps`` launches on torch's current stream (the
    stream the decode kernels are launched on), after ``warmup`` untimed launches."""
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        launch()
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    return [s.elapsed_time(e) for s, e in zip(starts, ends)], wall


def line(metric, achieved, ms, args, dtype, config, traffic=None, cpu=None, extra=None, traffic_profile=None,
         bound="hbm"):
    peak, unit = (PEAK_HBM_GBS, "GB/s") if bound == "hbm" else (PEAK_FP16_TFLOPS, "TFLOP/s")
    out = {
        "metric": metric, "value": round(achieved, 2), "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": config,
        "roofline": {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": traffic},
        "cpu_baseline": cpu,
    }
    if traffic is not None and traffic_profile:
        out["roofline"]["traffic_profile"] = os.path.relpath(traffic_profile, ROOT)
    if extra:
        out.update(extra)
    print(json.dumps(out), flush=True)


# ---------------------------------------------------------------- 3B-shaped streams

def run_quad3b(args, dev, log):
    shapes = stream_shapes(args.layers)
    t0 = time.time()
    pack = quad3b_pack(args.layers, dev)
    torch.cuda.synchronize()
    log(f"[bench] synthesized and packed: n={pack.n} plug={pack.plug_idx.numel()} r_max={pack.r_max:.4f} in "
        f"{time.time() - t0:.1f}s")

    st = QuadStream(pack, shapes, M=1)
    xs, outs = st.make_buffers()
    g = torch.Generator(device=dev).manual_seed(7)
    for x in xs:
        x.copy_(torch.randn(x.shape, generator=g, device=dev).to(torch.float16))
    st.bind(xs, outs)
    log(f"[bench] plan: {st.n_segs} segments, {st.n_tail} tail items, {st.n_waves} waves")

    # sanity: a k_proj and a down_proj of the stream against another kernel's decode (the
    # element-wise quad_dequant) times torch's float32 matmul; the CPU baseline below checks
    # layer 0 against the oracle
    st()
    torch.cuda.synchronize()
    first = [[o.cpu() for o in outs[p]] for p in range(len(LAYER))]
    luts = qk.header_luts(pack.r_max, device=dev)
    for p in (1, 6):
        n, k = shapes[p]
        pos = int(st.pos0[p])
        w = qk.quad_dequant(pack.codes[pos:pos + n * k].reshape(n, k).t(), luts, list(pack.s),
                            plug=(pack.plug_idx, pack.plug_vals), elem_base=pos)
        for m in range(4):
            check_close(outs[p][m].float().cpu().numpy(), (xs[p].float() @ w[m]).cpu().numpy(),
                        f"projection {p} model {m} vs the element-wise decode")
        del w

    per, wall = time_events(st, args.steps, args.warmup)
    ms = float(np.mean(per))
    algo = st.algorithmic_bytes()
    achieved = algo / (ms * 1e-3) / 1e9
    log(f"[bench] step: mean {ms:.4f} ms, median {np.median(per):.4f}, min {min(per):.4f}, wall/step "
        f"{wall / args.steps * 1e3:.4f} ms; {algo / 1e9:.4f} GB algorithmic -> {achieved:.1f} GB/s")

    cpu = None
    if not args.no_cpu:
        c = cpu_baseline(pack, shapes, args.cpu_sample_tuples, xs=[x.cpu() for x in xs[:len(first)]], outs=first)
        log(f"[bench] cpu baseline: unpack {c['unpack_s']:.2f}s + matmul {c['matmul_s']:.2f}s on "
            f"{c['sample_tuples']} tuples -> {c['step_s']:.2f}s per step (x{c['scale']:.1f}); GPU outputs of "
            f"{c['checked']} projections match it (normwise {c['worst_normwise']:.1e})")
        cpu = {"value": algo / c["step_s"] / 1e9, "unit": "GB/s", "cores": c["threads"], "kind": "port",
               "sample": (f"first {c['sample_tuples']} tuples of the stream ({c['sample_tuples'] / pack.n:.2%}): "
                          f"numpy float64 unpack_quad restatement (1 thread) {c['unpack_s']:.2f}s + torch CPU "
                          f"float32 x@W^T x4 ({c['threads']} threads) {c['matmul_s']:.2f}s, extrapolated x"
                          f"{c['scale']:.1f} to {c['step_s']:.1f}s per step; the GPU outputs of those "
                          f"{c['checked']} projections match it within rel 1e-3")}

    line(METRIC, achieved, ms, args, "fp32",
         {"workload": "quad-pack Qwen2.5-3B-shaped Linear stream, batch-1 decode step",
          "layers": args.layers, "projections": len(shapes), "models": 4, "batch": 1,
          "tuples": int(pack.n), "plug_entries": int(pack.plug_idx.numel()),
          "algorithmic_bytes": int(algo), "pct_of_peak": round(100 * achieved / PEAK_HBM_GBS, 2)},
         traffic=pmc_traffic("quad3b"), cpu=cpu, traffic_profile=PMC_SUMMARY["quad3b"])


def run_dual3b(args, dev, log, tails):
    shapes = stream_shapes(args.layers)
    t0 = time.time()
    pack = dual3b_pack(args.layers, dev, tails)
    torch.cuda.synchronize()
    log(f"[bench] synthesized and packed: {pack.n_codes} pairs, plug {pack.plug_idx.numel()}, tails "
        f"{pack.tail_lengths} in {time.time() - t0:.1f}s")

    st = DualStream(pack, shapes, M=1)
    xs, outs = st.make_buffers()
    g = torch.Generator(device=dev).manual_seed(7)
    for x in xs:
        x.copy_(torch.randn(x.shape, generator=g, device=dev).to(torch.float16))
    st.bind(xs, outs)
    log(f"[bench] plan: {st.n_segs} segments, {st.n_tail} tail items, {st.n_waves} waves, "
        f"{st.plug_windows} plug window(s) per step")

    # sanity: a k_proj against the single-Linear operator; the last down_proj's rows that lie
    # wholly in the fp16 tail against torch (model 2 has no weights there: 0); the CPU
    # baseline below checks layer 0 against the oracle
    st()
    torch.cuda.synchronize()
    first = [[o.cpu() for o in outs[p]] for p in range(len(LAYER))]
    amp, cos, sin = pk.header_luts(pack.amp_bits, pack.phase_bits, pack.mu, device=dev)
    n, k = shapes[1]
    pos = int(st.pos0[1])
    single = pk.polar_dual_bitpacked(xs[1], pack.codes[pos:pos + n * k].reshape(n, k).t(), pack.scales, amp, cos,
                                     sin, plug=(pack.plug_idx, pack.plug_val), elem_base=pos, layout=pack.layout,
                                     chunk_size=pack.chunk_size)
    checks = [(outs[1][m].float(), single[m].float(), f"k_proj model {m}") for m in range(2)]
    if tails:
        p = len(shapes) - 1
        n, k = shapes[p]
        r0 = max(0, -(-(pack.n_codes - int(st.pos0[p])) // k))     # first row wholly in the tail
        t0_ = int(st.pos0[p]) + r0 * k - pack.n_codes
        wt = pack.tails[0][t0_:t0_ + (n - r0) * k].float().reshape(n - r0, k)
        ref1 = xs[p].float() @ wt.t()
        checks.append((outs[p][0][:, r0:].float(), ref1, "tail rows model 1"))
        checks.append((outs[p][1][:, r0:].float(), torch.zeros_like(ref1), "tail rows model 2"))
    for got, ref, what in checks:
        d = (got - ref).abs().max().item()
        scale = max(ref.abs().max().item(), 1e-6)
        if not d <= 2e-3 * scale:
            raise SystemExit(f"dual stream sanity check failed on {what}: {d} vs {scale}")

    per, wall = time_events(st, args.steps, args.warmup)
    ms = float(np.mean(per))
    algo = st.algorithmic_bytes()
    achieved = algo / (ms * 1e-3) / 1e9
    log(f"[bench] step: mean {ms:.4f} ms, median {np.median(per):.4f}, min {min(per):.4f}, wall/step "
        f"{wall / args.steps * 1e3:.4f} ms; {algo / 1e9:.4f} GB algorithmic -> {achieved:.1f} GB/s")

    cpu = None
    if not args.no_cpu:
        c = cpu_baseline_dual(pack, shapes, args.cpu_sample_tuples, xs=[x.cpu() for x in xs[:len(first)]],
                              outs=first)
        log(f"[bench] cpu baseline: unpack {c['unpack_s']:.2f}s + matmul {c['matmul_s']:.2f}s on "
            f"{c['sample']} pairs -> {c['step_s']:.2f}s per step (x{c['scale']:.1f}); GPU outputs of "
            f"{c['checked']} projections match it (normwise {c['worst_normwise']:.1e})")
        cpu = {"value": algo / c["step_s"] / 1e9, "unit": "GB/s", "cores": c["threads"], "kind": "port",
               "sample": (f"first {c['sample']} pairs of the stream: numpy float64 unpack_dual restatement "
                          f"(1 thread) {c['unpack_s']:.2f}s + torch CPU float32 x@W^T x2 ({c['threads']} "
                          f"threads) {c['matmul_s']:.2f}s, extrapolated x{c['scale']:.1f} to "
                          f"{c['step_s']:.1f}s per step; the GPU outputs of those {c['checked']} projections "
                          f"match it within rel 1e-3")}
    mode = "5% of model 2 truncated, model 1's rest in fp16 tails" if tails else \
        "model 2 truncated by 5% and zero-padded (.dualpack format)"
    line("achieved HBM GB/s (% of peak) + ms per dual-pack 3B decode step, batch 1", achieved, ms, args, "fp32",
         {"workload": f"dual-pack Qwen2.5-3B-shaped Linear stream, batch-1 decode step, {mode}",
          "layers": args.layers, "projections": len(shapes), "models": 2, "batch": 1,
          "pairs": int(pack.n_codes), "tail_weights": pack.tail_lengths,
          "plug_entries": int(pack.plug_idx.numel()), "algorithmic_bytes": int(algo),
          "pct_of_peak": round(100 * achieved / PEAK_HBM_GBS, 2)},
         traffic=pmc_traffic("dual3b") if tails else None, cpu=cpu,
         traffic_profile=PMC_SUMMARY["dual3b"])


# ---------------------------------------------------------------- single Linear layers

def graph_of(launches):
    """One HIP graph that runs every launch once (captured on a side stream)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in launches:                      # warm the code paths outside the capture
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in launches:
            f()
    torch.cuda.synchronize()
    return g


def rotated_streams(make_stream, pack, shapes, M, copies, dev, quad):
    """``copies`` launchable single-Linear streams over distinct copies of the packed
    weights, each with its own activations and outputs."""
    import copy
    sts = []
    g = torch.Generator(device=dev).manual_seed(11)
    for c in range(copies):
        p = pack if c == 0 else copy.copy(pack)
        if c:
            p.codes = pack.codes.clone()
            p.plug_idx = pack.plug_idx.clone()
            if quad:
                p.plug_vals = pack.plug_vals.clone()
            else:
                p.plug_val = pack.plug_val.clone()
                p.scales = pack.scales.clone()
        st = make_stream(p, shapes, M=M)
        xs, outs = st.make_buffers()
        for x in xs:
            x.copy_(torch.randn(x.shape, generator=g, device=dev).to(torch.float16))
        st.bind(xs, outs)
        sts.append((st, xs, outs))
    return sts


def time_graph(sts, args):
    g = graph_of([st for st, _, _ in sts])
    per, wall = time_events(g.replay, args.steps, args.warmup)
    return float(np.median(per)) / len(sts), per


def run_dual2048(args, dev, log):
    N = K = 2048
    pack = dual2048_pack(dev)
    st0 = DualStream(pack, [(N, K)], M=1)
    copies = max(2, -(-MALL_BYTES // st0.algorithmic_bytes()))
    sts = rotated_streams(DualStream, pack, [(N, K)], 1, copies, dev, quad=False)
    sanity_dual_single(sts[0], pack, dev)
    ms, per = time_graph(sts, args)
    algo = sts[0][0].algorithmic_bytes()
    achieved = algo / (ms * 1e-3) / 1e9
    log(f"[bench] dual 2048x2048: {ms * 1e3:.2f} us per Linear ({copies} rotated copies) -> {achieved:.1f} GB/s")
    cpu = None if args.no_cpu else cpu_single_dual(pack, N, K)
    line("achieved HBM GB/s (% of peak) + us per dual-pack 2048x2048 Linear, batch 1", achieved, ms, args, "fp32",
         {"workload": "dual-pack Linear 2048x2048, 2 models, batch 1", "N": N, "K": K, "models": 2, "batch": 1,
          "plug_entries": int(pack.plug_idx.numel()), "rotated_copies": copies, "algorithmic_bytes": int(algo),
          "us_per_linear": round(ms * 1e3, 3), "pct_of_peak": round(100 * achieved / PEAK_HBM_GBS, 2)}, cpu=cpu,
         traffic=pmc_traffic("dual2048"), traffic_profile=PMC_SUMMARY["dual2048"])


def sanity_dual_single(entry, pack, dev):
    st, xs, outs = entry
    st()
    torch.cuda.synchronize()
    N, K = st.shapes[0]
    amp, cos, sin = pk.header_luts(pack.amp_bits, pack.phase_bits, pack.mu, device=dev)
    w = pk.dual_dequant(pack.codes.reshape(N, K).t(), pack.scales, amp, cos, sin, plug=(pack.plug_idx, pack.plug_val),
                        layout=pack.layout, chunk_size=pack.chunk_size)
    for m in range(2):
        ref = xs[0].float() @ w[m]
        d = (outs[0][m].float() - ref).abs().max().item()
        if not d <= 2e-3 * ref.abs().max().item():
            raise SystemExit(f"dual single-Linear sanity check failed on model {m}")


def cpu_single_dual(pack, N, K):
    from oracle import dualpack as odp
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    be = pack.codes.cpu().numpy().view(np.uint8).copy()
    dp = odp.DualPack(n_pairs=pack.n_codes, n1=pack.n1, n2=pack.n2, codes_be=be, scales=pack.scales.cpu().numpy(),
                      plug_idx=pack.plug_host().copy(), plug_val=pack.plug_val.cpu().numpy(), mu=pack.mu,
                      group_size=pack.group_size, chunk_size=pack.chunk_size)
    x = torch.from_numpy(np.random.default_rng(0).standard_normal((1, K)).astype(np.float32))
    tu, tm = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        w1, w2 = odp.decode_pairs_f64(dp)
        w1, w2 = w1.astype(np.float32).reshape(N, K), w2.astype(np.float32).reshape(N, K)
        t1 = time.perf_counter()
        for w in (w1, w2):
            x @ torch.from_numpy(w).t()
        t2 = time.perf_counter()
        tu.append(t1 - t0)
        tm.append(t2 - t1)
    s = float(np.median(tu)) + float(np.median(tm))
    algo = 2 * N * K + 2 * -(-N * K // pack.group_size) + 6 * pack.plug_idx.numel() + 2 * K + 4 * N
    return {"value": algo / s / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole Linear: numpy float64 unpack_dual restatement (1 thread) {np.median(tu):.3f}s + "
                      f"torch CPU float32 x@W^T x2 ({threads} threads) {np.median(tm):.4f}s, median of 3"}


def quad_linear_pack(N, K, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    w0 = student_t(N * K, 5, 0.02, g, dev)
    models = [[(w0 + torch.randn(N * K, generator=g, device=dev) * (0.002 * (m + 1))).to(torch.float16)]
              for m in range(4)]
    return pack_quad_device(models, plug_cap=0.001, select="norm")


class _batch_as_stream:
    """QuadBatch with the QuadStream interface used by the single-Linear benches."""

    def __init__(self, pack, shapes, M):
        (N, K), = shapes
        self.qb = QuadBatch(pack, N, K, 0, M)
        self.shapes = shapes

    def make_buffers(self):
        x, outs = self.qb.make_buffers()
        return [x], [outs]

    def bind(self, xs, outs):
        self.qb.bind(xs[0], outs[0])

    def __call__(self):
        self.qb()

    def algorithmic_bytes(self):
        return self.qb.algorithmic_bytes()


def sanity_quad_single(entry, pack, dev):
    st, xs, outs = entry
    st()
    torch.cuda.synchronize()
    N, K = st.shapes[0]
    luts = qk.header_luts(pack.r_max, device=dev)
    w = qk.quad_dequant(pack.codes.reshape(N, K).t(), luts, list(pack.s), plug=(pack.plug_idx, pack.plug_vals))
    for m in range(4):
        ref = xs[0].float() @ w[m]
        d = (outs[0][m].float() - ref).abs().max().item()
        if not d <= 2e-3 * ref.abs().max().item():
            raise SystemExit(f"quad single-Linear sanity check failed on model {m}")


def cpu_single_quad(pack, N, K, M):
    from oracle import quadpack as oqp
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    qp = oqp.QuadPack(n=pack.n, s=pack.s, r_max=pack.r_max, codes=pack.codes.cpu().view(torch.int32).numpy()
                      .view(np.uint32), plug_idx=pack.plug_host().copy(), plug_vals=pack.plug_vals.cpu().numpy())
    x = torch.from_numpy(np.random.default_rng(0).standard_normal((M, K)).astype(np.float32))
    tu, tm = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        ws = oqp.unpack_quad(qp)
        t1 = time.perf_counter()
        for w in ws:
            x @ torch.from_numpy(w.reshape(N, K)).t()
        t2 = time.perf_counter()
        tu.append(t1 - t0)
        tm.append(t2 - t1)
        del ws
    s = float(np.median(tu)) + float(np.median(tm))
    algo = 4 * N * K + 12 * pack.plug_idx.numel() + 2 * M * K + 8 * M * N
    return {"value": algo / s / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole Linear at {M} token(s): numpy float64 unpack_quad restatement (1 thread) "
                      f"{np.median(tu):.3f}s + torch CPU float32 x@W^T x4 ({threads} threads) "
                      f"{np.median(tm):.4f}s, median of 3"}


def run_quad_single(args, dev, log, N, K, M, name, pack=None):
    """Up to 4 tokens: the fused row decode (QuadStream of one projection); more: the
    matrix-core batch decode (QuadBatch), as quad_bitpacked routes (N,K) rows."""
    pack = pack if pack is not None else quad_linear_pack(N, K, dev, seed_of(2, 0, 0))
    caps = routes.quad_storage(1, K, 0, K, N, 1)            # (N,K) container rows, with plug entries
    make = QuadStream if routes.quad_route(M, K, N, caps, True) == "rows" else _batch_as_stream
    st0 = make(pack, [(N, K)], M=M)
    copies = max(2, -(-MALL_BYTES // st0.algorithmic_bytes()))
    sts = rotated_streams(make, pack, [(N, K)], M, copies, dev, quad=True)
    sanity_quad_single(sts[0], pack, dev)
    ms, per = time_graph(sts, args)
    algo = sts[0][0].algorithmic_bytes()
    achieved = algo / (ms * 1e-3) / 1e9
    tflops = 8.0 * M * N * K / (ms * 1e-3) / 1e12
    log(f"[bench] quad {name} {N}x{K} M={M}: {ms * 1e3:.2f} us per Linear ({copies} rotated copies) -> "
        f"{achieved:.1f} GB/s, {tflops:.2f} TFLOP/s")
    cpu = None if args.no_cpu else cpu_single_quad(pack, N, K, M)
    line(f"achieved HBM GB/s (% of peak) + us per quad-pack {name} {N}x{K} Linear, {M} token(s)", achieved, ms,
         args, "fp32",
         {"workload": f"quad-pack Linear {name} {N}x{K}, 4 models, {M} token(s) per model", "N": N, "K": K,
          "models": 4, "batch": M, "plug_entries": int(pack.plug_idx.numel()), "rotated_copies": copies,
          "algorithmic_bytes": int(algo), "us_per_linear": round(ms * 1e3, 3),
          "pct_of_peak": round(100 * achieved / PEAK_HBM_GBS, 2), "tflops": round(tflops, 3),
          "pct_of_fp16_mfma_peak": round(100 * tflops / PEAK_FP16_TFLOPS, 3)}, cpu=cpu,
         **({"traffic": pmc_traffic("quadgate"), "traffic_profile": PMC_SUMMARY["quadgate"]}
            if (N, K, M) == (11008, 2048, 1) and args.workload == "quadgate" else {}))
    return pack


def run_refbench(args, dev, log):
    """The reference's __main__ benchmarks: wall clock of 100 calls after 10 warm-ups
    (with a synchronize), as quad_kernels.py:175-200 / polar_kernels.py:165-184 time them,
    plus HIP events around the same calls; fp16 torch.matmul of the unpacked weights as
    the reference's comparison.  The weights (67 / 34 MB packed) stay in the 256 MB
    last-level cache between calls, as on the reference's own card."""
    K = N = 4096
    g = torch.Generator(device=dev).manual_seed(seed_of(6, 0, 0))
    ws = [torch.randn(K, N, generator=g, device=dev).to(torch.float16) for _ in range(4)]
    codes, luts, scales = qk.pack_quad_layer(*ws)
    packed, bmax, amp_lut, cos_lut, sin_lut = pk.quantize_polar_bitpacked(ws[0], ws[1])
    ops = {
        "quad": (lambda a: qk.quad_bitpacked(a, codes, luts, scales), lambda a: [torch.matmul(a, w) for w in ws],
                 lambda M: 4 * K * N + 2 * M * K + 8 * M * N),
        "dual": (lambda a: pk.polar_dual_bitpacked(a, packed, bmax, amp_lut, cos_lut, sin_lut),
                 lambda a: [torch.matmul(a, w) for w in ws[:2]],
                 lambda M: 2 * K * N + 2 * (K * N // 32) + 2 * M * K + 4 * M * N),
    }
    for name, (op, ref, algo) in ops.items():
        rows = []
        for M in (1, 8, 32, 128, 1024):
            a = torch.randn(M, K, generator=g, device=dev).to(torch.float16)
            got = op(a)
            want = ref(a)
            torch.cuda.synchronize()
            for o, r in zip(got, want):
                d = (o.float() - r.float()).abs().max().item()
                if not d <= 0.05 * r.float().abs().max().item():     # 8-bit (quad) / 6+10-bit (dual) codes
                    raise SystemExit(f"refbench {name} M={M}: max |diff| {d} vs fp16 matmul")
            for _ in range(10):
                op(a)
                ref(a)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(100):
                op(a)
            torch.cuda.synchronize()
            tq = (time.perf_counter() - t0) / 100
            t0 = time.perf_counter()
            for _ in range(100):
                ref(a)
            torch.cuda.synchronize()
            tf = (time.perf_counter() - t0) / 100
            per, _ = time_events(lambda: op(a), 30, 5)
            ev = float(np.median(per)) * 1e-3
            row = {"M": M, "packed_ms": round(tq * 1e3, 4), "fp16_matmul_ms": round(tf * 1e3, 4),
                   "speedup_vs_fp16": round(tf / tq, 3), "packed_event_ms": round(ev * 1e3, 4),
                   "gbs_event": round(algo(M) / ev / 1e9, 1)}
            extra = ""
            if name == "quad" and M > 64:
                # the fused large-batch kernel at every size (the operator's default above
                # 128 tokens is the fp16 decode + one batched GEMM)
                fz = lambda: qk.quad_bitpacked(a, codes, luts, scales, fused=True)
                for o, r in zip(fz(), want):
                    d = (o.float() - r.float()).abs().max().item()
                    if not d <= 0.05 * r.float().abs().max().item():
                        raise SystemExit(f"refbench fused M={M}: max |diff| {d} vs fp16 matmul")
                per, _ = time_events(fz, 30, 5)
                row["fused_event_ms"] = round(float(np.median(per)), 4)
                extra = f", fused kernel {row['fused_event_ms']:.3f} ms"
            rows.append(row)
            log(f"[bench] refbench {name} M={M}: {tq * 1e3:.3f} ms (events {ev * 1e3:.3f} ms) vs fp16 "
                f"{tf * 1e3:.3f} ms -> {tf / tq:.2f}x{extra}")
        first = rows[0]
        achieved = algo(1) / (first["packed_event_ms"] * 1e-3) / 1e9
        line(f"ms per {name} drop-in call on 4096x4096 weights vs fp16 matmul (the reference's own benchmark)",
             achieved, first["packed_event_ms"], args, "fp32",
             {"workload": f"{name} drop-in operator, 4096x4096 N(0,1) weights, M = 1, 8, 32, 128, 1024",
              "K": K, "N": N, "models": 4 if name == "quad" else 2, "rows": rows,
              "value_is": "GB/s of algorithmic bytes at M=1 (HIP events, weights cache-resident)"})


def run_quadbig(args, dev, log):
    """The fused large-batch kernel (quad_big_kernel) on the reference benchmark's layer
    (4 models of 4096 x 4096 N(0,1) weights packed by pack_quad_layer, (K,N) codes) at
    ``--big-tokens`` tokens, forced with fused=True at every size; checked against fp16
    torch.matmul of the original weights, timed with HIP events. The roofline is the
    matrix cores' (fp16 dense): 8 M K N flops per call."""
    K = N = 4096
    g = torch.Generator(device=dev).manual_seed(seed_of(6, 0, 0))
    ws = [torch.randn(K, N, generator=g, device=dev).to(torch.float16) for _ in range(4)]
    codes, luts, scales = qk.pack_quad_layer(*ws)
    for M in args.big_tokens:
        a = torch.randn(M, K, generator=g, device=dev).to(torch.float16)
        run = lambda: qk.quad_bitpacked(a, codes, luts, scales, fused=True)
        for o, w in zip(run(), ws):
            r = torch.matmul(a, w).float()
            d = (o.float() - r).abs().max().item()
            if not d <= 0.05 * r.abs().max().item():
                raise SystemExit(f"quadbig M={M}: max |diff| {d} vs fp16 matmul")
        per, _ = time_events(run, args.steps, args.warmup)
        ms = float(np.mean(per))
        tflops = 8.0 * M * K * N / (ms * 1e-3) / 1e12
        log(f"[bench] quadbig M={M}: {ms * 1e3:.1f} us per call -> {tflops:.0f} TFLOP/s")
        line("TFLOP/s of the fused large-batch quad decode (4 models) on a 4096x4096 layer", tflops, ms, args,
             "fp16 operands, fp32 sums",
             {"workload": f"quad_bitpacked(fused=True), 4096x4096 pack_quad_layer codes, {M} tokens", "K": K,
              "N": N, "models": 4, "tokens": M, "flops_per_call": 8 * M * K * N}, bound="mfma")


def run_dualmfma(args, dev, log):
    """The dual matrix-core decode (pp_dual_mfma) on the reference benchmark's dual layer
    (2 models of 4096 x 4096 N(0,1) weights packed by quantize_polar_bitpacked, int16 (K,N)
    codes) at ``--dual-tokens`` tokens, forced with fused=True; checked against fp16
    torch.matmul of the original weights, timed with HIP events. Roofline: the matrix
    cores' fp16 dense peak, 4 M K N flops per call."""
    K = N = 4096
    g = torch.Generator(device=dev).manual_seed(seed_of(6, 0, 1))
    ws = [torch.randn(K, N, generator=g, device=dev).to(torch.float16) for _ in range(2)]
    packed, bmax, amp_lut, cos_lut, sin_lut = pk.quantize_polar_bitpacked(ws[0], ws[1])
    for M in args.dual_tokens:
        a = torch.randn(M, K, generator=g, device=dev).to(torch.float16)
        run = lambda: pk.polar_dual_bitpacked(a, packed, bmax, amp_lut, cos_lut, sin_lut, fused=True)
        for o, w in zip(run(), ws):
            r = torch.matmul(a, w).float()
            d = (o.float() - r).abs().max().item()
            if not d <= 0.05 * r.abs().max().item():
                raise SystemExit(f"dualmfma M={M}: max |diff| {d} vs fp16 matmul")
        per, _ = time_events(run, args.steps, args.warmup)
        ms = float(np.mean(per))
        tflops = 4.0 * M * K * N / (ms * 1e-3) / 1e12
        log(f"[bench] dualmfma M={M}: {ms * 1e3:.1f} us per call -> {tflops:.0f} TFLOP/s")
        line("TFLOP/s of the dual matrix-core decode (2 models) on a 4096x4096 layer", tflops, ms, args,
             "fp16 operands, fp32 sums",
             {"workload": f"polar_dual_bitpacked(fused=True), 4096x4096 quantize_polar_bitpacked codes, {M} tokens",
              "K": K, "N": N, "models": 2, "tokens": M, "flops_per_call": 4 * M * K * N}, bound="mfma")


def run_dualrows(args, dev, log):
    """polar_dual_bitpacked on (N,K) rows of a .dualpack stream (the reference's (K,N) view of
    the container), 2048x2048, gate 11008x2048 and down 2048x11008, at ``--rows-tokens``:
    the default route (the container-row matrix-core decode from 1 token, 3 when N > K, to
    64) against ``fused=False`` (the row kernel to 4 tokens, then the fp16 decode + library
    GEMM), per Linear: each graph replays every rotated copy of the codes once (the MALL
    holds none of them), no plug table; checked against the fp16 decode + fp16 matmul."""
    for name, N, K in (("2048", 2048, 2048), ("gate", 11008, 2048), ("down", 2048, 11008)):
        g = torch.Generator(device=dev).manual_seed(seed_of(7, 0, N + K))
        w0 = student_t(N * K, 5, 0.02, g, dev)
        w1 = (w0 + torch.randn(N * K, generator=g, device=dev) * 0.002).to(torch.float16)
        w2 = (w0 + torch.randn(N * K, generator=g, device=dev) * 0.002).to(torch.float16)
        pack = pack_dual_device(w1, w2, plug_cap=0.001, select="norm")
        del w0, w1, w2
        amp, cs, sn = pk.header_luts(pack.amp_bits, pack.phase_bits, pack.mu, device=dev)
        copies = max(2, -(-MALL_BYTES // (2 * N * K)))
        views = [(pack.codes if c == 0 else pack.codes.clone())[:N * K].reshape(N, K).t() for c in range(copies)]
        wref = pk.dual_dequant(views[0], pack.scales, amp, cs, sn, layout=pack.layout, chunk_size=pack.chunk_size,
                               dtype=torch.float16)
        for M in args.rows_tokens:
            times = {}
            for fused in (None, False):
                route = pk.dual_call_route(views[0], M, layout=pack.layout, chunk_size=pack.chunk_size, fused=fused)
                xs = [torch.randn(M, K, generator=g, device=dev).to(torch.float16) for _ in views]
                fs = [(lambda v=v, x=x: pk.polar_dual_bitpacked(x, v, pack.scales, amp, cs, sn, layout=pack.layout,
                                                                chunk_size=pack.chunk_size, fused=fused))
                      for v, x in zip(views, xs)]
                for o, w in zip(fs[0](), wref):
                    r = torch.matmul(xs[0], w).float()
                    d = (o.float() - r).abs().max().item()
                    if not d <= 2e-2 * r.abs().max().item():
                        raise SystemExit(f"dualrows {name} M={M} route {route}: max |diff| {d} vs fp16 matmul")
                graph = graph_of(fs)
                per, _ = time_events(graph.replay, args.steps, args.warmup)
                times[fused] = (route, float(np.median(per)) / len(fs))
                del graph
            route, ms = times[None]
            algo = 2 * N * K + 2 * -(-N * K // pack.group_size) + 2 * M * K + 4 * M * N
            achieved = algo / (ms * 1e-3) / 1e9
            log(f"[bench] dual rows {name} {N}x{K} M={M}: {route} {ms * 1e3:.2f} us per Linear, "
                f"{times[False][0]} {times[False][1] * 1e3:.2f} us")
            line(f"achieved HBM GB/s (% of peak) + us per dual-pack container-row Linear {N}x{K}, {M} token(s)",
                 achieved, ms, args, "fp16 operands, fp32 sums",
                 {"workload": f"polar_dual_bitpacked on .dualpack (N,K) rows {N}x{K}, 2 models, {M} token(s)",
                  "N": N, "K": K, "models": 2, "tokens": M, "route": route, "rotated_copies": copies,
                  "algorithmic_bytes": int(algo), "us_per_linear": round(ms * 1e3, 3),
                  "fused_false_route": times[False][0], "fused_false_us": round(times[False][1] * 1e3, 3)})
        del views, pack, wref
        torch.cuda.empty_cache()


def run_sweep(args, dev, log):
    for name, N, K in (("gate_proj", 11008, 2048), ("down_proj", 2048, 11008)):
        if name not in args.sweep_shapes:
            continue
        pack = quad_linear_pack(N, K, dev, seed_of(4, 0, 0 if name == "gate_proj" else 1))
        for M in args.sweep_tokens:
            run_quad_single(args, dev, log, N, K, M, name, pack=pack)
        del pack
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--workload", default="quad3b",
                    choices=["quad3b", "dual3b", "dual3b-pad", "dual2048", "quadgate", "sweep", "refbench",
                             "quadbig", "dualmfma", "dualrows"])
    ap.add_argument("--big-tokens", type=int, nargs="+", default=[128, 1024])
    ap.add_argument("--dual-tokens", type=int, nargs="+", default=[8, 32, 64])
    ap.add_argument("--sweep-tokens", type=int, nargs="+", default=[1, 4, 16, 64])
    ap.add_argument("--rows-tokens", type=int, nargs="+", default=[1, 4, 16, 64])
    ap.add_argument("--sweep-shapes", nargs="+", default=["gate_proj", "down_proj"],
                    choices=["gate_proj", "down_proj"])
    ap.add_argument("--cpu-sample-tuples", type=int, default=77_070_336)  # one layer
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 2 GiB device-to-device copy (reference for the rocprof byte counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        src = torch.ones(2 << 30, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 2 << 30, "launches": 3}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (the decode step is a "
              "single-GPU path; a sharded step would run the same kernel on a row slice of every "
              "projection per GPU)", file=sys.stderr)
        sys.exit(2)
    log = (lambda *a: None) if args.quiet else (lambda *a: print(*a, file=sys.stderr, flush=True))
    dev = torch.device("cuda:0")
    if args.workload == "quad3b":
        run_quad3b(args, dev, log)
    elif args.workload in ("dual3b", "dual3b-pad"):
        run_dual3b(args, dev, log, tails=args.workload == "dual3b")
    elif args.workload == "dual2048":
        run_dual2048(args, dev, log)
    elif args.workload == "quadgate":
        run_quad_single(args, dev, log, 11008, 2048, 1, "gate_proj")
    elif args.workload == "refbench":
        run_refbench(args, dev, log)
    elif args.workload == "quadbig":
        run_quadbig(args, dev, log)
    elif args.workload == "dualmfma":
        run_dualmfma(args, dev, log)
    elif args.workload == "dualrows":
        run_dualrows(args, dev, log)
    else:
        run_sweep(args, dev, log)


if __name__ == "__main__":
    main()
