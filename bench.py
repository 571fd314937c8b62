#!/usr/bin/env python3
"""Batch-1 decode step over a quad-pack Qwen2.5-3B-shaped Linear stream on one MI355X.

Workload (one "step"): 36 layers x {q, o 2048x2048; k, v 256x2048; gate, up
11008x2048; down 2048x11008} projections, 4 models packed in one .quadpack v2
stream (2,774,532,096 uint32 tuples, top 0.1% of tuples by norm in the plug table),
one fp16 N(0,1) activation vector per projection, 4 fp16 outputs per projection,
decoded by one pp_quad_stream launch.  Weights are synthetic: per layer-seeded
Student-t(df=5) base scaled to std 0.02, model i = base + N(0, 0.002 i), fp16.

Prints ONE JSON line: achieved GB/s of algorithmic bytes (value), ms per step,
roofline (HIP-event kernel time vs 8 TB/s HBM) and the CPU baseline (the CPU
oracle's numpy unpack + torch CPU matmul on a bounded sample, extrapolated).

    python bench.py [--steps 30] [--warmup 10] [--layers 36] [--no-cpu]
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

from polar_pack_amd import quad_kernels as qk  # noqa: E402
from polar_pack_amd.packer import pack_quad_device  # noqa: E402
from polar_pack_amd.stream import QuadStream  # noqa: E402

METRIC = "achieved HBM GB/s (% of peak) + ms per quad-pack 3B decode step, batch 1"
PEAK_HBM_GBS = 8000.0
LAYER = [("q_proj", 2048, 2048), ("k_proj", 256, 2048), ("v_proj", 256, 2048), ("o_proj", 2048, 2048),
         ("gate_proj", 11008, 2048), ("up_proj", 11008, 2048), ("down_proj", 2048, 11008)]
PMC_SUMMARY = os.path.join(ROOT, "profiles", "quad_stream_3b_pmc.md")


def seed_of(config, layer, proj):
    return 20260000 + 1000 * config + 10 * layer + proj


def synth_models(n_layers, dev):
    """4 correlated fp16 models, flat (N,K) row-major per projection, stream order."""
    models = [[], [], [], []]
    t_scale = 0.02 / math.sqrt(5.0 / 3.0)         # Student-t(5) has variance 5/3
    for layer in range(n_layers):
        for p, (_, n, k) in enumerate(LAYER):
            g = torch.Generator(device=dev).manual_seed(seed_of(3, layer, p))
            z = torch.randn(n * k, generator=g, device=dev)
            chi = torch.zeros_like(z)
            for _ in range(5):
                chi += torch.randn(n * k, generator=g, device=dev) ** 2
            w0 = z / torch.sqrt(chi / 5.0) * t_scale
            del z, chi
            for m in range(4):
                d = torch.randn(n * k, generator=g, device=dev) * (0.002 * (m + 1))
                models[m].append((w0 + d).to(torch.float16))
                del d
            del w0
    return models


def cpu_baseline(pack, shapes, sample_tuples):
    """The CPU oracle's unpack (numpy float64, single thread) + torch CPU float32 matmul,
    on the first projections of the stream up to ~sample_tuples, extrapolated to the step."""
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
    for n, k in take:
        sub = oqp.QuadPack(n=n * k, s=qp.s, r_max=qp.r_max, codes=qp.codes[pos:pos + n * k],
                           plug_idx=(qp.plug_idx[(qp.plug_idx >= pos) & (qp.plug_idx < pos + n * k)] - pos).astype(np.uint32),
                           plug_vals=qp.plug_vals[(qp.plug_idx >= pos) & (qp.plug_idx < pos + n * k)])
        t0 = time.perf_counter()
        ws = oqp.unpack_quad(sub)
        t1 = time.perf_counter()
        x = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float32))
        for w in ws:
            y = x @ torch.from_numpy(w.reshape(n, k)).t()
        t2 = time.perf_counter()
        t_unpack += t1 - t0
        t_mm += t2 - t1
        pos += n * k
        del ws, y
    total_tuples = sum(n * k for n, k in shapes)
    scale = total_tuples / tuples
    return {"unpack_s": t_unpack, "matmul_s": t_mm, "sample_tuples": tuples, "scale": scale,
            "step_s": (t_unpack + t_mm) * scale, "threads": threads}


def read_pmc_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE), if committed."""
    try:
        text = open(PMC_SUMMARY).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch\s*[=:]\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=36)
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
              "single-GPU path; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)
    log = (lambda *a: None) if args.quiet else (lambda *a: print(*a, file=sys.stderr, flush=True))
    dev = torch.device("cuda:0")
    shapes = [(n, k) for _ in range(args.layers) for (_, n, k) in LAYER]

    t0 = time.time()
    models = synth_models(args.layers, dev)
    torch.cuda.synchronize()
    log(f"[bench] synthesized 4 x {sum(n * k for n, k in shapes)} fp16 weights in {time.time() - t0:.1f}s")
    t0 = time.time()
    pack = pack_quad_device(models, plug_cap=0.001, select="norm")
    torch.cuda.synchronize()
    del models
    torch.cuda.empty_cache()
    log(f"[bench] packed: n={pack.n} plug={pack.plug_idx.numel()} r_max={pack.r_max:.4f} in {time.time() - t0:.1f}s")

    st = QuadStream(pack, shapes, M=1)
    xs, outs = st.make_buffers()
    g = torch.Generator(device=dev).manual_seed(7)
    for x in xs:
        x.copy_(torch.randn(x.shape, generator=g, device=dev).to(torch.float16))
    st.bind(xs, outs)
    log(f"[bench] plan: {st.n_segs} segments, {st.n_tail} tail items, {st.n_waves} waves")

    # sanity: the stream output equals the per-projection operator on a k_proj and a down_proj
    st()
    torch.cuda.synchronize()
    luts = qk.header_luts(pack.r_max, device=dev)
    for p in (1, 6):
        n, k = shapes[p]
        pos = int(st.pos0[p])
        single = qk.quad_bitpacked(xs[p], pack.codes[pos:pos + n * k].reshape(n, k).t(), luts, list(pack.s),
                                   plug=(pack.plug_idx, pack.plug_vals), elem_base=pos)
        for m in range(4):
            d = (outs[p][m].float() - single[m].float()).abs().max().item()
            ref = single[m].float().abs().max().item()
            if not d <= 2e-3 * ref:
                raise SystemExit(f"stream/single mismatch on projection {p} model {m}: {d} vs {ref}")

    for _ in range(args.warmup):
        st()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record()
        st()
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    ms = float(np.mean(per))
    algo = st.algorithmic_bytes()
    achieved = algo / (ms * 1e-3) / 1e9
    log(f"[bench] step: mean {ms:.4f} ms, median {np.median(per):.4f}, min {min(per):.4f}, wall/step "
        f"{wall / args.steps * 1e3:.4f} ms; {algo / 1e9:.4f} GB algorithmic -> {achieved:.1f} GB/s")

    cpu = None
    if not args.no_cpu:
        c = cpu_baseline(pack, shapes, args.cpu_sample_tuples)
        log(f"[bench] cpu baseline: unpack {c['unpack_s']:.2f}s + matmul {c['matmul_s']:.2f}s on "
            f"{c['sample_tuples']} tuples -> {c['step_s']:.2f}s per step (x{c['scale']:.1f})")
        cpu = {"value": algo / c["step_s"] / 1e9, "unit": "GB/s", "cores": c["threads"], "kind": "port",
               "sample": (f"first {c['sample_tuples']} tuples of the stream ({c['sample_tuples'] / pack.n:.2%}): "
                          f"numpy float64 unpack_quad restatement (1 thread) {c['unpack_s']:.2f}s + torch CPU "
                          f"float32 x@W^T x4 ({c['threads']} threads) {c['matmul_s']:.2f}s, extrapolated x"
                          f"{c['scale']:.1f} to {c['step_s']:.1f}s per step")}

    traffic = read_pmc_traffic()
    out = {
        "metric": METRIC, "value": round(achieved, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "quad-pack Qwen2.5-3B-shaped Linear stream, batch-1 decode step",
                   "layers": args.layers, "projections": len(shapes), "models": 4, "batch": 1,
                   "tuples": int(pack.n), "plug_entries": int(pack.plug_idx.numel()),
                   "algorithmic_bytes": int(algo), "pct_of_peak": round(100 * achieved / PEAK_HBM_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
