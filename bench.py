#!/usr/bin/env python3
"""Benchmark of the quantized decode path on one MI355X.

Default workload (one "step"): the seven decode matvecs of one Llama-3-8B
layer at batch 1 with the Q4_K_M mix -- q/k/o/gate/up in Q4_K, v/down in
Q6_K -- on seeded synthetic weights (localai_amd/synth.py), weights already
resident in HBM. Several weight copies (> 2 x 256 MB Infinity Cache) are
rotated so every step streams from HBM. Each step is replayed from a HIP
graph captured on the launch stream (launch overhead of 7 small kernels
would otherwise dominate the ~20 us of GPU work).

Printed: one JSON line. `value` = algorithmic bytes of the layer (weights +
fp32 in/out vectors, 139,231,232 B) / measured time per layer, in GB/s.
`roofline` = the dominant kernel (Q4_K matvec, ffn_gate shape 14336x4096)
timed alone with HIP events on its stream. `cpu_baseline` = the reference's
own engine/native_quant.cpp kernels (built from source into oracle/_ref) on
the host cores, with the reference's thread policy.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--cpu-baseline auto|off]
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def log(msg):
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--workload', default='llama3_8b_decode_layer',
                    choices=['llama3_8b_decode_layer'])
    ap.add_argument('--cpu-baseline', default='auto', choices=['auto', 'off'])
    ap.add_argument('--seed', type=int, default=0)
    return ap.parse_args()


# ------------------------------------------------------------------ GPU side

def build_layer(torch, device, synth, copies, seed):
    """copies x 7 weight handles + the three input vectors + outputs."""
    rng = np.random.default_rng(seed)
    host = {name: synth.quant_tensor(rng, t, rows, cols) for name, t, rows, cols, _ in synth.LLAMA3_8B_LAYER}
    vecs = {'h': synth.activations(rng, 4096), 'attn': synth.activations(rng, 4096),
            'h2': synth.activations(rng, 4096), 'act': synth.activations(rng, 14336)}
    xs = {k: device.to_device_f32(v) for k, v in vecs.items()}
    mats = []
    for _ in range(copies):
        mats.append({name: device.QMat.from_ggml(host[name], t, rows, cols)
                     for name, t, rows, cols, _ in synth.LLAMA3_8B_LAYER})
    outs = {name: torch.empty(rows, dtype=torch.float32, device=device.device())
            for name, _, rows, _, _ in synth.LLAMA3_8B_LAYER}
    return host, vecs, xs, mats, outs


def run_layer(mats, xs, outs, synth, stream):
    for name, _, _, _, src in synth.LLAMA3_8B_LAYER:
        mats[name].matvec(xs[src], out=outs[name], stream=stream)


def capture(torch, fn, stream):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()                     # warm once outside the graph
        torch.cuda.current_stream().synchronize()
        with torch.cuda.graph(g, stream=stream):
            fn()
    torch.cuda.synchronize()
    return g


def time_graphs(torch, graphs, stream, steps, warmup):
    """Replay graphs round-robin on `stream`; HIP events on the same stream."""
    with torch.cuda.stream(stream):
        for i in range(warmup):
            graphs[i % len(graphs)].replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(steps):
            graphs[i % len(graphs)].replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps      # ms per step


# ---------------------------------------------------------------- CPU side

def cpu_has_avx2():
    try:
        flags = open('/proc/cpuinfo').read()
        return ' avx2 ' in flags and ' fma ' in flags
    except OSError:
        return False


def cpu_model():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def reference_threads(rows, t):
    """engine/gguf_parser.py:13-42 decode policy, capped by this host's cores."""
    if rows >= 65536 and t != 8:
        req = 8
    elif t == 12 and rows >= 4096:
        req = 8
    elif t == 14 and rows >= 4096:
        req = 7
    elif t == 8 or t in (12, 13, 14):
        req = 6
    else:
        req = 4
    return min(req, os.cpu_count() or 1)


def cpu_baseline(host, vecs, synth, layer_bytes):
    """Time the reference's AVX2 kernels (oracle/_ref) on one layer."""
    from oracle import ref
    if not (ref.available() and cpu_has_avx2()):
        return None
    threads = []
    calls = []
    for name, t, rows, cols, src in synth.LLAMA3_8B_LAYER:
        th = reference_threads(rows, t)
        threads.append(th)
        calls.append((host[name], vecs[src], rows, cols, t, th))
    for _ in range(3):
        for c in calls:
            ref.matvec(*c[:5], threads=c[5])
    samples = []
    t_end = time.perf_counter() + 10.0
    while len(samples) < 20 or (time.perf_counter() < t_end and len(samples) < 200):
        t0 = time.perf_counter_ns()
        for c in calls:
            ref.matvec(*c[:5], threads=c[5])
        samples.append((time.perf_counter_ns() - t0) / 1e3)
        if len(samples) >= 20 and time.perf_counter() > t_end:
            break
    us = float(np.median(samples))
    return {'value': round(layer_bytes / (us * 1e-6) / 1e9, 3), 'unit': 'GB/s',
            'us_per_layer': round(us, 1), 'cores': max(threads), 'kind': 'reference',
            'sample': f'{len(samples)} full layers (7 matvecs), median; engine/native_quant.cpp '
                      f'built with g++ -O2 -mavx2 -mfma, reference thread policy '
                      f'{dict(zip([n for n, *_ in synth.LLAMA3_8B_LAYER], threads))}; '
                      f'host {cpu_model()}, {os.cpu_count()} logical CPUs visible'}


def main():
    args = parse()
    if args.gpus != 1:
        print(f'bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU runs are not '
              f'part of this build', file=sys.stderr)
        sys.exit(2)
    import torch
    from localai_amd import device, synth, native_quant

    if native_quant.get_native() is None:
        raise SystemExit('no HIP device / library: the benchmark needs the GPU path')
    layer_bytes = synth.layer_algorithmic_bytes()
    weight_bytes = synth.layer_weight_bytes()
    copies = max(2, -(-2 * MALL_BYTES // weight_bytes) + 1)
    log(f'building {copies} weight copies ({copies * weight_bytes / 1e6:.0f} MB)')
    host, vecs, xs, mats, outs = build_layer(torch, device, synth, copies, args.seed)
    stream = torch.cuda.Stream()
    graphs = [capture(torch, lambda m=m: run_layer(m, xs, outs, synth, stream), stream) for m in mats]
    log('graphs captured; timing layer')
    ms = time_graphs(torch, graphs, stream, args.steps, args.warmup)
    gbs = layer_bytes / (ms * 1e-3) / 1e9

    # dominant kernel: Q4_K matvec at the ffn_gate shape, rotated over > 2x MALL
    gate_bytes = 14336 * 16 * 144 + 4 * 4096 + 4 * 14336
    nrot = -(-2 * MALL_BYTES // (14336 * 16 * 144)) + 1
    gate_host = host['ffn_gate']
    gmats = [device.QMat.from_ggml(gate_host, 12, 14336, 4096) for _ in range(nrot)]
    gout = torch.empty(14336, dtype=torch.float32, device=device.device())
    # one graph launching the kernel once on each of the nrot copies (no copy twice in a row)
    ggraph = capture(torch, lambda: [m.matvec(xs['h2'], out=gout, stream=stream) for m in gmats], stream)
    log('timing dominant kernel')
    kms = time_graphs(torch, [ggraph], stream, max(20, args.steps // 4), 5) / nrot
    achieved = gate_bytes / (kms * 1e-3) / 1e9

    # parity spot check of this run's outputs (GPU vs a fresh GPU run is not a check; the
    # oracle comparison lives in tests/ -- here only sanity: finite outputs)
    for name, o in outs.items():
        if not torch.isfinite(o).all():
            raise SystemExit(f'non-finite output in {name}')

    cpu = None
    if args.cpu_baseline != 'off':
        log('timing CPU baseline (reference AVX2 kernels)')
        cpu = cpu_baseline(host, vecs, synth, layer_bytes)

    line = {
        'metric': 'µs/layer + achieved HBM GB/s (% of peak) for Q4_K/Q6_K matvec & MoE layer',
        'value': round(gbs, 2), 'unit': 'GB/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'us_per_layer': round(ms * 1e3, 3),
        'hbm_frac': round(gbs / HBM_PEAK_GBS, 4),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'fp32',
        'data': 'synthetic (seeded GGML Q4_K/Q6_K bytes, fp32 N(0,1) activations)',
        'config': {'workload': 'llama3_8b_decode_layer_q4_k_m', 'matvecs': 7, 'batch': 1,
                   'shapes': [[n, {12: 'Q4_K', 14: 'Q6_K'}[t], r, c] for n, t, r, c, _ in synth.LLAMA3_8B_LAYER],
                   'algorithmic_bytes_per_layer': layer_bytes, 'weight_copies_rotated': copies,
                   'launch': 'hip graph per layer'},
        'roofline': {'bound': 'hbm', 'kernel': 'gemv_kernel<Q4_K,1> 14336x4096',
                     'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(achieved / HBM_PEAK_GBS, 4), 'traffic': None,
                     'us_per_launch': round(kms * 1e3, 3), 'bytes_per_launch': gate_bytes},
        'cpu_baseline': cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
