#!/usr/bin/env python3
"""Benchmark of the quantized-matmul / MoE path on one MI355X.

With no --workload the run prints ONE JSON line: the headline workload
(llama3_8b_decode_layer) at top level, and every other workload below under
"workloads". With --workload NAME only that workload is measured.

Workloads (one "step" = one pass of the path over one batch of synthetic
input, weights already resident in HBM, seeded data from localai_amd/synth.py):

  llama3_8b_decode_layer (headline)  the seven decode matvecs of one
      Llama-3-8B layer at batch 1, Q4_K_M mix (q/k/o/gate/up Q4_K, v/down
      Q6_K). value = algorithmic bytes / time (GB/s). q/k/v and gate/up,
      which read the same vector, are each one fused launch
      (localai_hip_matvec_many); the one-launch-per-matvec time is reported
      beside it.
  q4k_matvec        one Q4_K matvec at the ffn_gate shape 14336x4096.
  q8_0_matvec       one Q8_0 matvec at the same shape.
  vocab_head        the Llama-3-8B vocabulary head, Q6_K 128256x4096 (431 MB).
  legacy_host_matvec  localai_q4k_matvec with host pointers at the ffn_gate
      shape, as LocalAI's own native_quant.matvec calls it (weights in a
      registered host range, cached on the device; x and y copied per call),
      timed on the host around each call.
  q8_0_prefill      Q8_0 GEMM 14336x4096 weights x 512 tokens (TFLOP/s).
  zaya_moe_decode   ZAYA-shaped MoE FFN: hidden 2048, 16 experts, top-2,
      intermediate 4096, Q6_K experts, T = 1 (T = 8 reported alongside).
  qwen3_moe_prefill Qwen3-MoE-style prefill: hidden 2048, 128 experts, top-8,
      intermediate 768, Q4_K experts, 512 tokens, Zipf(1.1) logit bias.
  llama3_8b_layer_chain  the same seven matvecs with the glue
      of the decode step between them (residual adds, both RMSNorms, SiLU*up,
      RoPE of q and k; localai_hip_layer_chain as four glued launches, the
      one-launch form beside it).
  llama3_8b_attention_decode  decode attention of one token over a 4096-
      position fp32 KV cache: 32 query heads, 8 kv heads, head_dim 128
      (localai_hip_attention_decode, the token's k / v row written by the
      same call).
  qwen35_delta_net_step  Qwen3.5's gated delta-net step, 32 heads x 128 x
      128 fp32 state read and written once (localai_hip_delta_net_step).
  hbm_read_floor    the streaming-read kernel (localai_hip_stream_read) over
      the same byte counts: one 33 MB launch, the layer's four dependent
      launches, and the whole layer's 139 MB as one launch -- what a launch
      of that size can stream at best on this GPU.
  hbm_copy          a plain 256 MiB device-to-device copy: the calibration
      kernel for rocprofv3 FETCH_SIZE / WRITE_SIZE (known bytes per launch).

Weight copies beyond 2 x the 256 MB Infinity Cache are rotated so every step
streams its weights from HBM; one HIP graph holds a whole rotation of steps
(as a decode step's graph holds every layer), is replayed on the launch
stream and timed with HIP events on that stream, exactly K steps.
`roofline` is the dominant kernel of the workload timed alone the same way
(or the whole call where it is a composition of kernels), its `traffic` the
HBM bytes per launch from the committed rocprofv3 counter passes
(profiles/traffic.json); `cpu_baseline` is the reference's own
engine/native_quant.cpp kernels (built from source into oracle/_ref) on a
bounded sample, on the host cores, pinned (sched_setaffinity) to one logical
CPU per physical core, at the reference's thread policy and on all cores
(the reference's pool caps at 8 threads), with the NumPy dequantize + matmul
path timed beside it for the dense configs.

stdout carries the one JSON line (every workload's time, value, roofline and
CPU baseline, kept short); stderr carries the full record as a line starting
`[bench] detail` (step statistics, all-core and NumPy CPU legs, shapes).

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--cpu-baseline auto|off]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFS = 2500.0      # dense f16/bf16 MFMA
MALL_BYTES = 256 << 20
METRIC = 'µs/layer + achieved HBM GB/s (% of peak) for Q4_K/Q6_K matvec & MoE layer'
WORKLOADS = ['llama3_8b_decode_layer', 'q4k_matvec', 'q8_0_matvec', 'vocab_head', 'legacy_host_matvec', 'q8_0_prefill',
             'zaya_moe_decode', 'qwen3_moe_prefill', 'llama3_8b_layer_chain', 'llama3_8b_attention_decode',
             'qwen35_delta_net_step', 'hbm_read_floor', 'hbm_copy', 'moe_decode_shapes']
# the default run: the headline, then these under "workloads"
DEFAULT_SUITE = ['q4k_matvec', 'q8_0_prefill', 'zaya_moe_decode', 'qwen3_moe_prefill', 'q8_0_matvec', 'vocab_head',
                 'legacy_host_matvec', 'llama3_8b_layer_chain', 'llama3_8b_attention_decode', 'qwen35_delta_net_step',
                 'hbm_read_floor']


def log(msg):
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--workload', default=None, choices=WORKLOADS,
                    help='one workload only (default: the headline plus every workload of the suite)')
    ap.add_argument('--cpu-baseline', default='auto', choices=['auto', 'off'])
    ap.add_argument('--seed', type=int, default=0)
    return ap.parse_args()


def rotations(bytes_per_step):
    """Copies needed so consecutive steps touch more than 2 x MALL."""
    return max(2, -(-2 * MALL_BYTES // max(1, bytes_per_step)) + 1)


# ------------------------------------------------------------------ GPU timing

def capture(torch, fn, stream):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()                     # warm once outside the graph
        torch.cuda.current_stream().synchronize()
        with torch.cuda.graph(g, stream=stream):
            fn()
    torch.cuda.synchronize()
    return g


DIST = []   # per-step distributions recorded by the timers, in call order


def record_distribution(torch, graph, per_replay, stream, min_steps=100):
    """After a timed region: replay `graph` (per_replay steps each) at least
    min_steps steps' worth, an event pair around each replay on the launch
    stream; keeps the median and p90 of the per-step times."""
    reps = max(10, -(-min_steps // per_replay))
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    with torch.cuda.stream(stream):
        for a, b in evs:
            a.record(stream)
            graph.replay()
            b.record(stream)
    torch.cuda.synchronize()
    per = np.array([a.elapsed_time(b) / per_replay for a, b in evs])
    DIST.append({'median_ms': round(float(np.median(per)), 6), 'p90_ms': round(float(np.percentile(per, 90)), 6),
                 'samples': reps, 'steps_per_sample': per_replay,
                 'how': 'per-step time of each replay of the timed graph, measured after the timed region'})


def time_steps(torch, fns, stream, steps, warmup):
    """Time exactly `steps` steps of the rotation fns[0], fns[1], ... (one
    function per weight copy). One HIP graph holds a whole rotation, as a
    decode step's graph holds every layer, so the host launches once per
    rotation rather than once per step; a second graph holds the first
    steps mod n. HIP events on the launch stream; returns ms per step."""
    n = len(fns)
    full = capture(torch, lambda: [f() for f in fns], stream)
    q, r = divmod(steps, n)
    part = capture(torch, lambda: [f() for f in fns[:r]], stream) if r else None
    with torch.cuda.stream(stream):
        for _ in range(max(1, -(-warmup // n))):
            full.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(q):
            full.replay()
        if part is not None:
            part.replay()
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    record_distribution(torch, full, n, stream)
    return ms      # ms per step


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


def ref_ok():
    from oracle import ref
    return ref.available() and cpu_has_avx2()


def time_cpu(fn, min_samples=5, budget_s=10.0, warm=2):
    for _ in range(warm):
        fn()
    samples = []
    t_end = time.perf_counter() + budget_s
    while len(samples) < min_samples or (time.perf_counter() < t_end and len(samples) < 200):
        t0 = time.perf_counter_ns()
        fn()
        samples.append((time.perf_counter_ns() - t0) / 1e3)
        if len(samples) >= min_samples and time.perf_counter() > t_end:
            break
    return float(np.median(samples)), len(samples)


def host_info():
    """lscpu model name and the physical cores this process may run on, with
    one logical CPU per physical core (the CPUs the baselines are pinned to)."""
    import subprocess
    info = {'model': cpu_model(), 'logical_cpus': os.cpu_count()}
    allowed = sorted(os.sched_getaffinity(0)) if hasattr(os, 'sched_getaffinity') else list(range(os.cpu_count()))
    primary = {}
    try:
        out = subprocess.run(['lscpu'], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(':')
            if k.strip() == 'Model name':
                info['model'] = v.strip()
        out = subprocess.run(['lscpu', '-p=CPU,CORE,SOCKET'], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith('#'):
                continue
            cpu, core, sock = (int(x) for x in line.split(','))
            if cpu in allowed:
                primary.setdefault((sock, core), cpu)
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    cores = sorted(primary.values()) if primary else allowed
    info['physical_cores'] = len(cores)
    info['allowed_cpus'] = len(allowed)
    info['_cores'] = cores
    return info


HOST = {}


def host():
    if not HOST:
        HOST.update(host_info())
    return HOST


def host_note():
    h = host()
    return (f"host {h['model']}, {h['physical_cores']} physical cores / {h['allowed_cpus']} logical CPUs "
            f"available, pinned to one logical CPU per physical core")


class pinned:
    """Pin this process (and the threads the reference's pool starts) to the
    first n physical cores, one logical CPU each, as `taskset` would."""

    def __init__(self, n):
        self.cpus = host()['_cores'][:max(1, n)]

    def __enter__(self):
        self.old = os.sched_getaffinity(0) if hasattr(os, 'sched_setaffinity') else None
        if self.old is not None:
            os.sched_setaffinity(0, self.cpus)
        return self.cpus

    def __exit__(self, *exc):
        if self.old is not None:
            os.sched_setaffinity(0, self.old)


def cpu_runs(call, policy_threads, work, unit, sample, scale_us=1.0, min_samples=20, budget_s=8.0, numpy_call=None,
             numpy_work=None):
    """The reference kernels at the reference's thread policy (pinned to that
    many physical cores) and on all physical cores (threads capped at 8 like
    the reference's pool), plus the NumPy dequantize + matmul path when
    numpy_call is given. call(None) runs one sample at the policy's thread
    counts, call(n) with n threads everywhere; work is the bytes or flops it
    represents (GB/s or TFLOP/s from the median). `sample` names the bounded
    sample in a few words; the host is reported once, at the top of the line."""
    div = 1e9 if unit == 'GB/s' else 1e12
    allc = host()['physical_cores']
    with pinned(policy_threads):
        us, n = time_cpu(lambda: call(None), min_samples=min_samples, budget_s=budget_s)
    ta = min(8, allc)
    with pinned(allc):
        us_all, n_all = time_cpu(lambda: call(ta), min_samples=min_samples, budget_s=budget_s)
    out = {'value': sig(work / (us * 1e-6) / div), 'unit': unit, 'cores': policy_threads, 'kind': 'reference',
           'sample': sample, 'us': round(us * scale_us, 1), 'samples': n,
           'all_cores': {'value': sig(work / (us_all * 1e-6) / div), 'threads': ta, 'cores': allc,
                         'us': round(us_all * scale_us, 1), 'samples': n_all}}
    if numpy_call is not None:
        with pinned(allc):
            us_np, n_np = time_cpu(numpy_call, min_samples=2, budget_s=budget_s, warm=1)
        out['numpy'] = {'value': sig((numpy_work or work) / (us_np * 1e-6) / div), 'unit': unit,
                        'us': round(us_np, 1), 'samples': n_np,
                        'what': 'oracle restatement of engine/dequant.py dequantize + NumPy matmul '
                                '(engine/gguf_parser.py:273-288 fallback), all physical cores'}
    return out


def sig(v, digits=4):
    """v rounded to `digits` significant digits (keeps the one-line record short)."""
    if v is None or v == 0 or not np.isfinite(v):
        return v
    return float(f'{v:.{digits}g}')


# ---------------------------------------------------------------- workloads

def wl_layer(args, torch, device, synth):
    layer = synth.LLAMA3_8B_LAYER
    layer_bytes = synth.layer_algorithmic_bytes()
    weight_bytes = synth.layer_weight_bytes()
    copies = rotations(weight_bytes)
    rng = np.random.default_rng(args.seed)
    host = {name: synth.quant_tensor(rng, t, rows, cols) for name, t, rows, cols, _ in layer}
    vecs = {'h': synth.activations(rng, 4096), 'attn': synth.activations(rng, 4096),
            'h2': synth.activations(rng, 4096), 'act': synth.activations(rng, 14336)}
    xs = {k: device.to_device_f32(v) for k, v in vecs.items()}
    log(f'building {copies} weight copies ({copies * weight_bytes / 1e6:.0f} MB)')
    mats = [{name: device.QMat.from_ggml(host[name], t, rows, cols) for name, t, rows, cols, _ in layer}
            for _ in range(copies)]
    outs = {name: torch.empty(rows, dtype=torch.float32, device=device.device()) for name, _, rows, _, _ in layer}
    stream = torch.cuda.Stream()

    groups = {}
    for name, _, _, _, src in layer:
        groups.setdefault(src, []).append(name)

    def run(m):
        # matrices that read the same vector (q/k/v, gate/up) go out as one launch
        for src, names in groups.items():
            if len(names) == 1:
                m[names[0]].matvec(xs[src], out=outs[names[0]], stream=stream)
            else:
                device.matvec_many([m[n] for n in names], xs[src], outs=[outs[n] for n in names], stream=stream)

    def run_single(m):
        for name, _, _, _, src in layer:
            m[name].matvec(xs[src], out=outs[name], stream=stream)

    log('timing layer')
    ms = time_steps(torch, [lambda m=m: run(m) for m in mats], stream, args.steps, args.warmup)
    ms_single = time_steps(torch, [lambda m=m: run_single(m) for m in mats], stream, args.steps, args.warmup)
    for name, o in outs.items():
        if not torch.isfinite(o).all():
            raise SystemExit(f'non-finite output in {name}')
    roof = gate_up_roofline(args, torch, device, host['ffn_gate'], host['ffn_up'], xs['h2'], stream)
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        log('timing CPU baseline (reference AVX2 kernels)')
        from oracle import ref
        calls = [(host[name], vecs[src], rows, cols, t, reference_threads(rows, t))
                 for name, t, rows, cols, src in layer]
        cpu = cpu_runs(lambda th: [ref.matvec(*c[:5], threads=c[5] if th is None else th) for c in calls],
                       max(c[5] for c in calls), layer_bytes, 'GB/s',
                       '7 localai_*_matvec per layer')
    gbs = layer_bytes / (ms * 1e-3) / 1e9
    return {
        'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
        'us_per_layer_one_launch_per_matvec': round(ms_single * 1e3, 3),
        'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
        'data': 'synthetic (seeded GGML Q4_K/Q6_K bytes, fp32 N(0,1) activations)',
        'config': {'workload': 'llama3_8b_decode_layer_q4_k_m', 'matvecs': 7, 'batch': 1,
                   'shapes': [[n, {12: 'Q4_K', 14: 'Q6_K'}[t], r, c] for n, t, r, c, _ in layer],
                   'algorithmic_bytes_per_layer': layer_bytes, 'weight_copies_rotated': copies,
                   'launch': 'one hip graph per rotation of layer copies; q/k/v and gate/up each one fused launch (shared input)'},
        'roofline': roof, 'cpu_baseline': cpu}


def gate_up_roofline(args, torch, device, gate_host, up_host, x, stream):
    """The layer's dominant kernel: the fused ffn_gate + ffn_up launch (two
    Q4_K 14336 x 4096 matvecs on one x), rotated over > 2x MALL, timed
    alone."""
    nbytes = 2 * 14336 * 16 * 144 + 4 * 4096 + 2 * 4 * 14336
    nrot = rotations(2 * 14336 * 16 * 144)
    pairs = [(device.QMat.from_ggml(gate_host, 12, 14336, 4096), device.QMat.from_ggml(up_host, 12, 14336, 4096))
             for _ in range(nrot)]
    gout = [torch.empty(14336, dtype=torch.float32, device=device.device()) for _ in range(2)]
    log('timing dominant kernel')
    kms = time_steps(torch, [lambda p=p: device.matvec_many(list(p), x, outs=gout, stream=stream) for p in pairs],
                     stream, args.steps, args.warmup)
    achieved = nbytes / (kms * 1e-3) / 1e9
    for p in pairs:
        for m in p:
            m.close()
    return {'bound': 'hbm', 'kernel': 'gemv_mfma<Q4_K> gate+up paired',
            'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
            'frac': round(achieved / HBM_PEAK_GBS, 4), 'traffic': measured_traffic('layer', 'gate_up'),
            'us_per_launch': round(kms * 1e3, 3), 'bytes_per_launch': nbytes}


def gate_roofline(args, torch, device, gate_host, x, stream, t=12):
    """Q4_K (or Q8_0, t = 8) matvec at the ffn_gate shape, rotated over
    > 2x MALL, timed alone."""
    wbytes = 14336 * 16 * 144 if t == 12 else 14336 * 128 * 34
    gate_bytes = wbytes + 4 * 4096 + 4 * 14336
    nrot = rotations(wbytes)
    gmats = [device.QMat.from_ggml(gate_host, t, 14336, 4096) for _ in range(nrot)]
    gout = torch.empty(14336, dtype=torch.float32, device=device.device())
    log('timing dominant kernel')
    kms = time_steps(torch, [lambda m=m: m.matvec(x, out=gout, stream=stream) for m in gmats], stream, args.steps,
                     args.warmup)
    achieved = gate_bytes / (kms * 1e-3) / 1e9
    for m in gmats:
        m.close()
    return {'bound': 'hbm', 'kernel': f"gemv_mfma_{'q4k' if t == 12 else 'q8_0'} 14336x4096",
            'achieved': round(achieved, 1),
            'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': round(achieved / HBM_PEAK_GBS, 4),
            'traffic': measured_traffic('q4k' if t == 12 else 'q8_matvec', 'gate'),
            'us_per_launch': round(kms * 1e3, 3), 'bytes_per_launch': gate_bytes}


def measured_traffic(workload, kernel):
    """HBM bytes per launch of one kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (profiles/traffic.json, calibrated on a
    copy of known size); None if absent."""
    try:
        with open(os.path.join(ROOT, 'profiles', 'traffic.json')) as f:
            return int(json.load(f)[workload][kernel]['traffic_bytes'])
    except (OSError, ValueError, KeyError, TypeError):
        return None


def wl_q4k(args, torch, device, synth):
    rng = np.random.default_rng(args.seed)
    raw = synth.quant_tensor(rng, 12, 14336, 4096)
    xv = synth.activations(rng, 4096)
    x = device.to_device_f32(xv)
    stream = torch.cuda.Stream()
    roof = gate_roofline(args, torch, device, raw, x, stream)
    nbytes = roof['bytes_per_launch']
    ms = roof['us_per_launch'] / 1e3
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        from oracle import ref, quant
        th = reference_threads(14336, 12)

        def numpy_path():
            return quant.dequantize(raw, 12, (14336, 4096)) @ xv
        cpu = cpu_runs(lambda t: ref.matvec(raw, xv, 14336, 4096, 12, threads=th if t is None else t), th, nbytes,
                       'GB/s', 'localai_q4k_matvec', numpy_call=numpy_path)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
            'data': 'synthetic (seeded GGML Q4_K bytes, fp32 N(0,1) x)',
            'config': {'workload': 'q4k_matvec_14336x4096', 'batch': 1, 'algorithmic_bytes': nbytes},
            'roofline': roof, 'cpu_baseline': cpu}


def wl_q8_matvec(args, torch, device, synth):
    """Q8_0 decode matvec at the ffn_gate shape (the q8_0_row path of a Q8_0
    model's decode step): i8 MFMA over the Q8_0 tile form."""
    rng = np.random.default_rng(args.seed)
    raw = synth.quant_tensor(rng, 8, 14336, 4096)
    xv = synth.activations(rng, 4096)
    x = device.to_device_f32(xv)
    stream = torch.cuda.Stream()
    roof = gate_roofline(args, torch, device, raw, x, stream, t=8)
    nbytes = roof['bytes_per_launch']
    ms = roof['us_per_launch'] / 1e3
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        from oracle import ref
        th = reference_threads(14336, 8)
        cpu = cpu_runs(lambda t: ref.matvec(raw, xv, 14336, 4096, 8, threads=th if t is None else t), th, nbytes,
                       'GB/s', 'localai_q8_0_matvec')
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
            'data': 'synthetic (seeded GGML Q8_0 bytes, fp32 N(0,1) x)',
            'config': {'workload': 'q8_0_matvec_14336x4096', 'batch': 1, 'algorithmic_bytes': nbytes},
            'roofline': roof, 'cpu_baseline': cpu}


def wl_vocab_head(args, torch, device, synth):
    """The vocabulary head of a Llama-3-8B decode step (engine/model.py:235-237,
    output.weight 128256 x 4096, Q6_K in a Q4_K_M file): the largest matvec of
    the step, 431 MB, one launch."""
    rows, cols, t = 128256, 4096, 14
    rng = np.random.default_rng(args.seed)
    raw = synth.quant_tensor(rng, t, rows, cols)
    xv = synth.activations(rng, cols)
    x = device.to_device_f32(xv)
    wbytes = rows * (cols // 256) * 210
    nbytes = wbytes + 4 * cols + 4 * rows
    copies = rotations(wbytes)
    log(f'vocab head: {copies} weight copies ({copies * wbytes / 1e6:.0f} MB)')
    mats = [device.QMat.from_ggml(raw, t, rows, cols) for _ in range(copies)]
    out = torch.empty(rows, dtype=torch.float32, device=device.device())
    stream = torch.cuda.Stream()
    ms = time_steps(torch, [lambda m=m: m.matvec(x, out=out, stream=stream) for m in mats], stream, args.steps,
                    args.warmup)
    if not torch.isfinite(out).all():
        raise SystemExit('non-finite vocabulary head output')
    for m in mats:
        m.close()
    gbs = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        from oracle import ref
        th = reference_threads(rows, t)
        cpu = cpu_runs(lambda n: ref.matvec(raw, xv, rows, cols, t, threads=th if n is None else n), th, nbytes,
                       'GB/s', 'localai_q6k_matvec', min_samples=5, budget_s=8)
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
            'data': 'synthetic (seeded GGML Q6_K bytes, fp32 N(0,1) x)',
            'config': {'workload': 'llama3_8b_vocab_head_q6k_128256x4096', 'algorithmic_bytes': nbytes,
                       'weight_copies_rotated': copies},
            'roofline': {'bound': 'hbm', 'kernel': 'gemv_mfma<Q6_K> 128256x4096', 'achieved': round(gbs, 1),
                         'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': round(gbs / HBM_PEAK_GBS, 4),
                         'traffic': measured_traffic('vocab_head', 'head'), 'us_per_launch': round(ms * 1e3, 3),
                         'bytes_per_launch': nbytes},
            'cpu_baseline': cpu}


def wl_legacy(args, torch, device, synth):
    """What LocalAI's own native_quant.matvec (engine/native_quant.py:102-126)
    sees with this library behind its ctypes binding: localai_q4k_matvec with
    host pointers at the ffn_gate shape, x uploaded and y downloaded by the
    call, the weights in a registered (GGUF-map-like) host range so their
    device copy is cached. Timed on the host around each synchronous call;
    the first, uploading call of an unregistered range is timed beside it."""
    import ctypes
    from localai_amd import _lib
    lib = _lib.load()
    rows, cols, t = 14336, 4096, 12
    rng = np.random.default_rng(args.seed)
    raw = np.frombuffer(synth.quant_tensor(rng, t, rows, cols), dtype=np.uint8).copy()
    xv = synth.activations(rng, cols)
    out = np.empty(rows, np.float32)
    u8, f32 = ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_float)
    rp, xp, op = raw.ctypes.data_as(u8), xv.ctypes.data_as(f32), out.ctypes.data_as(f32)
    nbytes = raw.nbytes + 4 * cols + 4 * rows

    def call():
        lib.localai_q4k_matvec(rp, xp, op, rows, cols, 8)
        if lib.localai_hip_last_status():
            raise SystemExit('legacy call failed: ' + lib.localai_hip_last_error().decode())
    t0 = time.perf_counter_ns()
    call()                                      # unregistered: upload + repack + matvec
    upload_us = (time.perf_counter_ns() - t0) / 1e3
    _lib.check(lib.localai_hip_register_host(ctypes.c_void_p(raw.ctypes.data), raw.nbytes))
    call()                                      # first registered call builds the cached copy
    samples = []
    for _ in range(max(50, args.steps)):
        t0 = time.perf_counter_ns()
        call()
        samples.append((time.perf_counter_ns() - t0) / 1e3)
    _lib.check(lib.localai_hip_unregister_host(ctypes.c_void_p(raw.ctypes.data)))
    if not np.isfinite(out).all():
        raise SystemExit('non-finite legacy output')
    us = float(np.median(samples))
    gbs = nbytes / (us * 1e-6) / 1e9
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        from oracle import ref
        th = reference_threads(rows, t)
        cpu = cpu_runs(lambda n: ref.matvec(raw, xv, rows, cols, t, threads=th if n is None else n), th, nbytes,
                       'GB/s', 'localai_q4k_matvec', min_samples=10, budget_s=5)
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': us / 1e3, 'us_per_layer': round(us, 2),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
            'data': 'synthetic (seeded GGML Q4_K bytes in host memory, fp32 N(0,1) x)',
            'config': {'workload': 'legacy_host_q4k_matvec_14336x4096', 'p90_us': round(float(np.percentile(samples, 90)), 2),
                       'unregistered_first_call_us': round(upload_us, 1), 'samples': len(samples)},
            'roofline': {'bound': 'hbm', 'kernel': 'whole host call',
                         'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                         'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': measured_traffic('q4k', 'gate'),
                         'us_per_launch': round(us, 2), 'bytes_per_launch': nbytes},
            'cpu_baseline': cpu}


def wl_q8_prefill(args, torch, device, synth):
    rows, cols, tokens = 14336, 4096, 512
    flops = 2 * rows * cols * tokens
    rng = np.random.default_rng(args.seed)
    raw = synth.quant_tensor(rng, 8, rows, cols)
    xh = synth.activations(rng, tokens, cols)
    x = device.to_device_f32(xh)
    wbytes = rows * (cols // 32) * 34
    copies = rotations(wbytes)
    log(f'building {copies} Q8_0 weight copies')
    mats = [device.QMat.from_ggml(raw, 8, rows, cols) for _ in range(copies)]
    out = torch.empty((tokens, rows), dtype=torch.float32, device=device.device())
    stream = torch.cuda.Stream()
    ms = time_steps(torch, [lambda m=m: m.matmul(x, out=out, stream=stream) for m in mats], stream,
                    max(10, args.steps // 4), max(3, args.warmup // 4))
    if not torch.isfinite(out).all():
        raise SystemExit('non-finite GEMM output')
    tfs = flops / (ms * 1e-3) / 1e12
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        from oracle import ref, quant
        srows = 224                      # 1/64 of the rows, all 512 tokens
        sub = raw[:srows * (cols // 32) * 34]
        th = reference_threads(rows, 8)
        sflops = 2 * srows * cols * tokens
        nrows = 1792                     # NumPy path: 1/8 of the rows

        def numpy_path():
            return xh @ quant.dequantize(raw[:nrows * (cols // 32) * 34], 8, (nrows, cols)).T
        cpu = cpu_runs(lambda t: ref.matmul(sub, xh, srows, cols, 8, threads=th if t is None else t), th, sflops,
                       'TFLOP/s', f'localai_q8_0_matmul, {srows} rows, us scaled',
                       scale_us=rows / srows, min_samples=3, budget_s=12,
                       numpy_call=numpy_path, numpy_work=2 * nrows * cols * tokens)
    return {'value': round(tfs, 2), 'unit': 'TFLOP/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'mfma_frac': round(tfs / MFMA_F16_PEAK_TFS, 4), 'dtype': 'f16 MFMA, fp32 accumulate',
            'data': 'synthetic (seeded GGML Q8_0 bytes, fp32 N(0,1) activations)',
            'config': {'workload': 'q8_0_prefill_gemm_14336x4096x512', 'tokens': tokens, 'flops': flops,
                       'weight_copies_rotated': copies},
            'roofline': {'bound': 'mfma', 'kernel': 'x_to_f16 + gemm_cu_q80 (call)',
                         'achieved': round(tfs, 1), 'peak': MFMA_F16_PEAK_TFS, 'unit': 'TFLOP/s',
                         'frac': round(tfs / MFMA_F16_PEAK_TFS, 4), 'traffic': measured_traffic('q8', 'gemm'),
                         'us_per_launch': round(ms * 1e3, 3), 'flops_per_launch': flops},
            'cpu_baseline': cpu}


def _moe_setup(args, synth, E, H, I, k, t, T, bias):
    rng = np.random.default_rng(args.seed)
    gu = synth.quant_tensor(rng, t, 2 * I, H, batch=E)
    dn = synth.quant_tensor(rng, t, H, I, batch=E)
    rw = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    h = synth.activations(rng, T, H)
    return gu, dn, rw, h


def _moe_gpu(args, torch, device, synth, E, H, I, k, t, T, bias, per_expert_bytes, label):
    from localai_amd.moe import MoELayer
    gu, dn, rw, h = _moe_setup(args, synth, E, H, I, k, t, T, bias)
    hd = device.to_device_f32(h)
    probe = MoELayer(rw, gu, dn, t, E, H, I, k, router_b=bias)
    _, idx, _ = probe.forward_device(hd)
    distinct = int(np.unique(idx.cpu().numpy()).size)
    touched = distinct * per_expert_bytes
    nbytes = touched + E * H * 4 + 2 * T * H * 4 + (E * 4 if bias is not None else 0)
    copies = rotations(touched)
    log(f'{label}: T={T}, {distinct} distinct experts, {copies} layer copies')
    layers = [probe] + [MoELayer(rw, gu, dn, t, E, H, I, k, router_b=bias) for _ in range(copies - 1)]
    stream = torch.cuda.Stream()
    out = torch.empty((T, H), dtype=torch.float32, device=device.device())
    oi = torch.empty((T, k), dtype=torch.int32, device=device.device())
    og = torch.empty((T, k), dtype=torch.float32, device=device.device())
    for L in layers:
        L.workspace(T)
    ms = time_steps(torch, [lambda L=L: L.forward_device(hd, out=out, idx=oi, gates=og, stream=stream)
                            for L in layers], stream, args.steps, args.warmup)
    if not torch.isfinite(out).all():
        raise SystemExit('non-finite MoE output')
    _moe_gpu.last = (layers, hd, stream)
    return ms, nbytes, distinct, copies, (gu, dn, rw, h, idx.cpu().numpy())


def experts1_roofline(args, torch, device, E, H, I, k, per_expert):
    """The fused one-token expert kernel (localai_hip_moe_experts1: gate_up
    and down of the chosen experts in one launch) timed alone over the rotated
    layer copies of the last _moe_gpu call, with its router's choice fixed."""
    import ctypes
    from localai_amd import _lib
    layers, hd, stream = _moe_gpu.last
    lib = _lib.load()
    _, idx, gates = layers[0].forward_device(hd)
    out = torch.empty(H, dtype=torch.float32, device=hd.device)
    sp = ctypes.c_void_p(int(stream.cuda_stream))

    def run(L):
        ws = L.workspace(1)
        _lib.check(lib.localai_hip_moe_experts1(device.ptr(hd), H, L.gate_up.handle, L.down.handle, k,
                                                device.ptr(idx), device.ptr(gates), -1, device.ptr(out),
                                                device.ptr(ws), ws.numel(), sp))
    ms = time_steps(torch, [lambda L=L: run(L) for L in layers], stream, args.steps, args.warmup)
    nbytes = k * per_expert + 2 * H * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {'bound': 'hbm', 'kernel': 'moe_decode1_kernel (2 experts)',
            'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': round(gbs / HBM_PEAK_GBS, 4),
            'traffic': measured_traffic('zaya', 'decode1'), 'us_per_launch': round(ms * 1e3, 3),
            'bytes_per_launch': nbytes}


def expert_gemm_roofline(args, torch, device, E, H, I, k, T, distinct):
    """The prefill layer's dominant kernel, the gate_up expert GEMM (with
    SiLU*up), run alone (localai_hip_moe_expert_gemm) on the routing tables
    each rotated layer copy's last forward left in its workspace. Its bytes:
    the gate_up weights of the touched experts, the f16 rows of h and the f16
    SiLU*up rows it writes for the down GEMM; its flops 2 * T * k * H * 2I.
    The binding roof is HBM (about 180 flop per byte against a ridge of about
    315)."""
    import ctypes
    from localai_amd import _lib
    layers, hd, stream = _moe_gpu.last
    lib = _lib.load()
    sp = ctypes.c_void_p(int(stream.cuda_stream))

    def run(L):
        ws = L.workspace(T)
        _lib.check(lib.localai_hip_moe_expert_gemm(L.gate_up.handle, L.down.handle, T, E, k, device.ptr(ws),
                                                   ws.numel(), 0, sp))
    kms = time_steps(torch, [lambda L=L: run(L) for L in layers], stream, args.steps, args.warmup)
    gu_bytes = 2 * I * (H // 256) * 144
    nbytes = distinct * gu_bytes + T * H * 2 + T * k * I * 2
    flops = 2 * T * k * H * 2 * I
    gbs = nbytes / (kms * 1e-3) / 1e9
    tfs = flops / (kms * 1e-3) / 1e12
    return {'bound': 'hbm', 'kernel': 'gate_up expert GEMM',
            'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': round(gbs / HBM_PEAK_GBS, 4),
            'traffic': measured_traffic('qwen3', 'gate_up'), 'us_per_launch': round(kms * 1e3, 3),
            'bytes_per_launch': nbytes, 'tflops': round(tfs, 1), 'mfma_frac': round(tfs / MFMA_F16_PEAK_TFS, 4)}


def _moe_cpu(gu, dn, rw, h, idx, E, H, I, k, t, T, bias, threads):
    """numpy router + the reference kernels per selected expert (engine/zaya.py:303-306)."""
    from oracle import ref
    from oracle.quant import block_layout
    block, bpb = block_layout(t)
    gub = 2 * I * (H // block) * bpb
    dnb = H * (I // block) * bpb
    gbuf, dbuf = np.frombuffer(gu, np.uint8), np.frombuffer(dn, np.uint8)

    def layer():
        logits = h @ rw.T + (bias if bias is not None else 0.0)
        sel = np.argsort(-logits, axis=1, kind='stable')[:, :k]
        out = np.zeros((T, H), np.float32)
        for e in np.unique(sel):
            toks = np.nonzero((sel == e).any(axis=1))[0]
            g_raw = gbuf[e * gub:(e + 1) * gub].tobytes()
            d_raw = dbuf[e * dnb:(e + 1) * dnb].tobytes()
            if len(toks) == 1:
                gu_o = ref.matvec(g_raw, h[toks[0]], 2 * I, H, t, threads=threads)[None]
            else:
                gu_o = ref.matmul(g_raw, h[toks], 2 * I, H, t, threads=threads)
            a = gu_o[:, :I] / (1.0 + np.exp(-np.clip(gu_o[:, :I], -80, 80))) * gu_o[:, I:]
            if len(toks) == 1:
                y = ref.matvec(d_raw, a[0].astype(np.float32), H, I, t, threads=threads)[None]
            else:
                y = ref.matmul(d_raw, a.astype(np.float32), H, I, t, threads=threads)
            sl = logits[toks][:, :]
            for j, tk in enumerate(toks):
                s = sel[tk]
                z = np.exp(logits[tk, s] - logits[tk, s].max())
                out[tk] += (z / z.sum())[list(s).index(e)] * y[j]
        return out
    return layer


def wl_zaya(args, torch, device, synth):
    E, H, I, k, t = 16, 2048, 4096, 2, 14
    per_expert = 2 * I * (H // 256) * 210 + H * (I // 256) * 210
    res = {}
    roof = None
    for T in (1, 8):
        ms, nbytes, distinct, copies, data = _moe_gpu(args, torch, device, synth, E, H, I, k, t, T, None,
                                                      per_expert, 'zaya')
        res[T] = (ms, nbytes, distinct, copies, data)
        if T == 1:
            roof = experts1_roofline(args, torch, device, E, H, I, k, per_expert)
        _moe_gpu.last = None
    ms, nbytes, distinct, copies, data = res[1]
    gbs = nbytes / (ms * 1e-3) / 1e9
    ms8, nb8, d8, _, _ = res[8]
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        gu, dn, rw, h, idx = data
        cpu = cpu_runs(lambda th: _moe_cpu(gu, dn, rw, h, idx, E, H, I, k, t, 1, None,
                                           threads=4 if th is None else th)(), 4, nbytes, 'GB/s',
                       'numpy router + localai_q6k_matvec',
                       min_samples=5, budget_s=8)
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
            'data': 'synthetic (seeded Q6_K experts, router N(0,0.02), h N(0,1))',
            'config': {'workload': 'zaya_moe_decode_h2048_e16_top2_i4096_q6k', 'tokens': 1,
                       'distinct_experts': distinct, 'algorithmic_bytes': nbytes, 'layer_copies_rotated': copies,
                       'tokens_8': {'us_per_layer': round(ms8 * 1e3, 3), 'distinct_experts': d8,
                                    'algorithmic_bytes': nb8,
                                    'GB/s': round(nb8 / (ms8 * 1e-3) / 1e9, 2)}},
            'roofline': roof, 'cpu_baseline': cpu}


def wl_moe_decode_shapes(args, torch, device, synth):
    """Decode (fewer than 32 tokens) of two more MoE shapes, not in the default
    run: Qwen3-MoE-like (hidden 2048, 128 Q4_K experts, top-8, intermediate
    768, Zipf router bias) at 1 and 4 tokens -- the router over (expert,
    token) one-wave workgroups, the top-k inside the permutation, the grouped
    i8 MFMA kernels and the combine -- and Mixtral-like (hidden 4096, 8 Q4_K
    experts, top-2, intermediate 14336: down rows of 56 blocks of 256, the
    streamed kernels) at 1 and 8 tokens."""
    per_q4 = lambda H, I: (2 * I * (H // 256) + H * (I // 256)) * 144   # noqa: E731
    cases = {}
    for name, (E, H, I, k, bias), Ts in (('qwen3_like', (128, 2048, 768, 8, synth.zipf_bias(128)), (1, 4)),
                                         ('mixtral_like', (8, 4096, 14336, 2, None), (1, 8))):
        for T in Ts:
            ms, nbytes, distinct, copies, _ = _moe_gpu(args, torch, device, synth, E, H, I, k, 12, T, bias,
                                                       per_q4(H, I), name)
            _moe_gpu.last = None
            cases[f'{name}_t{T}'] = {'us_per_layer': round(ms * 1e3, 3), 'distinct_experts': distinct,
                                     'algorithmic_bytes': nbytes, 'GB/s': round(nbytes / (ms * 1e-3) / 1e9, 1),
                                     'layer_copies_rotated': copies}
    first = cases['qwen3_like_t1']
    return {'value': first['GB/s'], 'unit': 'GB/s', 'ms_per_step': first['us_per_layer'] * 1e-3,
            'us_per_layer': first['us_per_layer'], 'hbm_frac': round(first['GB/s'] / HBM_PEAK_GBS, 4),
            'dtype': 'fp32', 'data': 'synthetic (seeded Q4_K experts, router N(0,0.02), h N(0,1))',
            'config': {'workload': 'moe_decode_qwen3_like_and_mixtral_like', 'cases': cases},
            'roofline': None, 'cpu_baseline': None}


def wl_qwen3(args, torch, device, synth):
    E, H, I, k, t, T = 128, 2048, 768, 8, 12, 512
    per_expert = 2 * I * (H // 256) * 144 + H * (I // 256) * 144
    bias = synth.zipf_bias(E)
    ms, nbytes, distinct, copies, data = _moe_gpu(args, torch, device, synth, E, H, I, k, t, T, bias,
                                                  per_expert, 'qwen3')
    roof = expert_gemm_roofline(args, torch, device, E, H, I, k, T, distinct)
    _moe_gpu.last = None
    flops = 2 * T * k * (H * 2 * I + I * H)
    gbs = nbytes / (ms * 1e-3) / 1e9
    tfs = flops / (ms * 1e-3) / 1e12
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        gu, dn, rw, h, idx = data
        th = reference_threads(2 * I, 12)
        cpu = cpu_runs(lambda t_: _moe_cpu(gu, dn, rw, h, idx, E, H, I, k, t, T, bias,
                                           threads=th if t_ is None else t_)(), th, flops, 'TFLOP/s',
                       'numpy router + localai_q4k_matmul',
                       min_samples=2, budget_s=12)
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'tflops': round(tfs, 2),
            'mfma_frac': round(tfs / MFMA_F16_PEAK_TFS, 4), 'dtype': 'fp32 / f16 MFMA',
            'data': 'synthetic (seeded Q4_K experts, router N(0,0.02) + Zipf(1.1) logit bias, h N(0,1))',
            'config': {'workload': 'qwen3_moe_prefill_h2048_e128_top8_i768_q4k_t512', 'tokens': T,
                       'distinct_experts': distinct, 'algorithmic_bytes': nbytes, 'flops': flops,
                       'layer_copies_rotated': copies},
            'roofline': roof, 'cpu_baseline': cpu}


def wl_chain(args, torch, device, synth):
    """The decode layer's seven matvecs with the glue between them
    (localai_hip_layer_chain): o + residual, RMSNorm + gate/up, SiLU*up +
    down + residual, RMSNorm + next layer's q/k/v + RoPE. The value is the
    default form, four launches with the glue fused into the matvecs; the
    one-launch form (device-side waits between the stages) is timed beside
    it."""
    from localai_amd.layer import DecodeLayerChain, set_mode
    layer = synth.LLAMA3_8B_LAYER
    layer_bytes = synth.layer_algorithmic_bytes()
    copies = rotations(synth.layer_weight_bytes())
    rng = np.random.default_rng(args.seed)
    host = {name: synth.quant_tensor(rng, t, rows, cols) for name, t, rows, cols, _ in layer}
    pre = device.to_device_f32(synth.activations(rng, 4096))
    att = device.to_device_f32(synth.activations(rng, 4096))
    w1 = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    w2 = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    log(f'chain: building {copies} layer copies')
    chains = [DecodeLayerChain({n: device.QMat.from_ggml(host[n], t, r, c) for n, t, r, c, _ in layer}, w1, w2,
                               1e-5, head_dim=128) for _ in range(copies)]
    stream = torch.cuda.Stream()
    inv = 1.0 / (500000.0 ** (np.arange(64, dtype=np.float32) / 64))
    rope = (device.to_device_f32(np.cos(np.float32(37) * inv).astype(np.float32)),
            device.to_device_f32(np.sin(np.float32(37) * inv).astype(np.float32)))
    outs = tuple(torch.empty_like(o) for o in chains[0].forward_device(pre, att, rope=rope))
    torch.cuda.synchronize()
    steps = [lambda c=c: c.forward_device(pre, att, rope=rope, out=outs, stream=stream) for c in chains]
    set_mode(True)
    try:
        ms1 = time_steps(torch, steps, stream, args.steps, args.warmup)
        chains[0].check(stream)
    finally:
        set_mode(False)
    ms = time_steps(torch, steps, stream, args.steps, args.warmup)
    gbs = layer_bytes / (ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_baseline != 'off' and ref_ok():
        cpu = cpu_runs(_chain_cpu(host, layer, rng, w1, w2), max(reference_threads(r, t) for _, t, r, _, _ in layer),
                       layer_bytes, 'GB/s', '7 localai_*_matvec + NumPy glue', min_samples=10,
                       budget_s=6)
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
            'data': 'synthetic (seeded GGML Q4_K/Q6_K bytes, fp32 N(0,1) activations, norm weights U(0.5,1.5))',
            'config': {'workload': 'llama3_8b_decode_layer_chain_rope', 'algorithmic_bytes_per_layer': layer_bytes,
                       'weight_copies_rotated': copies},
            'one_launch': {'us_per_layer': round(ms1 * 1e3, 3),
                           'GB/s': round(layer_bytes / (ms1 * 1e-3) / 1e9, 1)},
            'roofline': {'bound': 'hbm', 'kernel': '4 glued matvec launches', 'achieved': round(gbs, 1),
                         'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': None,
                         'us_per_launch': round(ms * 1e3, 3), 'bytes_per_launch': layer_bytes},
            'cpu_baseline': cpu}


def _chain_cpu(host, layer, rng, w1, w2):
    """The reference's decode-layer step on the CPU: its seven native matvecs
    (reference thread policy) with the float32 NumPy glue of
    engine/model.py:181-233 between them (residual adds, RMSNorm :82,
    SiLU * up, RoPE of q and k)."""
    from oracle import ref
    x0 = synth_act(rng, 4096)
    att = synth_act(rng, 4096)
    cos = np.cos(np.arange(64, dtype=np.float32) * 0.01).astype(np.float32)
    sin = np.sin(np.arange(64, dtype=np.float32) * 0.01).astype(np.float32)
    info = {n: (t, r, c) for n, t, r, c, _ in layer}

    def mv(name, x, th):
        t, r, c = info[name]
        return ref.matvec(host[name], x, r, c, t, threads=reference_threads(r, t) if th is None else th)

    def norm(x, w):
        return x * (1.0 / np.sqrt(np.mean(x * x) + np.float32(1e-5))) * w

    def rope(v):                 # adjacent pairs per 128-wide head (engine/model.py:83-100, llama)
        v = v.reshape(-1, 64, 2)
        a, b = v[..., 0], v[..., 1]
        return np.stack([a * cos - b * sin, a * sin + b * cos], axis=-1).reshape(-1)

    def step(th):
        x1 = x0 + mv('attn_output', att, th)
        h = norm(x1, w1)
        g, u = mv('ffn_gate', h, th), mv('ffn_up', h, th)
        x2 = x1 + mv('ffn_down', (g / (1.0 + np.exp(-g)) * u).astype(np.float32), th)
        h2 = norm(x2, w2)
        return rope(mv('attn_q', h2, th)), rope(mv('attn_k', h2, th)), mv('attn_v', h2, th)
    return step


def synth_act(rng, n):
    return rng.standard_normal(n).astype(np.float32)


def wl_floor(args, torch, device, synth):
    """Streaming-read floors (localai_hip_stream_read): what one launch of a
    given size can read at best, rotated beyond the Infinity Cache like the
    matvec workloads."""
    from localai_amd import _lib
    lib = _lib.load()
    segs = {'qkv': 9469952 + 2379776 + 3461120, 'o': 9469952, 'gate_up': 2 * 33030144, 'down': 48168960}
    segs = {k: v - v % 16 for k, v in segs.items()}
    layer = sum(segs.values())
    copies = rotations(layer)
    bufs = [torch.empty(layer, dtype=torch.uint8, device=device.device()).fill_(i + 1) for i in range(copies)]
    out = torch.zeros(4, dtype=torch.int32, device=device.device())
    stream = torch.cuda.Stream()
    sp = lambda: ctypes_stream(stream)   # noqa: E731

    def read(buf, off, n):
        _lib.check(lib.localai_hip_stream_read(device.ptr(buf) + off, n, device.ptr(out), sp()))

    def per_layer_chain(buf):
        off = 0
        for name in ('qkv', 'o', 'gate_up', 'down'):
            read(buf, off, segs[name])
            off += segs[name]
    res = {}
    ms = time_steps(torch, [lambda b=b: read(b, 0, 33030144) for b in bufs], stream, args.steps, args.warmup)
    res['one_launch_33MB'] = {'us': round(ms * 1e3, 3), 'GB/s': round(33030144 / (ms * 1e-3) / 1e9, 1),
                              'frac': round(33030144 / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    # each of the four alone: the floor of that launch of the chain
    res['per_launch_us'] = {}
    off = 0
    for name in ('qkv', 'o', 'gate_up', 'down'):
        ms = time_steps(torch, [lambda b=b, o=off, n=segs[name]: read(b, o, n) for b in bufs], stream, args.steps,
                        args.warmup)
        res['per_launch_us'][name] = round(ms * 1e3, 3)
        off += segs[name]
    ms = time_steps(torch, [lambda b=b: per_layer_chain(b) for b in bufs], stream, args.steps, args.warmup)
    res['layer_as_four_launches'] = {'us': round(ms * 1e3, 3), 'GB/s': round(layer / (ms * 1e-3) / 1e9, 1),
                                     'frac': round(layer / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                     'bytes': segs}
    ms1 = time_steps(torch, [lambda b=b: read(b, 0, layer) for b in bufs], stream, args.steps, args.warmup)
    gbs = layer / (ms1 * 1e-3) / 1e9
    res['layer_as_one_launch'] = {'us': round(ms1 * 1e3, 3), 'GB/s': round(gbs, 1),
                                  'frac': round(gbs / HBM_PEAK_GBS, 4)}
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms1, 'hbm_frac': round(gbs / HBM_PEAK_GBS, 4),
            'dtype': 'u8', 'data': 'constant bytes', 'floors': res,
            'config': {'workload': 'hbm_stream_read', 'bytes_per_layer': layer, 'copies_rotated': copies},
            'roofline': {'bound': 'hbm', 'kernel': 'stream_read_kernel', 'achieved': round(gbs, 1),
                         'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': None},
            'cpu_baseline': None}


def _cpu_port(fn, work, unit, sample):
    """A NumPy restatement of the reference's own code for a path with no
    compiled reference kernel here, timed on all physical cores (pinned)."""
    div = 1e9 if unit == 'GB/s' else 1e12
    allc = host()['physical_cores']
    with pinned(allc):
        us, n = time_cpu(fn, min_samples=5, budget_s=6)
    return {'value': sig(work / (us * 1e-6) / div), 'unit': unit, 'cores': allc, 'kind': 'port',
            'sample': sample, 'us': round(us, 1), 'samples': n}


def wl_attention(args, torch, device, synth):
    """Llama-3-8B decode attention at context 4096 (localai_hip_attention_decode):
    32 query heads over 8 kv heads of head_dim 128, fp32 cache, the token at
    position 4095 (its k / v row written into the cache by the same call)."""
    from localai_amd import attention
    from oracle import attention as oatt
    nh, nkv, hd, ctx = 32, 8, 128, 4096
    pos = ctx - 1
    rng = np.random.default_rng(args.seed)
    row = nkv * hd * 4
    nbytes = 2 * pos * row + 2 * row + nh * hd * 4 + 2 * row + nh * hd * 4
    copies = rotations(2 * ctx * row)
    kc = rng.standard_normal((ctx, nkv, hd)).astype(np.float32)
    vc = rng.standard_normal((ctx, nkv, hd)).astype(np.float32)
    qv = rng.standard_normal(nh * hd).astype(np.float32)
    kn = rng.standard_normal(nkv * hd).astype(np.float32)
    vn = rng.standard_normal(nkv * hd).astype(np.float32)
    log(f'attention: {copies} cache copies ({copies * 2 * ctx * row / 1e6:.0f} MB)')
    kd, vd = torch.from_numpy(kc).to(device.device()), torch.from_numpy(vc).to(device.device())
    caches = []
    for _ in range(copies):
        c = attention.KVCache(1, nkv, hd, ctx, n_heads=nh)
        c.k[0].copy_(kd)
        c.v[0].copy_(vd)
        caches.append(c)
    del kd, vd
    q, k, v = (device.to_device_f32(a) for a in (qv, kn, vn))
    out = torch.empty(nh * hd, dtype=torch.float32, device=device.device())
    stream = torch.cuda.Stream()
    ms = time_steps(torch, [lambda c=c: attention.attention_decode(q, k, v, c, 0, pos, nh, out=out, stream=stream)
                            for c in caches], stream, args.steps, args.warmup)
    want, kc2, vc2 = oatt.gqa_decode(qv, kc, vc, pos, nh, nkv, hd, k_new=kn, v_new=vn)
    got = out.cpu().numpy()
    err = float(np.abs(got - want).max() / np.abs(want).max())
    if not err <= 2e-5:
        raise SystemExit(f'attention output off by {err:.2e} (normwise)')
    gbs = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_baseline != 'off':
        cpu = _cpu_port(lambda: oatt.gqa_decode_f32(qv, kc2, vc2, pos, nh, nkv, hd), nbytes, 'GB/s',
                        'model.py:223-227 NumPy f32')
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
            'data': 'synthetic (N(0,1) fp32 cache, q, k, v)',
            'config': {'workload': 'llama3_8b_attention_decode_ctx4096', 'n_heads': nh, 'n_kv_heads': nkv,
                       'head_dim': hd, 'positions': ctx, 'algorithmic_bytes': nbytes, 'layer_copies_rotated': copies,
                       'normwise_vs_oracle': err},
            'roofline': {'bound': 'hbm', 'kernel': 'attn_chunk + attn_merge (call)',
                         'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                         'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': measured_traffic('attention', 'chunk'),
                         'us_per_launch': round(ms * 1e3, 3), 'bytes_per_launch': nbytes},
            'cpu_baseline': cpu}


def wl_delta_net(args, torch, device, synth):
    """Qwen3.5 gated delta-net step (localai_hip_delta_net_step) at the
    default linear-attention shape: 32 value heads, key and value dim 128."""
    from localai_amd import attention
    from oracle import attention as oatt
    heads, kd, vd = 32, 128, 128
    rng = np.random.default_rng(args.seed)
    sbytes = heads * kd * vd * 4
    nbytes = 2 * sbytes + (2 * heads * kd + 2 * heads * vd + 2 * heads) * 4
    copies = rotations(2 * sbytes)
    st = (rng.standard_normal((heads, kd, vd)) * 0.1).astype(np.float32)
    qv = rng.standard_normal((heads, kd)).astype(np.float32)
    kv = rng.standard_normal((heads, kd)).astype(np.float32)
    qv /= np.linalg.norm(qv, axis=1, keepdims=True) * np.sqrt(kd)
    kv /= np.linalg.norm(kv, axis=1, keepdims=True)
    vv = rng.standard_normal((heads, vd)).astype(np.float32)
    decay = -rng.uniform(0.001, 0.1, heads).astype(np.float32)
    beta = rng.uniform(0.1, 0.9, heads).astype(np.float32)
    states = [device.to_device_f32(st) for _ in range(copies)]
    q, k, v, dc, bt = (device.to_device_f32(a) for a in (qv, kv, vv, decay, beta))
    core = torch.empty((heads, vd), dtype=torch.float32, device=device.device())
    check = device.to_device_f32(st)
    attention.delta_net_step(check, q, k, v, dc, bt, core=core)
    S, want = oatt.delta_net_step(st, qv, kv, vv, decay, beta)
    torch.cuda.synchronize()
    if not (np.array_equal(core.cpu().numpy(), want) and np.array_equal(check.cpu().numpy(), S)):
        raise SystemExit('delta net step differs from the float32 reference loop')
    stream = torch.cuda.Stream()
    ms = time_steps(torch, [lambda s_=s_: attention.delta_net_step(s_, q, k, v, dc, bt, core=core, stream=stream)
                            for s_ in states], stream, args.steps, args.warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_baseline != 'off':
        cpu = _cpu_port(lambda: oatt.delta_net_step(st, qv, kv, vv, decay, beta), nbytes, 'GB/s',
                        'numba_kernels.py:11-45 NumPy f32')
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'us_per_layer': round(ms * 1e3, 3),
            'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'dtype': 'fp32',
            'data': 'synthetic (state N(0, 0.01), L2-normalised q / k as engine/qwen35.py:206-208)',
            'config': {'workload': 'qwen35_delta_net_step_h32_k128_v128', 'heads': heads, 'key_dim': kd,
                       'value_dim': vd, 'algorithmic_bytes': nbytes, 'layer_copies_rotated': copies,
                       'bit_exact_vs_reference_loop': True},
            'roofline': {'bound': 'hbm', 'kernel': 'delta_net_kernel<128>', 'achieved': round(gbs, 1),
                         'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': round(gbs / HBM_PEAK_GBS, 4),
                         'traffic': measured_traffic('delta_net', 'step'), 'us_per_launch': round(ms * 1e3, 3),
                         'bytes_per_launch': nbytes},
            'cpu_baseline': cpu}


def ctypes_stream(stream):
    import ctypes
    return ctypes.c_void_p(int(stream.cuda_stream))


def wl_copy(args, torch, device, synth):
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device=device.device()).fill_(1)
    dst = torch.empty_like(src)
    stream = torch.cuda.Stream()
    g = capture(torch, lambda: dst.copy_(src), stream)
    ms = time_graphs(torch, [g], stream, args.steps, args.warmup)
    gbs = 2 * n / (ms * 1e-3) / 1e9
    return {'value': round(gbs, 2), 'unit': 'GB/s', 'ms_per_step': ms, 'hbm_frac': round(gbs / HBM_PEAK_GBS, 4),
            'dtype': 'u8', 'data': 'constant bytes',
            'config': {'workload': 'hbm_copy_256MiB', 'read_bytes': n, 'write_bytes': n},
            'roofline': {'bound': 'hbm', 'kernel': 'torch copy', 'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS,
                         'unit': 'GB/s', 'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': None},
            'cpu_baseline': None}


FUNCS = {'llama3_8b_decode_layer': 'wl_layer', 'q4k_matvec': 'wl_q4k', 'q8_0_matvec': 'wl_q8_matvec',
         'vocab_head': 'wl_vocab_head', 'legacy_host_matvec': 'wl_legacy',
         'q8_0_prefill': 'wl_q8_prefill',
         'zaya_moe_decode': 'wl_zaya', 'qwen3_moe_prefill': 'wl_qwen3', 'llama3_8b_layer_chain': 'wl_chain',
         'hbm_read_floor': 'wl_floor', 'hbm_copy': 'wl_copy', 'llama3_8b_attention_decode': 'wl_attention',
         'qwen35_delta_net_step': 'wl_delta_net', 'moe_decode_shapes': 'wl_moe_decode_shapes'}


def run_workload(name, args, torch, device, synth):
    DIST.clear()
    r = globals()[FUNCS[name]](args, torch, device, synth)
    if DIST and 'step_stats' not in r:
        r['step_stats'] = DIST[0]
    return r


# extra per-workload figures kept in the one-line record (path into the
# full record -> short key)
EXTRAS = {
    'llama3_8b_decode_layer': [(('us_per_layer_one_launch_per_matvec',), 'us_one_launch_per_matvec')],
    'zaya_moe_decode': [(('config', 'tokens_8', 'us_per_layer'), 'us_t8'), (('config', 'tokens_8', 'GB/s'), 'gbs_t8'),
                        (('config', 'distinct_experts'), 'experts_t1'),
                        (('config', 'tokens_8', 'distinct_experts'), 'experts_t8')],
    'qwen3_moe_prefill': [(('tflops',), 'tflops'), (('mfma_frac',), 'mfma_frac'),
                          (('config', 'distinct_experts'), 'experts')],
    'llama3_8b_layer_chain': [(('one_launch', 'us_per_layer'), 'us_one_launch')],
    'legacy_host_matvec': [(('config', 'unregistered_first_call_us'), 'us_unregistered_first_call')],
    'hbm_read_floor': [(('floors', 'one_launch_33MB', 'us'), 'us_33MB'),
                       (('floors', 'layer_as_four_launches', 'us'), 'us_layer_4_launches'),
                       (('floors', 'layer_as_one_launch', 'us'), 'us_layer_1_launch')],
}


def _dig(d, path):
    for k in path:
        if not isinstance(d, dict) or k not in d:
            return None
        d = d[k]
    return d


def compact_roofline(rl):
    if not rl:
        return None
    out = {k: rl.get(k) for k in ('bound', 'achieved', 'peak', 'unit', 'frac', 'traffic')}
    out['achieved'] = sig(out['achieved'])
    out['kernel'] = rl.get('kernel')
    out['us'] = sig(rl.get('us_per_launch'))
    for k in ('tflops', 'mfma_frac'):
        if k in rl:
            out[k] = rl[k]
    return out


def compact_cpu(cb):
    if not cb:
        return None
    out = {k: cb.get(k) for k in ('value', 'unit', 'cores', 'kind', 'sample')}
    out['us'] = round(cb['us']) if cb.get('us') is not None else None
    return out


def compact(name, r):
    """One workload in the one-line record: time, value, fraction of its
    roof, the roofline of its dominant kernel and the CPU baseline (the
    full record goes to stderr)."""
    c = {'us': sig(r.get('us_per_layer', r['ms_per_step'] * 1e3)),
         'value': sig(r['value']), 'unit': r['unit'],
         'frac': r.get('mfma_frac') if r['unit'] == 'TFLOP/s' else r.get('hbm_frac')}
    for path, key in EXTRAS.get(name, []):
        v = _dig(r, path)
        if v is not None:
            c[key] = sig(v) if isinstance(v, float) else v
    c['roofline'] = compact_roofline(r.get('roofline'))
    c['cpu_baseline'] = compact_cpu(r.get('cpu_baseline'))
    return c


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
    name = args.workload or 'llama3_8b_decode_layer'
    log(f'workload {name}')
    r = run_workload(name, args, torch, device, synth)
    full = {}
    if args.workload is None:
        for other in DEFAULT_SUITE:
            log(f'workload {other}')
            w = run_workload(other, args, torch, device, synth)
            w['ms_per_step'] = round(w['ms_per_step'], 6)
            full[other] = w
            torch.cuda.empty_cache()
    ms = r['ms_per_step']
    line = {'metric': METRIC, 'value': r['value'], 'unit': r['unit'], 'n_gpus': 1, 'steps': args.steps,
            'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'higher_is_better': True, 'scaling': 'weak',
            'vs_baseline': None, 'dtype': r.get('dtype'), 'data': r.get('data'),
            'config': {k: v for k, v in r.get('config', {}).items() if not isinstance(v, (list, dict)) and k != 'launch'}}
    head = compact(name, r)
    for k in ('value', 'unit'):
        head.pop(k)
    line.update(head)
    if args.cpu_baseline != 'off':
        h = host()
        line['host'] = f"{h['model']}, {h['physical_cores']} physical cores"
    if full:
        line['workloads'] = {k: compact(k, v) for k, v in full.items()}
    # the full record (step statistics, all-core and NumPy CPU legs, shapes)
    # on stderr, then the one line on stdout
    detail = dict(r, workloads=full)
    print('[bench] detail ' + json.dumps(detail, default=str), file=sys.stderr, flush=True)
    print(json.dumps(line, separators=(',', ':')), flush=True)


if __name__ == '__main__':
    main()
