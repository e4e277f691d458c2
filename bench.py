"""Benchmark: synthetic 40-layer MoE-FFN stack on one MI355X.

One step = one request of the headline workload: a 4096-token prefill in two
2048-token chunks (W8A16 grouped MFMA GEMMs; the second chunk runs one layer
behind the first on a second stream, both 40-layer passes replayed as one HIP
graph) followed by 33 serial decode tokens (W8A8 expert
GEMVs, the 40-layer decode step replayed as a HIP graph), over random-init
int8 group-128 weights (~33.4 GB) resident in HBM, plus the 16-row tile-layout
copy of the int8 bank (~32.4 GB) that the prefill grouped GEMMs read.

Prints one JSON line.  value = prefill tok/s; decode tok/s, decode HBM GB/s
and the roofline of the dominant kernel ride along.  Per-kernel times come
from HIP events recorded on the launch stream inside the timed steps, around
one extra eager prefill chunk and one extra eager decode token per step
(graphs cannot hold event records); those two are timed apart from tok/s.
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
INT8_PEAK_TOPS = 5033.2
PREFILL_TOKENS, CHUNK, DECODE_TOKENS = 4096, 2048, 33
H, I, E, K = 2048, 512, 256, 8
GU_EXPERT_BYTES = 2 * I * H + 2 * I * (H // 128) * 4        # 2,162,688
DN_EXPERT_BYTES = H * I + H * (I // 128) * 4                # 1,081,344
EXPERT_BYTES = GU_EXPERT_BYTES + DN_EXPERT_BYTES            # 3,244,032
DECODE_LAYER_BYTES = 9 * EXPERT_BYTES + E * H * 2 + H * 2   # 30,248,960
PREFILL_PHASES = ['norm_gate', 'router_logits', 'topk', 'route_plan', 'gate_up', 'down',
                  'combine']
DECODE_PHASES = ['decode_router', 'decode_gate_up', 'decode_down']


def parse():
    p = argparse.ArgumentParser()
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=3)
    p.add_argument('--warmup', type=int, default=2)
    p.add_argument('--layers', type=int, default=40)
    p.add_argument('--no-cpu-baseline', action='store_true')
    p.add_argument('--cpu-decode-tokens', type=int, default=DECODE_TOKENS,
                   help='decode tokens the CPU baseline runs through all layers (default: all 33)')
    p.add_argument('--no-events', action='store_true',
                   help='time whole steps only (no per-phase HIP events)')
    p.add_argument('--copy-probe', action='store_true',
                   help='only run a plain streaming kernel over 256 MiB (torch.neg on int32, '
                        'five launches): the known-size reference for HBM traffic counters')
    p.add_argument('--power-probe', action='store_true',
                   help='only replay the two-chunk prefill graph back to back for about 6 s while '
                        'sampling the board power and graphics clocks with amd-smi; also time '
                        'replays that follow a 30 ms idle gap')
    return p.parse_args()


def copy_probe(dev):
    n = 64 << 20  # int32 elements: 256 MiB read and 256 MiB written per launch
    src = torch.ones(n, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({'copy_probe': 'torch.neg int32', 'bytes_read_per_launch': n * 4,
                      'bytes_written_per_launch': n * 4, 'launches': 5}), flush=True)


def power_probe(stack, dev, seconds=6.0):
    """Board power and graphics clocks while the two-chunk prefill graph
    replays back to back, then while the 40-layer decode step does (amd-smi
    sampled from a host thread), and the prefill replay time back to back
    against after a 30 ms idle gap.  Prints one JSON line."""
    import subprocess
    import threading
    x = torch.randn((PREFILL_TOKENS, H), device=dev).to(torch.bfloat16)
    pst = x.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack.prefill_(pst.clone(), CHUNK)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack.prefill_(pst, CHUNK)
    torch.cuda.synchronize()
    samples, phase, stop = [], ['idle'], [False]

    def sample():
        while not stop[0]:
            try:
                out = subprocess.run(['amd-smi', 'metric', '-g', '0', '-p', '-c', '--json'],
                                     capture_output=True, text=True, timeout=5).stdout
                d = json.loads(out)
                d = d['gpu_data'][0] if isinstance(d, dict) and 'gpu_data' in d else d[0]
                clk = d['clock']
                gfx = [v['clk']['value'] for k, v in clk.items() if k.startswith('gfx_')
                       and isinstance(v, dict) and isinstance(v.get('clk'), dict)
                       and isinstance(v['clk'].get('value'), (int, float))]
                pw = d['power']['socket_power']
                samples.append((phase[0], min(gfx), max(gfx),
                                pw['value'] if isinstance(pw, dict) else pw))
            except Exception as e:  # no amd-smi, or another output format
                samples.append((phase[0], None, None, repr(e)[:80]))
            time.sleep(0.05)

    th = threading.Thread(target=sample)
    th.start()
    time.sleep(1.0)
    phase[0] = 'prefill'
    ev = []
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            a, b = make_events(2)
            a.record()
            pst.copy_(x)
            graph.replay()
            b.record()
            ev.append((a, b))
        torch.cuda.synchronize()
    # the 40-layer decode step, replayed back to back for comparison
    tok = torch.randn((1, H), device=dev).to(torch.bfloat16)
    dst = tok.clone()
    with torch.cuda.stream(side):
        stack.forward(dst.clone())
    torch.cuda.current_stream().wait_stream(side)
    dgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(dgraph):
        stack.forward(dst)
    torch.cuda.synchronize()
    phase[0] = 'decode'
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds / 2:
        for _ in range(100):
            dst.copy_(tok)
            dgraph.replay()
        torch.cuda.synchronize()
    phase[0] = 'after'
    time.sleep(1.0)
    stop[0] = True
    th.join()
    back_to_back = sorted(a.elapsed_time(b) for a, b in ev)
    gapped = []
    for _ in range(10):
        time.sleep(0.03)
        a, b = make_events(2)
        a.record()
        pst.copy_(x)
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        gapped.append(a.elapsed_time(b))
    gapped.sort()

    def stats(tag):
        rows = [r for r in samples if r[0] == tag and r[1] is not None]
        if not rows:
            return None
        pw = sorted(r[3] for r in rows)
        lo = sorted(r[1] for r in rows)  # per sample, the slowest of the XCDs' clocks
        return {'samples': len(rows), 'gfx_mhz_min': lo[0], 'gfx_mhz_median': lo[len(lo) // 2],
                'gfx_mhz_max': max(r[2] for r in rows), 'socket_w_median': pw[len(pw) // 2],
                'socket_w_max': pw[-1]}
    print(json.dumps({'power_probe': 'two-chunk prefill graph replayed back to back',
                      'replays': len(ev),
                      'replay_ms_median': round(back_to_back[len(back_to_back) // 2], 3),
                      'replay_ms_after_30ms_idle_median': round(gapped[len(gapped) // 2], 3),
                      'idle': stats('idle'), 'prefill': stats('prefill'), 'decode': stats('decode'),
                      'errors': sorted({r[3] for r in samples if r[1] is None})[:3]}), flush=True)


def log(msg):
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


class HipEvent:
    """Timing-only HIP event created with hipEventDisableSystemFence: its
    record skips the system-scope cache writeback and invalidation a default
    event performs, which would otherwise add microseconds to every short
    kernel it brackets.  `cuda_event` is the raw handle that the library's
    phase-event argument takes."""
    _hip = None

    @classmethod
    def hip(cls):
        if cls._hip is None:
            import ctypes
            try:
                cls._hip = ctypes.CDLL('libamdhip64.so')
            except OSError:
                cls._hip = ctypes.CDLL('/opt/rocm/lib/libamdhip64.so')
            cls._hip.hipEventCreateWithFlags.argtypes = [ctypes.c_void_p, ctypes.c_uint]
            cls._hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            cls._hip.hipEventElapsedTime.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                                     ctypes.c_void_p]
        return cls._hip

    def __init__(self):
        import ctypes
        self._ct = ctypes
        handle = ctypes.c_void_p()
        if self.hip().hipEventCreateWithFlags(ctypes.byref(handle), 0x20000000):
            raise RuntimeError('hipEventCreateWithFlags failed')
        self.cuda_event = handle.value

    def record(self):
        if self.hip().hipEventRecord(self.cuda_event, torch.cuda.current_stream().cuda_stream):
            raise RuntimeError('hipEventRecord failed')

    def elapsed_time(self, end):
        ms = self._ct.c_float()
        if self.hip().hipEventElapsedTime(self._ct.byref(ms), self.cuda_event, end.cuda_event):
            raise RuntimeError('hipEventElapsedTime failed')
        return ms.value


def make_events(n):
    return [HipEvent() for _ in range(n)]


def pmc_traffic():
    """HBM bytes per launch of each kernel from the rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes, already scaled by the copy-kernel calibration, as
    recorded in profiles/pmc_traffic.txt (lines 'kernel bytes')."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'profiles', 'pmc_traffic.txt')
    table = {}
    if os.path.exists(path):
        for line in open(path):
            parts = line.split()
            if len(parts) == 2 and not line.startswith('#') and parts[1].isdigit():
                table[parts[0]] = int(parts[1])
    return table


def prefill_bytes(active, tokens=CHUNK):
    routes = tokens * K
    return {
        'gate_up': (active + 1) * GU_EXPERT_BYTES + tokens * H * 2 + (routes + tokens) * I * 2,
        'down': (active + 1) * DN_EXPERT_BYTES + (routes + tokens) * I * 2
        + (routes + tokens) * H * 2,
    }


def prefill_flops(tokens=CHUNK):
    rows = tokens * K + tokens
    return {'gate_up': 2.0 * rows * 2 * I * H, 'down': 2.0 * rows * H * I}


LM_HEAD_N = 248320  # vocabulary of the 35B-A3B configuration


def lm_head_probe(dev, reps=20):
    """The lm_head W8A16 GEMV of one decode token: y [1, 248320] =
    x [1, 2048] . bf16(q * s)^T over a random int8 [248320, 2048] weight with
    fp32 group-128 scales (the largest dense read of a real decode step, run
    through int8.linear).  Returns its average time and HBM rate."""
    from localmoe35ba3b_amd.operators.int8 import linear
    n, k = LM_HEAD_N, H
    q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev)
    s = torch.rand((n, k // 128), device=dev) * 1e-3 + 1e-5
    x = torch.randn((1, k), device=dev).to(torch.bfloat16)
    for _ in range(3):
        linear(x, q, s)
    ev = make_events(reps + 1)
    ev[0].record()
    for i in range(reps):
        linear(x, q, s)
        ev[i + 1].record()
    torch.cuda.synchronize()
    us = sorted(ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(reps))[reps // 2]
    nbytes = n * k + n * (k // 128) * 4 + k * 2 + n * 2
    return {'avg_us': round(us, 2), 'launches': reps, 'bytes_per_launch': nbytes,
            'gbs': round(nbytes / us / 1e3, 1), 'hbm_frac': round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            'shape': f'[1, {k}] x [{n}, {k}] int8 g128'}


def isolated_probe(dev, spin_cycles, reps=32):
    """The single-kernel configurations of the workload, each timed on its own
    with per-launch HIP events behind a spin kernel that holds the stream
    until every launch is queued (so the events see the launches back to
    back, not the host's launch gaps); medians over the launches.  The
    HBM-bound cases rotate over weight copies of at least 512 MB in total,
    twice the 256 MB Infinity Cache, so every launch streams its weights from
    HBM.  Covers the dense W8A16 linear [4096, 2048] at 1 and 2048 rows, the
    W8A8 gate_up + SwiGLU [1024, 2048] at 1, 4 and 8 rows, and the int8 MFMA
    W8A8 GEMM at 2048 x 4096 x 2048 (the one-token MoE layer is the stack's
    decode layer, timed per kernel in the request).  The GEMVs also report
    `graph_us`, the per-launch time of 64 launches replayed as one HIP graph,
    and `launch_floor` gives both timings of a one-element fill: per-launch
    events cost about as much as a short kernel itself.
    `w8a8_gate_up_swiglu_m8_over_m1` is the 8-row time over the one-row time,
    in both timings."""
    from localmoe35ba3b_amd.convert import quantize_g128
    from localmoe35ba3b_amd.operators import int8, w8a8
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    def run(fn, n):  # spin_cycles: about 12 ms, longer than queueing n launches takes
        fn(0)
        torch.cuda.synchronize()
        ev = make_events(n + 1)
        torch.cuda._sleep(spin_cycles)
        ev[0].record()
        for i in range(n):
            fn(i)
            ev[i + 1].record()
        torch.cuda.synchronize()
        return sorted(ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(n))[n // 2]

    def run_graph(fn, n, replays=5):
        """Per-launch time of n launches captured as one HIP graph, the way a
        decode step replays them: median over replays of (replay time / n)."""
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            fn(0)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(replays):
            ev = make_events(2)
            ev[0].record()
            g.replay()
            ev[1].record()
            torch.cuda.synchronize()
            ts.append(ev[0].elapsed_time(ev[1]) * 1e3 / n)
        return sorted(ts)[replays // 2]

    def hbm(us, nbytes, shape, graph_us=None):
        r = {'avg_us': round(us, 2), 'bytes_per_launch': nbytes,
             'gbs': round(nbytes / us / 1e3, 1),
             'hbm_frac': round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), 'shape': shape}
        if graph_us is not None:
            r['graph_us'] = round(graph_us, 2)
            r['graph_hbm_frac'] = round(nbytes / graph_us / 1e3 / HBM_PEAK_GBS, 4)
        return r

    # The floor of both timings: a one-element fill, timed the same two ways.
    one = torch.empty(1, device=dev)
    out = {'launch_floor': {'avg_us': round(run(lambda i: one.fill_(1.0), reps), 2),
                            'graph_us': round(run_graph(lambda i: one.fill_(1.0), 64), 2),
                            'shape': 'torch fill_ of one fp32 element'}}
    w = torch.randn((4096, H), generator=gen, device=dev) * 0.02
    q, s = quantize_g128(w)
    del w
    pool = 64  # 64 x 8.66 MB
    qp = q.unsqueeze(0).expand(pool, -1, -1).contiguous()
    sp = s.unsqueeze(0).expand(pool, -1, -1).contiguous()
    x1 = torch.randn((1, H), generator=gen, device=dev).to(torch.bfloat16)
    fn1 = lambda i: int8.linear(x1, qp[i % pool], sp[i % pool])
    out['w8a16_linear_m1'] = hbm(run(fn1, reps), 4096 * H + 4096 * (H // 128) * 4 + H * 2 + 4096 * 2,
                                 '[1, 2048] x [4096, 2048] int8 g128', run_graph(fn1, 64))
    del qp, sp
    x2 = torch.randn((CHUNK, H), generator=gen, device=dev).to(torch.bfloat16)
    flops = 2.0 * CHUNK * 4096 * H
    us = run(lambda i: int8.linear(x2, q, s), 8)
    out['w8a16_linear_m2048'] = {'avg_us': round(us, 2), 'tflops': round(flops / us / 1e6, 1),
                                 'mfma_frac': round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                                 'shape': '[2048, 2048] x [4096, 2048] int8 g128'}
    xq, xs = w8a8.quantize(x2)
    us = run(lambda i: w8a8.gemm(xq, xs, q, s), 8)
    out['w8a8_gemm_m2048'] = {'avg_us': round(us, 2), 'tops': round(flops / us / 1e6, 1),
                              'int8_mfma_frac': round(flops / us / 1e6 / INT8_PEAK_TOPS, 4),
                              'shape': '[2048, 2048] x [4096, 2048] int8 g128 (rows pre-quantized)'}
    w = torch.randn((2 * I, H), generator=gen, device=dev) * 0.02
    q2, s2 = quantize_g128(w)
    del w, q, s
    pool = 256  # 256 x 2.16 MB
    q2p = q2.unsqueeze(0).expand(pool, -1, -1).contiguous()
    s2p = s2.unsqueeze(0).expand(pool, -1, -1).contiguous()
    for m in (1, 4, 8):
        xm = torch.randn((m, H), generator=gen, device=dev).to(torch.bfloat16)
        fnm = lambda i: w8a8.linear(xm, q2p[i % pool], s2p[i % pool], swiglu=True)
        out[f'w8a8_gate_up_swiglu_m{m}'] = hbm(
            run(fnm, reps), GU_EXPERT_BYTES + H * 2 * m + I * 2 * m,
            f'[{m}, 2048] x [1024, 2048] int8 g128', run_graph(fnm, 64))
    m1, m8 = out['w8a8_gate_up_swiglu_m1'], out['w8a8_gate_up_swiglu_m8']
    out['w8a8_gate_up_swiglu_m8_over_m1'] = {'event': round(m8['avg_us'] / m1['avg_us'], 3),
                                             'graph': round(m8['graph_us'] / m1['graph_us'], 3)}
    return out


def skewed_prefill_probe(dev, reps=5):
    """One MoE layer on a 2048-token chunk with the router logits biased by a
    Zipf(1.1) per-expert offset (runtime.stack.zipf_bias): few hot experts
    with many rows each, many empty.  Times each phase with HIP events and
    reports the grouped GEMMs against the bf16 MFMA peak.  Returns the
    report and the layer's host copy, input and output (the CPU baseline
    times the same layer)."""
    from localmoe35ba3b_amd.runtime.stack import SyntheticMoEStack, zipf_bias
    st = SyntheticMoEStack(layers=1, seed=3, device=dev, max_tokens=CHUNK, router_bias=zipf_bias())
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    x = torch.randn((CHUNK, H), generator=gen, device=dev).to(torch.bfloat16)
    ids = torch.empty((CHUNK, K), dtype=torch.int32, device=dev)
    out = x.clone()
    st.layer_forward(out, 0, ids)
    torch.cuda.synchronize()
    counts = np.bincount(ids.cpu().numpy().reshape(-1), minlength=E)
    active = int((counts > 0).sum())
    ev = [make_events(8) for _ in range(reps)]
    for r in range(reps):
        st.layer_forward(x.clone(), 0, events=ev[r])
    torch.cuda.synchronize()
    ms = {p: sorted(ev[r][i].elapsed_time(ev[r][i + 1]) for r in range(reps))[reps // 2]
          for i, p in enumerate(PREFILL_PHASES)}
    fl = prefill_flops()
    pb = prefill_bytes(active)
    report = {'active_experts': active, 'max_rows': int(counts.max()),
              'layer_us': round(sum(ms.values()) * 1e3, 2)}
    for p in ('gate_up', 'down'):
        us = ms[p] * 1e3
        report[p] = {'avg_us': round(us, 2), 'tflops': round(fl[p] / us / 1e6, 1),
                     'mfma_frac': round(fl[p] / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                     'bytes_per_launch': pb[p], 'gbs': round(pb[p] / us / 1e3, 1)}
    host = {'layer': st.layer_host(0), 'x': x.float().cpu().numpy(),
            'out': out.float().cpu().numpy(), 'ids': ids.cpu().numpy()}
    del st
    torch.cuda.empty_cache()
    return report, host


def cpu_info():
    """CPU model, logical CPUs this process may run on, and the physical cores
    among them (distinct (package, core) pairs of the sysfs topology)."""
    model = 'unknown'
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                model = line.split(':', 1)[1].strip()
                break
    except OSError:
        pass
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        base = f'/sys/devices/system/cpu/cpu{c}/topology/'
        try:
            cores.add((open(base + 'physical_package_id').read().strip(),
                       open(base + 'core_id').read().strip()))
        except OSError:
            cores.add(('?', str(c)))
    return {'model': model, 'logical_cpus': len(cpus), 'physical_cores': len(cores)}


def cpu_baseline(stack, x, decode_records, n_dec, zipf_host, threads, info):
    """The CPU oracle (the reference's dequantize-then-matmul arithmetic on the
    host: torch-CPU bf16 F.linear after dequantization, numpy int W8A8) timed
    on this host with `threads` threads, on the workload's own inputs:
      config 1  W8A16 [4096, 2048] at M = 1 and M = 2048, in full
      config 2  W8A8 gate_up [1024, 2048] + SwiGLU at M = 1, 4, 8, in full
      config 3  one MoE layer on one token (W8A8 routed experts): the mean of
                the 40 x 33 token-layers of config 5's decode
      config 4  one MoE layer on the Zipf-skewed 2048-token chunk, in full
      config 5  decode: all 33 tokens through all 40 layers, in full, each
                layer on the input the GPU saw there; prefill: one
                2048-token chunk through one layer, extrapolated x80
    The decode and Zipf runs assert what they compute: routing ids equal to
    the GPU's bit for bit, layer outputs within the bf16 tolerance."""
    from oracle import moe_oracle as O
    from localmoe35ba3b_amd.runtime.stack import EPS
    torch.set_num_threads(threads)

    def close(a, b, what):
        rel = float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
        if not rel <= 2e-2:
            raise AssertionError(f'cpu baseline: {what} differs from the GPU (rel {rel:.3e})')
        return rel

    out = {}
    g = torch.Generator()
    g.manual_seed(0)
    wq, ws = O.quantize_weight((torch.randn(4096, H, generator=g) * 0.02).numpy())
    for m in (1, 2048):
        xm = O.bf16(torch.randn(m, H, generator=g).numpy())
        t0 = time.perf_counter()
        O.w8a16_linear(xm, wq, ws)
        dt = time.perf_counter() - t0
        out[f'w8a16_linear_m{m}'] = {'s': round(dt, 4), 'tok_s': round(m / dt, 2)}
    gq, gs = O.quantize_weight((torch.randn(2 * I, H, generator=g) * 0.02).numpy())
    for m in (1, 4, 8):
        xm = O.bf16(torch.randn(m, H, generator=g).numpy())
        t0 = time.perf_counter()
        O.swiglu(O.w8a8_linear(xm, gq, gs))
        dt = time.perf_counter() - t0
        out[f'w8a8_gate_up_swiglu_m{m}'] = {'s': round(dt, 4), 'tok_s': round(m / dt, 2)}
    log('cpu configs 1-2 done')
    if zipf_host is not None:
        t0 = time.perf_counter()
        ref, (_, _, ri) = O.moe_layer(zipf_host['x'], zipf_host['layer'], k=K, eps=EPS)
        dt = time.perf_counter() - t0
        if not np.array_equal(ri, zipf_host['ids']):
            raise AssertionError('cpu baseline: Zipf-chunk routing differs from the GPU')
        rel = close(zipf_host['out'], ref, 'Zipf-chunk layer output')
        out['zipf_prefill_layer'] = {'s': round(dt, 3), 'tok_s': round(CHUNK / dt, 2),
                                     'rel_err_vs_gpu': round(rel, 6)}
        log(f'cpu config 4 (Zipf chunk layer): {dt:.2f} s, routing exact')
    layer0 = stack.layer_host(0)
    t0 = time.perf_counter()
    O.moe_layer(x[:CHUNK].float().cpu().numpy(), layer0, k=K, eps=EPS)
    t_chunk_layer = time.perf_counter() - t0
    del layer0
    log(f'cpu prefill sample (one chunk, one layer): {t_chunk_layer:.2f} s')
    t_dec, worst = 0.0, 0.0
    for tok in range(n_dec):
        for l, (h_in, ids, h_out, host) in enumerate(decode_records(tok)):
            t0 = time.perf_counter()
            ref, (_, _, ri) = O.moe_layer(h_in, host, k=K, eps=EPS)
            t_dec += time.perf_counter() - t0
            if not np.array_equal(ri, ids):
                raise AssertionError(f'cpu baseline: decode token {tok} layer {l} routing differs')
            worst = max(worst, close(h_out, ref, f'decode token {tok} layer {l} output'))
        if tok % 8 == 7:
            log(f'cpu decode: {tok + 1} tokens, {t_dec:.1f} s')
    out['moe_layer_decode_1tok'] = {'s': round(t_dec / max(n_dec * stack.L, 1), 5)}
    prefill_tok_s = CHUNK / (t_chunk_layer * stack.L)
    return {
        'value': round(prefill_tok_s, 3), 'unit': 'tok/s', 'cores': threads, 'kind': 'port',
        'decode_tok_s': round(n_dec / t_dec, 4) if n_dec else None,
        'cpu': info, 'configs': out,
        'checks': {'decode_token_layers': n_dec * stack.L, 'routing': 'bit-exact',
                   'max_rel_err_vs_gpu': round(worst, 6)},
        'sample': (f'oracle (torch-CPU dequant + F.linear, numpy int W8A8) on {threads} threads '
                   f'of {info["physical_cores"]} physical cores ({info["model"]}): value = one '
                   f'2048-token prefill chunk through 1 of {stack.L} layers '
                   f'({t_chunk_layer:.2f} s), extrapolated x{stack.L} layers; decode = all '
                   f'{n_dec} tokens through all {stack.L} layers in full ({t_dec:.1f} s) on the '
                   f'GPU\'s per-layer inputs, routing asserted bit-exact and outputs within '
                   f'2e-2; configs 1-4 timed in full'),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f'bench.py measures one GPU; --gpus {args.gpus} is not supported (across GPUs the '
              'path would replicate the bank per GPU or shard experts with an all-to-all per '
              'layer; neither is built)', file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from localmoe35ba3b_amd.runtime.stack import SyntheticMoEStack

    dev = torch.device('cuda:0')
    if args.copy_probe:
        copy_probe(dev)
        return
    t_build = time.perf_counter()
    stack = SyntheticMoEStack(layers=args.layers, seed=4, device=dev, max_tokens=CHUNK)
    torch.cuda.synchronize()
    if args.power_probe:
        power_probe(stack, dev)
        return
    t_build = time.perf_counter() - t_build
    log(f'stack built: {stack.L} layers, {stack.bank_bytes() / 1e9:.2f} GB in HBM, {t_build:.1f} s')
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    x = torch.randn((PREFILL_TOKENS, H), generator=gen, device=dev).to(torch.bfloat16)
    dec_in = torch.randn((DECODE_TOKENS, 1, H), generator=gen, device=dev).to(torch.bfloat16)
    nchunks = PREFILL_TOKENS // CHUNK
    L = stack.L

    # decode step = all layers on one token, captured once as a HIP graph
    static = dec_in[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack.forward(static.clone())
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack.forward(static)
    # Per-kernel decode times: ROCm graphs cannot hold event records, so each
    # timed request ends with one more decode token launched eagerly with HIP
    # events between its kernels.  A spin kernel placed in front holds the
    # stream until all 40 layers are queued, so the events see the kernels
    # back to back, as in the graph, not the host's launch gaps.  That token
    # is timed apart from the 33 graph-replayed tokens of decode tok/s.
    dec_ev = None if args.no_events else [make_events(4) for _ in range(L)]
    spin_cycles = 0
    if dec_ev is not None:
        a, b = make_events(2)
        a.record()
        torch.cuda._sleep(1 << 20)
        b.record()
        torch.cuda.synchronize()
        spin_cycles = int((1 << 20) * 3.0 / max(a.elapsed_time(b), 1e-3))  # ~3 ms

    # prefill: both 2048-token chunks through all layers, the second chunk on
    # a second stream one layer behind the first (MoEStack.prefill_),
    # captured once as a HIP graph; the prompt is copied into its input
    pstatic = x.clone()
    with torch.cuda.stream(side):
        stack.prefill_(pstatic.clone(), CHUNK)
    torch.cuda.current_stream().wait_stream(side)
    pgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(pgraph):
        stack.prefill_(pstatic, CHUNK)
    # Per-kernel prefill times: one more chunk per timed step, launched
    # eagerly with events between its kernels behind a spin kernel (as for
    # decode), timed apart from prefill tok/s.
    pf_events = None if args.no_events else [make_events(8) for _ in range(L)]
    pprobe = torch.empty_like(x[:CHUNK])

    def prefill():
        pstatic.copy_(x)
        pgraph.replay()

    def prefill_kernel_probe():
        # chained like the timed graph: after layer 0 the norm phase is empty
        # and each combine does the next layer's norm work
        pprobe.copy_(x[:CHUNK])
        torch.cuda._sleep(3 * spin_cycles)
        for l in range(L):
            stack.layer_forward(pprobe, l, events=pf_events[l],
                                next_layer=l + 1 if l + 1 < L else None, input_normed=l > 0)

    def decode():
        for i in range(DECODE_TOKENS):
            static.copy_(dec_in[i])
            graph.replay()

    def decode_kernel_probe():
        static.copy_(dec_in[-1])
        torch.cuda._sleep(spin_cycles)
        for l in range(L):
            stack.layer_forward(static, l, events=dec_ev[l])

    def step(m=None):
        """One step: the timed prefill and decode, then the per-kernel probes."""
        if m is not None:
            m[0].record()
        prefill()
        if m is not None:
            m[1].record()
        decode()
        if m is not None:
            m[2].record()
        if dec_ev is not None:
            decode_kernel_probe()
        if pf_events is not None:
            prefill_kernel_probe()
            torch.cuda.synchronize()

    # Warm-up steps do a timed step's work, probes included, so the first
    # timed step starts from the state every later one starts from.
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log('warmup done')

    marks = [make_events(3) for _ in range(args.steps)]
    phase_ms = {p: 0.0 for p in PREFILL_PHASES}
    norm_first_ms = 0.0  # the norm kernel runs for the first layer of the chain only
    dec_ms = {p: 0.0 for p in DECODE_PHASES}
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for s in range(args.steps):
        step(marks[s])
        if pf_events is not None:
            for l in range(L):
                ev = pf_events[l]
                for i, p in enumerate(PREFILL_PHASES):
                    phase_ms[p] += ev[i].elapsed_time(ev[i + 1])
                norm_first_ms += ev[0].elapsed_time(ev[1]) if l == 0 else 0.0
            for l in range(L):
                for j, p in enumerate(DECODE_PHASES):
                    dec_ms[p] += dec_ev[l][j].elapsed_time(dec_ev[l][j + 1])
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    pf_steps = [m[0].elapsed_time(m[1]) for m in marks]
    dec_steps = [m[1].elapsed_time(m[2]) for m in marks]
    t_prefill = sum(pf_steps) / 1e3
    t_decode = sum(dec_steps) / 1e3
    steps = args.steps
    log(f'timed {steps} steps: {wall:.3f} s')
    prefill_tok_s = steps * PREFILL_TOKENS / t_prefill
    decode_tok_s = steps * DECODE_TOKENS / t_decode
    decode_gbs = DECODE_LAYER_BYTES * L * decode_tok_s / 1e9

    # untimed: routing statistics (active experts per layer-chunk)
    ids = torch.empty((CHUNK, K), dtype=torch.int32, device=dev)
    active = []
    out = x.clone()
    for c in range(nchunks):
        hc = out[c * CHUNK:(c + 1) * CHUNK]
        for l in range(L):
            stack.layer_forward(hc, l, ids)
            active.append(int(torch.unique(ids).numel()))

    launches_pf = steps * L  # prefill launches timed: the probe chunk of every request
    mean_active = float(np.mean(active))
    kernels = {}
    if pf_events is not None:
        pb = [prefill_bytes(a) for a in active]
        fl = prefill_flops()
        for p in ('gate_up', 'down'):
            avg_us = phase_ms[p] / launches_pf * 1e3
            avg_bytes = float(np.mean([b[p] for b in pb]))
            kernels['prefill_' + p] = {
                'avg_us': round(avg_us, 2), 'launches': launches_pf,
                'total_ms': round(phase_ms[p], 3), 'bytes_per_launch': int(avg_bytes),
                'gbs': round(avg_bytes / avg_us / 1e3, 1),
                'tflops': round(fl[p] / avg_us / 1e6, 1)}
        for p in ('router_logits', 'topk', 'route_plan', 'combine'):
            kernels['prefill_' + p] = {'avg_us': round(phase_ms[p] / launches_pf * 1e3, 2),
                                       'total_ms': round(phase_ms[p], 3)}
        # chained layers: the norm kernel runs for layer 0 only; the other
        # layers' norm phase is empty (only its pair of events is timed)
        kernels['prefill_norm_gate'] = {
            'avg_us': round(norm_first_ms / steps * 1e3, 2), 'launches': steps,
            'total_ms': round(norm_first_ms, 3),
            'empty_phase_avg_us': round((phase_ms['norm_gate'] - norm_first_ms) /
                                        max(1, steps * (L - 1)) * 1e3, 2)}
    n_dec = steps * L  # decode launches timed: the probe token of every request
    dec_bytes = {'decode_router': E * H * 2 + H * 2,
                 'decode_gate_up': 9 * GU_EXPERT_BYTES,
                 'decode_down': 9 * DN_EXPERT_BYTES}
    if dec_ev is not None:
        for p in DECODE_PHASES:
            avg_us = dec_ms[p] / n_dec * 1e3
            kernels[p] = {'avg_us': round(avg_us, 2), 'launches': n_dec,
                          'bytes_per_launch': dec_bytes[p],
                          'gbs': round(dec_bytes[p] / avg_us / 1e3, 1),
                          'hbm_frac': round(dec_bytes[p] / avg_us / 1e3 / HBM_PEAK_GBS, 4),
                          'ms_per_request': round(avg_us * L * DECODE_TOKENS / 1e3, 3)}

    # dominant kernel by total time within one request
    per_req = {}
    if pf_events is not None:
        # the probe times one chunk per request; a request has nchunks of them
        per_req['prefill_gate_up'] = phase_ms['gate_up'] / steps * nchunks
        per_req['prefill_down'] = phase_ms['down'] / steps * nchunks
        per_req['prefill_router_logits'] = phase_ms['router_logits'] / steps * nchunks
        for p in DECODE_PHASES:
            per_req[p] = dec_ms[p] / steps * DECODE_TOKENS
    roofline = None
    if per_req:
        dom = max(per_req, key=per_req.get)
        k = kernels[dom]
        achieved = k['bytes_per_launch'] / k['avg_us'] / 1e3
        roofline = {'bound': 'hbm', 'kernel': dom, 'achieved': round(achieved, 1),
                    'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': round(achieved / HBM_PEAK_GBS, 4),
                    'traffic': pmc_traffic().get(dom), 'bytes_per_launch': k['bytes_per_launch'],
                    'avg_us': k['avg_us']}

    kernels['lm_head_gemv'] = lm_head_probe(dev)  # after the timed steps, timed on its own
    skewed, zipf_host = (None, None) if args.no_events else skewed_prefill_probe(dev)
    isolated = None if args.no_events else isolated_probe(dev, 4 * spin_cycles)

    cpu = None
    if not args.no_cpu_baseline:
        info = cpu_info()
        threads = max(1, min(info['physical_cores'], 16))
        ids_buf = torch.empty((1, K), dtype=torch.int32, device=dev)

        def decode_records(i):
            """Untimed: decode token i's per-layer inputs, routing and outputs
            on the GPU, with host copies of the experts each layer selected."""
            hg = dec_in[i].clone()
            recs = []
            for l in range(L):
                h_in = hg.float().cpu().numpy()
                stack.layer_forward(hg, l, ids_buf)
                ids_np = ids_buf.cpu().numpy()
                recs.append((h_in, ids_np, hg.float().cpu().numpy(),
                             stack.layer_host(l, experts=ids_np[0])))
            return recs

        n_dec = min(args.cpu_decode_tokens, DECODE_TOKENS)
        cpu = cpu_baseline(stack, x, decode_records, n_dec, zipf_host, threads, info)

    line = {
        'metric': 'MoE-FFN prefill/decode tok/s (4K chunk); decode HBM GB/s and % of peak',
        'value': round(prefill_tok_s, 1), 'unit': 'tok/s', 'n_gpus': 1, 'steps': steps,
        'warmup': args.warmup, 'ms_per_step': round(wall / steps * 1e3, 3),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16',
        'data': 'synthetic (random-init int8 g128 weights, N(0,1) activations)',
        'config': {'workload': f'{L}-layer MoE-FFN stack: 4096-token prefill (2x2048 chunks, '
                               f'W8A16) + 33 decode tokens (W8A8 experts), 256 experts top-8 + '
                               f'shared, hidden 2048, intermediate 512',
                   'layers': L, 'prefill_tokens': PREFILL_TOKENS, 'chunk': CHUNK,
                   'prefill_schedule': 'chunk 2 enters layer l once chunk 1 has left layer '
                                       'l-1 (second stream); one HIP graph',
                   'decode_tokens': DECODE_TOKENS, 'bank_gb': round(stack.bank_bytes() / 1e9, 2),
                   'prefill_tile_copy_gb': round(stack.tile_bytes() / 1e9, 2)},
        'prefill_tok_s': round(prefill_tok_s, 1),
        'prefill_ms_steps': [round(t, 3) for t in pf_steps],
        'decode_ms_steps': [round(t, 3) for t in dec_steps],
        'decode_tok_s': round(decode_tok_s, 1),
        'decode_hbm_gbs': round(decode_gbs, 1),
        'decode_hbm_frac': round(decode_gbs / HBM_PEAK_GBS, 4),
        'decode_dtype': 'int8 (W8A8 experts), bf16 (shared expert, router fp64)',
        'prefill_dtype': ('bf16 activations and outputs; gate_up on fp16 MFMAs (exact q, exact '
                          'fp16 copies of the rows, group scales on the fp32 sums), down on bf16 '
                          'MFMAs of bf16(q*s); router fp64/bf16'
                          if stack._structs[0].gu_q_tiles_format == 1 and stack.gu_q_tiles is not None
                          else 'bf16 MFMAs of bf16(q*s), fp32 accumulation; router fp64/bf16'),
        'mean_active_experts': round(mean_active, 1),
        'roofline': roofline,
        'kernels': kernels,
        'prefill_zipf_layer': skewed,
        'isolated_kernels': isolated,
        'cpu_baseline': cpu,
        'build_s': round(t_build, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
