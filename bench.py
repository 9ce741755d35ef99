"""Benchmark of the quantized routed-MoE layer on one MI355X.

A step is one forward pass of the whole ornith_g256 MoE layer over one batch
of N tokens: router logits + softmax/top-8, permutation, the 8 routed experts
and the shared expert (gate-up, SiLU, down, all G256 4-bit with dequantisation
fused into the integer dot), and the slot-order combination.  Inputs and all
weights are resident in HBM; 40 independently generated layers are cycled so
the 256 MB MALL cannot serve repeated weights.  The step sequence is captured
in a HIP graph and replayed; K steps are timed with HIP events on the replay
stream.

Default workload: N=1 decode (the metric's headline).  The same JSON line also
reports, under "per_tokens", N=32, the 1120-token prefill (router bias with
Zipf(1.1) expert popularity, plus the dense G256 linear [6144, 2048] on the
same rows) and the 8192-token prefill (Zipf(1.3), plus the G256 LM head
[151936, 2048] on 32 rows).

"roofline" is that of the kernel with the largest total time: after the timed
graph replays, K more steps run eagerly with every library kernel launch
bracketed by a HIP event pair on the launch's own stream (the library's
timing hook, include/ornith_timing.h); its average interval is the
denominator of the kernel's algorithmic bytes (or ops) per launch.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / 'ornith-ciru-halo-agent_amd'))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0          # MI355X dense int8 MFMA
FP32_PEAK_TFLOPS = 157.3         # MI355X dense fp32 matrix peak
BF16_PEAK_TFLOPS = 2500.0
GATEUP_BYTES = 1024 * 2048 // 2 + 4 * 1024 * 8       # one gate-up bank: u4 codes + fp16 scale|offset words
DOWN_BYTES = 2048 * 512 // 2 + 4 * 2048 * 2          # one down bank
EXPERT_BYTES = GATEUP_BYTES + DOWN_BYTES              # 1,622,016
ROUTER_BYTES = 256 * 2048 * 2 + 2048 * 2
HEAD_N, HEAD_ROWS = 151936, 32
DENSE_N = 6144

# HBM bytes per launch (L2 misses: FETCH_SIZE + WRITE_SIZE) from rocprofv3
# --pmc runs, scaled by the factor a plain copy of known size reads (bench.py
# --copy-calibration); keyed by (kernel, tokens).  Commands and raw figures:
# profiles/decode_n1_n32_hbm_traffic_pmc.md, profiles/prefill_1120_8192_hbm_traffic_pmc.md.
MEASURED_TRAFFIC = {
    ('layer1', 1): 16768264, ('route1', 1): 1166652, ('gateup1', 1): 9949504, ('down1', 1): 5118494,
    ('route_select', 32): 5329307, ('gateup', 32): 176476340, ('down', 32): 94490777, ('reduce', 32): 2596402,
    ('router', 1120): 15343263, ('topk', 1120): 2186638, ('permute_scan_act', 1120): 7786592,
    ('permute_scatter', 1120): 320474, ('gateup_mfma', 1120): 190732263, ('quant_middle', 1120): 26020249,
    ('down_mfma', 1120): 177260462, ('reduce', 1120): 87590525,
    ('router', 8192): 50519818, ('topk', 8192): 9599320, ('permute_scan_act', 8192): 56100945,
    ('permute_scatter', 8192): 1531030, ('gateup_mfma', 8192): 625504138,
    ('quant_middle', 8192): 189713102, ('down_mfma', 8192): 845063402, ('reduce', 8192): 639829271,
}


def kernel_cost(name, T, unique):
    """Algorithmic work of one launch of `name` for a T-token layer that touches
    `unique` routed experts: (bound, amount, peak, unit).  hbm amounts are the
    compulsory bytes (weights of the touched banks + activations in and out);
    mfma amounts are the int8 ops of the exact integer dots (2 per MAC).  The
    grouped prefill projections report whichever roof binds at this T (the
    larger of bytes / HBM peak and ops / int8 peak): HBM at 1120 tokens, the
    matrix cores for the gate-up at 8192."""
    banks = unique + 1
    routes = 9 * T
    if name == 'layer1':            # the whole single-token layer in one launch
        return 'hbm', banks * EXPERT_BYTES + ROUTER_BYTES + T * 2048 * 2 * 2, HBM_PEAK_GBS, 'GB/s'
    if name in ('route1', 'route', 'route_select'):
        return 'hbm', ROUTER_BYTES + T * 2048 * 2, HBM_PEAK_GBS, 'GB/s'
    if name in ('gateup1', 'gateup'):
        return 'hbm', banks * GATEUP_BYTES + T * 2048 + routes * 512 * 4, HBM_PEAK_GBS, 'GB/s'
    if name in ('down1', 'down'):
        return 'hbm', banks * DOWN_BYTES + routes * 512 * 4 + T * 2048 * 2, HBM_PEAK_GBS, 'GB/s'
    if name in ('gateup_mfma', 'down_mfma'):
        if name == 'gateup_mfma':       # codes + meta, A8 gate input in, fp32 middle rows out
            nbytes, ops = banks * GATEUP_BYTES + T * 2048 + routes * 512 * 4, 2 * routes * 1024 * 2048
        else:                           # codes + meta, A8 middle rows in, fp32 route rows out
            nbytes, ops = banks * DOWN_BYTES + routes * 512 + routes * 2048 * 4, 2 * routes * 2048 * 512
        if nbytes / (HBM_PEAK_GBS * 1e9) >= ops / (INT8_PEAK_TOPS * 1e12):
            return 'hbm', nbytes, HBM_PEAK_GBS, 'GB/s'
        return 'mfma', ops, INT8_PEAK_TOPS, 'TFLOP/s'
    if name == 'router':      # exact K=1 fp32 matrix steps (the shared-gate row on the VALU)
        return 'mfma', 2 * T * 257 * 2048, FP32_PEAK_TFLOPS, 'TFLOP/s'
    if name == 'permute_scan_act':  # the scan's block counts are noise beside the gate-input quantisation
        return 'hbm', T * 2048 * 2 + T * 2048 + T * 8 * (2 + 4), HBM_PEAK_GBS, 'GB/s'
    return 'hbm', T * 2048 * 2, HBM_PEAK_GBS, 'GB/s'


def parse():
    p = argparse.ArgumentParser()
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=200)
    p.add_argument('--warmup', type=int, default=40)
    p.add_argument('--tokens', type=int, default=1)
    p.add_argument('--layers', type=int, default=40)
    p.add_argument('--extra-tokens', default='32,1120,8192')
    p.add_argument('--copy-calibration', action='store_true',
                   help='only run a plain 256 MiB device copy (PMC scale factor for FETCH_SIZE/WRITE_SIZE)')
    p.add_argument('--oracle-seconds', type=float, default=5.0)
    p.add_argument('--no-cpu-baseline', action='store_true')
    p.add_argument('--part', choices=('head', 'dense', 'w8head', 'gateup-bf16-model'), default=None,
                   help='time only the G256 LM head (32x151936), the dense 6144x2048 prefill (1120 rows), or '
                        'the bf16 model of the grouped prefill gate-up, and print one JSON line (for profiling)')
    return p.parse_args()


class LayerRunner:
    """Holds L layers of weights and per-T buffers; captures one graph of L steps."""

    def __init__(self, layers, T, device, silu, sigmoid, bias=None):
        import torch
        from ornith_g256 import native
        self.torch, self.native = torch, native
        self.layers, self.T, self.device = layers, T, device
        self.silu, self.sigmoid, self.bias = silu, sigmoid, bias
        gen = torch.Generator(device=device)
        gen.manual_seed(1000 + T)
        self.x = torch.randn((T, 2048), generator=gen, device=device).to(torch.bfloat16)
        layout = native.routed_layout(T, 'layer')
        self.ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
        self.out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
        self.tw = torch.empty((T, 8), dtype=torch.float32, device=device)
        self.ti = torch.empty((T, 8), dtype=torch.int32, device=device)
        self.sl = torch.empty((T,), dtype=torch.bfloat16, device=device)
        self.flags = torch.zeros(1, dtype=torch.int32, device=device)
        self.graphs = {}

    def check_flags(self):
        """Raise if any launch of this runner set a sticky native flag."""
        f = int(self.flags.item())
        if f:
            raise RuntimeError(f'native flags raised at {self.T} tokens: {f}')

    def step(self, i):
        L = self.layers[i % len(self.layers)]
        self.native.moe_layer(self.x, L['router'], self.bias, L['gate'], L['w13'][0], L['w13'][1], L['w2'][0],
                              L['w2'][1], L['s13'][0], L['s13'][1], L['s2'][0], L['s2'][1], self.silu, self.sigmoid,
                              self.ws, self.tw, self.ti, self.sl, self.out, self.flags, self.T)

    def graph(self, n):
        torch = self.torch
        if n not in self.graphs:
            s = torch.cuda.Stream(device=self.device)
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for i in range(n):          # warm the launch path outside capture
                    self.step(i)
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(n):
                    self.step(i)
            torch.cuda.synchronize()
            self.graphs[n] = g
        return self.graphs[n]

    def time_steps(self, steps, warmup):
        torch = self.torch
        L = len(self.layers)
        full = self.graph(L)
        rem = steps % L
        tail = self.graph(rem) if rem else None
        for _ in range(max(1, warmup // L)):
            full.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps // L):
            full.replay()
        if tail is not None:
            tail.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    def routed_experts_touched(self):
        """Average number of distinct routed experts per layer."""
        counts = []
        for i in range(len(self.layers)):
            self.step(i)
            counts.append(int(self.ti.unique().numel()))
        return sum(counts) / len(counts)

    def kernel_times(self, steps):
        """Eager pass of `steps` layers with every library kernel launch
        bracketed by a HIP event pair on its stream: {kernel: (launches, ms)}."""
        torch, native = self.torch, self.native
        torch.cuda.synchronize()
        with native.KernelTimer('*') as kt:
            for i in range(steps):
                self.step(i)
            torch.cuda.synchronize()
            return {n: kt.read(n) for n in kt.names()}


def algorithmic(T, unique):
    """Compulsory bytes and flops of one layer (touched experts + shared + router + I/O)."""
    bytes_ = (unique + 1) * EXPERT_BYTES + ROUTER_BYTES + T * 2048 * 2 * 2
    flops = 2 * (T * 9 * (1024 * 2048 + 2048 * 512) + T * 257 * 2048)
    return bytes_, flops


def roofline(times, T, unique):
    """Roofline of the kernel with the largest total time in `times`."""
    name = max(times, key=lambda n: times[n][0] * times[n][1])
    launches, ms = times[name]
    bound, amount, peak, unit = kernel_cost(name, T, unique)
    scale = 1e9 if unit == 'GB/s' else 1e12
    achieved = amount / (ms * 1e-3) / scale
    traffic = MEASURED_TRAFFIC.get((name, T))
    return {'bound': bound, 'achieved': achieved, 'peak': peak, 'unit': unit, 'frac': achieved / peak,
            'traffic': traffic, 'kernel': name, 'avg_us': ms * 1e3, 'launches': launches,
            'algorithmic_per_launch': amount}


def gateup_bf16_model_us(device, steps=10):
    """The bf16 matrix-core design of the grouped prefill gate-up, modelled
    by this library's code-reading bf16 GEMM (each 64-column code tile
    dequantised into LDS once per 256-row tile, bf16 MFMA, fp32 accumulation)
    at shapes whose (256-row tiles) x (1024-column blocks) equal the m-tiles of
    the grouped gate-up with every tile full: 6144 x 12288 x 2048 = 288 tiles
    (8192 tokens, 73728 routes) and 1280 x 8192 x 2048 = 40 tiles (1120
    tokens, 10080 routes).  No row gather and no SiLU epilogue: a lower bound
    of the grouped kernel's time."""
    import torch
    from ornith_g256 import native
    res = {}
    for M, N, live in ((6144, 12288, 73728), (1280, 8192, 10080)):
        gen = torch.Generator(device=device)
        gen.manual_seed(5)
        x = torch.randn((M, 2048), generator=gen, device=device).to(torch.bfloat16)
        codes = torch.randint(0, 2 ** 31 - 1, (N * 2048 // 8,), generator=gen, device=device, dtype=torch.int32)
        scale = (torch.rand((N * 2048 // 256,), generator=gen, device=device) * 0.015 + 0.005).half()
        meta = scale.view(torch.int16).to(torch.int32) & 0xffff
        ws = torch.empty((M + 15) // 16 * 16 * 2048 * 2, dtype=torch.uint8, device=device)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=device)
        flags = torch.zeros(1, dtype=torch.int32, device=device)
        call = lambda: native.dense_out(x, codes, meta, ws, out, flags, M, N, 2048, 2, 128)
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        with native.KernelTimer('*') as kt:
            for _ in range(steps):
                call()
            torch.cuda.synchronize()
            gemm = kt.read('dense_gemm')[1] * 1e3
        if int(flags.item()):
            raise RuntimeError(f'native flags raised by the bf16 gate-up model at {M}x{N}: {int(flags.item())}')
        res[f'{M}x{N}x2048'] = {'gemm_us': gemm, 'tflops': 2 * M * N * 2048 / gemm / 1e6,
                                'routes_modelled': live, 'tiles': M // 256 * (N // 1024)}
    return res


def graph_ms(call, n, reps=3):
    """Milliseconds per call of `call(0..n-1)` captured once into a CUDA
    graph and replayed `reps` times (warmed up outside the capture first), so
    host-side gaps between the calls do not count, as in a serving loop that
    replays captured steps."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n):
            call(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            call(i)
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (reps * n)


def dense_prefill_ms(T, device, steps=20):
    """Dense G256 linear [6144, 2048] on T rows through ornith_g256::dense_out.
    Up to 64 rows (the A8 GEMV, weight-streaming) 48 weight copies (312 MB)
    rotate so the 6.5 MB bank is not MALL-resident; above, one copy."""
    import torch
    from ornith_g256 import native
    gen = torch.Generator(device=device)
    gen.manual_seed(77)
    x = torch.randn((T, 2048), generator=gen, device=device).to(torch.bfloat16)
    banks = []
    for _ in range(48 if T <= 64 else 1):
        codes = torch.randint(0, 2 ** 31 - 1, (DENSE_N * 2048 // 8,), generator=gen, device=device,
                              dtype=torch.int32)
        meta = (torch.rand((DENSE_N * 2048 // 256,), generator=gen, device=device) * 0.015 + 0.005).half()
        banks.append((codes, meta.view(torch.int16).to(torch.int32) & 0xffff))
    layout = native.dense_layout(T, DENSE_N, 2048)
    ws = torch.empty(max(layout.workspace_bytes, T * 2048 * 2 + DENSE_N * 2048 * 2), dtype=torch.uint8,
                     device=device)
    out = torch.empty((T, DENSE_N), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    call = lambda i: native.dense_out(x, *banks[i % len(banks)], ws, out, flags, T, DENSE_N, 2048, 2, 128)
    for i in range(3):
        call(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        call(i)
    b.record()
    torch.cuda.synchronize()
    if int(flags.item()):
        raise RuntimeError(f'native flags raised by the dense linear at {T} rows: {int(flags.item())}')
    wall = a.elapsed_time(b) / steps
    if T > 64:
        return graph_ms(call, steps)
    # Small T is bound by the host's per-call launch cost; also report the
    # device time (sum of the library kernels' event-timed durations) and the
    # per-call time of captured calls.
    with native.KernelTimer('*') as kt:
        for i in range(steps):
            call(i)
        torch.cuda.synchronize()
        device_ms = sum(kt.read(n)[1] for n in kt.names())
    return wall, device_ms, graph_ms(call, steps)


def head_ms(device, steps=20):
    """G256 LM head [151936, 2048] on 32 rows: fp32 logits, bf16 logits, argmax.
    Two weight copies alternate, so the 160 MB bank is not MALL-resident."""
    import torch
    from ornith_g256 import native, synthetic
    gen = torch.Generator(device=device)
    gen.manual_seed(78)
    banks = [synthetic.bank(gen, HEAD_N, 2048, device) for _ in range(2)]
    x = torch.randn((HEAD_ROWS, 2048), generator=gen, device=device).to(torch.bfloat16)
    ws = torch.empty(native.lib().ornith_dense_g256_head_workspace_bytes(64, HEAD_N), dtype=torch.uint8,
                     device=device)
    logits = torch.empty((HEAD_ROWS, HEAD_N), dtype=torch.float32, device=device)
    lb = torch.empty((HEAD_ROWS, HEAD_N), dtype=torch.bfloat16, device=device)
    am = torch.empty((HEAD_ROWS,), dtype=torch.int64, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    call = lambda i: native.dense_head(x, *banks[i % 2], ws, logits, lb, am, flags, 64)
    for i in range(4):
        call(i)
    torch.cuda.synchronize()
    ms = graph_ms(call, steps)
    if int(flags.item()):
        raise RuntimeError(f'native flags raised by the G256 head: {int(flags.item())}')
    return ms


def w8_head_us(device, rows=(1, 8, 64), steps=20):
    """The reference's W8 G128 LM head [248320, 2048] (head_i8_tile_api.h:22)
    at each row count: microseconds per call (captured calls replayed; the
    eager figure, host gaps included, beside it) with two 520 MB weight copies
    alternating (not MALL-resident), plus the kernel's average and its HBM
    rate over the weight and scale bytes."""
    import torch
    from ornith_g256 import native
    gen = torch.Generator(device=device)
    gen.manual_seed(79)
    N = native.HEAD_VOCAB
    banks = [(torch.randint(-2 ** 31, 2 ** 31, (N // 16, 128, 4, 16), generator=gen, dtype=torch.int64,
                            device=device).to(torch.int32),
              (torch.rand((N, 16), generator=gen, device=device) * 0.0015 + 0.0005).half()) for _ in range(2)]
    layout = native.head_layout(64, N)
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    result = {}
    for m in rows:
        x = torch.randn((m, 2048), generator=gen, device=device).to(torch.bfloat16)
        out = torch.empty((m, N), dtype=torch.bfloat16, device=device)
        call = lambda i: native.head_out(x, *banks[i % 2], ws, out, flags, 2)
        for i in range(4):
            call(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(steps):
            call(i)
        b.record()
        torch.cuda.synchronize()
        with native.KernelTimer('head_w8_mfma') as kt:
            for i in range(steps):
                call(i)
            torch.cuda.synchronize()
            _, kms = kt.read('head_w8_mfma')
        weight_bytes = N * 2048 + N * 16 * 2
        result[str(m)] = dict(us_per_call=graph_ms(call, steps) * 1e3, us_per_call_eager=a.elapsed_time(b) / steps * 1e3,
                              kernel_us=kms * 1e3, weight_gbs=weight_bytes / (kms * 1e-3) / 1e9)
    if int(flags.item()):
        raise RuntimeError(f'native flags raised by the W8 head: {int(flags.item())}')
    return result


def copy_calibration(device):
    """A plain 256 MiB device-to-device copy, ten times (PMC scale factor)."""
    import torch
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({'copy_bytes': n, 'copies': 10}))


def cpu_model():
    """The host CPU's model name (lscpu's "Model name", read from /proc/cpuinfo)."""
    try:
        for line in Path('/proc/cpuinfo').read_text().splitlines():
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def _median_seconds(fn, warmup, reps):
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_baseline():
    """The reference's dequant + matmul semantics as PyTorch CPU eager
    (oracle/cpu_eager.py) on the host cores, per benchmark configuration:
    median of `reps` after `warmup` runs.  A reported baseline, not a target."""
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle import cpu_eager as CE
    threads = torch.get_num_threads()
    layer = CE.random_layer(7)
    gen = torch.Generator().manual_seed(8)
    dense_bank = CE.random_bank(gen, 0, DENSE_N, 2048)
    head_bank = CE.random_bank(gen, 0, HEAD_N, 2048)
    rank = torch.randperm(256, generator=torch.Generator().manual_seed(31)).float() + 1.0
    zipf = lambda s: -s * torch.log(rank)
    xs = {t: torch.randn((t, 2048), generator=gen).to(torch.bfloat16) for t in (1, 32, 1120, 8192)}
    configs = {}

    def record(name, tokens, seconds, sample, **extra):
        configs[name] = dict(tokens_per_s=tokens / seconds, ms=seconds * 1e3, sample=sample, **extra)

    t = _median_seconds(lambda: CE.dense(xs[1], *dense_bank), 2, 5)
    record('dense_1x6144x2048', 1, t, 'median of 5 after 2 warm-ups')
    t = _median_seconds(lambda: CE.moe_layer(xs[1], layer), 2, 5)
    record('moe_n1', 1, t, 'median of 5 after 2 warm-ups')
    t = _median_seconds(lambda: CE.moe_layer(xs[32], layer), 1, 3)
    record('moe_n32', 32, t, 'median of 3 after 1 warm-up')
    t = _median_seconds(lambda: CE.moe_layer(xs[1120], layer, zipf(1.1)), 1, 3)
    record('moe_n1120_zipf1.1', 1120, t, 'median of 3 after 1 warm-up')
    t = _median_seconds(lambda: CE.dense(xs[1120], *dense_bank), 1, 3)
    record('dense_1120x6144x2048', 1120, t, 'median of 3 after 1 warm-up')
    t = _median_seconds(lambda: CE.moe_layer(xs[8192], layer, zipf(1.3)), 0, 1)
    record('moe_n8192_zipf1.3', 8192, t, 'one run (after the smaller configurations warmed the pool)')
    t = _median_seconds(lambda: CE.dense(xs[8192][-32:].contiguous(), *head_bank), 0, 1)
    record('lm_head_32x151936', 32, t, 'one run')
    n1 = configs['moe_n1']
    return dict(value=n1['tokens_per_s'], unit='tokens/s', cores=threads, kind='port',
                sample='one N=1 MoE layer (router softmax/top-8, 8 routed + shared expert), PyTorch CPU eager fp32 '
                       'dequantise + H128 + matmul per call, median of 5; every configuration in per_config',
                cpu_model=cpu_model(), os_cpu_count=os.cpu_count(),
                affinity_cpus=len(os.sched_getaffinity(0)), torch_threads=threads, per_config=configs)


def oracle_timing(seconds):
    """The bit-exact numpy oracle (the correctness checker, not a baseline):
    single-token layers repeated for about `seconds`."""
    import numpy as np
    sys.path.insert(0, str(ROOT))
    sys.path.insert(0, str(ROOT / 'tests'))
    from oracle import ornith_oracle as O
    from _ornith import LazyExperts, bf16_normal, moe_weights
    from ornith_g256 import tables
    silu, sigmoid = tables.load_numpy()
    w = moe_weights(7)
    rng = np.random.default_rng(8)
    s13, s2 = w['s13'].expert(), w['s2'].expert()
    runs, t0 = 0, time.perf_counter()
    while True:
        x = bf16_normal(rng, (1, 2048))
        logits = O.router_logits(x, np.concatenate([w['router'], w['gate']]))
        rw, ids, _ = O.softmax_topk(logits[:, :256])
        O.routed_layer_shared(x, rw, ids, LazyExperts(w['w13']), w['w13'].sbits, w['w13'].obits,
                              LazyExperts(w['w2']), w['w2'].sbits, w['w2'].obits, *s13, *s2,
                              O.f32_to_bf16(logits[:, 256]), silu, sigmoid)
        runs += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return dict(tokens_per_s=runs / el, layers=runs, seconds=el, threads=1,
                what='numpy A8-exact oracle, single-token layers with shared expert (element-wise numpy, one thread)')


def binding_roof(T, unique, ms):
    """Per-layer roofline: t_mem = algorithmic bytes / HBM peak, t_mfma =
    algorithmic MACs x 2 / matrix peak (int8, the arithmetic used; bf16 for
    reference), binding = the larger; fractions = roof time / measured."""
    bytes_, flops = algorithmic(T, unique)
    t_mem = bytes_ / (HBM_PEAK_GBS * 1e9)
    t_int8 = flops / (INT8_PEAK_TOPS * 1e12)
    t_bf16 = flops / (BF16_PEAK_TFLOPS * 1e12)
    t = ms * 1e-3
    return dict(algorithmic_bytes=bytes_, algorithmic_ops=flops, t_mem_us=t_mem * 1e6, t_mfma_int8_us=t_int8 * 1e6,
                t_mfma_bf16_us=t_bf16 * 1e6, binding='hbm' if t_mem >= t_int8 else 'mfma',
                frac_binding=max(t_mem, t_int8) / t, frac_hbm=t_mem / t, frac_mfma_int8=t_int8 / t,
                frac_mfma_bf16=t_bf16 / t)


def main():
    args = parse()
    if args.gpus != 1:
        print(f'bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU expert-parallel '
              f'path is not part of this library.', file=sys.stderr)
        sys.exit(2)
    import torch
    from ornith_g256 import native, synthetic, tables
    dev = torch.device('cuda:0')
    if args.copy_calibration:
        copy_calibration(dev)
        return
    native.lib()
    if args.part == 'head':
        print(json.dumps({'lm_head_32x151936_us': head_ms(dev, args.steps) * 1e3}))
        return
    if args.part == 'w8head':
        print(json.dumps({'w8_head_248320': w8_head_us(dev, steps=args.steps)}))
        return
    if args.part == 'gateup-bf16-model':
        print(json.dumps({'gateup_bf16_model': gateup_bf16_model_us(dev, args.steps)}))
        return
    if args.part == 'dense':
        wall1, device1, graph1 = dense_prefill_ms(1, dev, 48)
        print(json.dumps({'dense_6144x2048_1120_us': dense_prefill_ms(1120, dev, args.steps) * 1e3,
                          'dense_6144x2048_1_us': wall1 * 1e3, 'dense_6144x2048_1_device_us': device1 * 1e3,
                          'dense_6144x2048_1_graph_us': graph1 * 1e3}))
        return
    silu, sigmoid = tables.load(dev)
    layers = [synthetic.moe_layer(10_000 + i, dev) for i in range(args.layers)]
    torch.cuda.synchronize()

    zipf = {1120: 1.1, 8192: 1.3}      # router-bias skew of the prefill workloads
    bias_of = lambda T: synthetic.zipf_bias(zipf[T], 31, dev) if T in zipf else None
    runner = LayerRunner(layers, args.tokens, dev, silu, sigmoid, bias_of(args.tokens))
    ms = runner.time_steps(args.steps, args.warmup)
    runner.check_flags()
    unique = runner.routed_experts_touched()
    runner.check_flags()
    times = runner.kernel_times(args.steps)
    runner.check_flags()
    bytes_, flops = algorithmic(args.tokens, unique)
    layer_gbs = bytes_ / (ms * 1e-3) / 1e9

    per_tokens = {}
    for t in [int(v) for v in args.extra_tokens.split(',') if v]:
        if t == args.tokens:
            continue
        r = LayerRunner(layers, t, dev, silu, sigmoid, bias_of(t))
        tms = r.time_steps(max(args.layers, 40), 0)
        r.check_flags()
        u = r.routed_experts_touched()
        r.check_flags()
        b, f = algorithmic(t, u)
        kt = r.kernel_times(len(layers))
        r.check_flags()
        entry = dict(tokens_per_s=t / (tms * 1e-3), us_per_layer=tms * 1e3, unique_experts=u,
                     router_zipf_s=zipf.get(t), hbm_frac=b / (tms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     roofline=roofline(kt, t, u), layer_roof=binding_roof(t, u, tms),
                     kernels_us={n: v[1] * 1e3 for n, v in kt.items()})
        if t == 1120:
            entry['dense_6144x2048_us'] = dense_prefill_ms(t, dev) * 1e3
        if t == 8192:
            entry['lm_head_32x151936_us'] = head_ms(dev) * 1e3
        per_tokens[str(t)] = entry
        del r
    heads = {'w8_248320x2048': w8_head_us(dev)}
    per_tokens[str(args.tokens)] = dict(tokens_per_s=args.tokens / (ms * 1e-3), us_per_layer=ms * 1e3,
                                        unique_experts=unique, hbm_frac=layer_gbs / HBM_PEAK_GBS,
                                        layer_roof=binding_roof(args.tokens, unique, ms),
                                        kernels_us={n: v[1] * 1e3 for n, v in times.items()})
    if args.tokens == 1:
        wall1, device1, graph1 = dense_prefill_ms(1, dev, 48)
        per_tokens['1']['dense_6144x2048_us'] = wall1 * 1e3
        per_tokens['1']['dense_6144x2048_device_us'] = device1 * 1e3
        per_tokens['1']['dense_6144x2048_graph_us'] = graph1 * 1e3

    result = {
        'metric': 'MoE layer tokens/s',
        'value': args.tokens / (ms * 1e-3),
        'unit': 'tokens/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': ms,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'int8xu4 dot, fp32 tree (A8)',
        'data': 'synthetic (seeded, benchmark distributions); random-init weights of the Ornith MoE layer shape',
        'config': {'workload': f'routed MoE layer decode N={args.tokens}: E256 top-8 H2048 I512, G256 4-bit '
                               f'gate-up/down + always-on shared expert, router softmax/top-8',
                   'tokens': args.tokens, 'layers_cycled': args.layers},
        'roofline': roofline(times, args.tokens, unique),
        'layer_hbm_frac': layer_gbs / HBM_PEAK_GBS,
        'per_tokens': per_tokens,
        'heads': heads,
    }
    if not args.no_cpu_baseline:
        result['cpu_baseline'] = cpu_baseline()
        result['oracle'] = oracle_timing(args.oracle_seconds)
    print(json.dumps(result))


if __name__ == '__main__':
    main()
