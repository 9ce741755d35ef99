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
reports N=32 and N=1120 under "per_tokens".
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
BF16_PEAK_TFLOPS = 2500.0
EXPERT_BYTES = 1024 * 2048 // 2 + 4 * 1024 * 8 + 2048 * 512 // 2 + 4 * 2048 * 2   # 1,622,016
ROUTER_BYTES = 256 * 2048 * 2 + 2048 * 2


def parse():
    p = argparse.ArgumentParser()
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=200)
    p.add_argument('--warmup', type=int, default=40)
    p.add_argument('--tokens', type=int, default=1)
    p.add_argument('--layers', type=int, default=40)
    p.add_argument('--extra-tokens', default='32,1120')
    p.add_argument('--cpu-seconds', type=float, default=15.0)
    p.add_argument('--no-cpu-baseline', action='store_true')
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
        ids = self.ti.cpu()
        return int(ids.unique().numel())


def algorithmic(T, unique):
    """Compulsory bytes and flops of one layer (touched experts + shared + router + I/O)."""
    bytes_ = (unique + 1) * EXPERT_BYTES + ROUTER_BYTES + T * 2048 * 2 * 2
    flops = 2 * (T * 9 * (1024 * 2048 + 2048 * 512) + T * 257 * 2048)
    return bytes_, flops


def cpu_baseline(seconds):
    """The CPU oracle (numpy restatement of the reference A8 layer) on the host
    cores: one N=1 layer with a shared expert, repeated for about `seconds`."""
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
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get('num_threads', 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = 1
    return dict(value=runs / el, unit='tokens/s', cores=threads, kind='port',
                sample=f'{runs} single-token MoE layers (router, top-8, 8 routed + shared expert, A8 exact) '
                       f'in {el:.1f}s, numpy oracle, fresh expert unpacking per layer')


def main():
    args = parse()
    if args.gpus != 1:
        print(f'bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU expert-parallel '
              f'path is not part of this build.', file=sys.stderr)
        sys.exit(2)
    import torch
    from ornith_g256 import native, synthetic, tables
    dev = torch.device('cuda:0')
    native.lib()
    silu, sigmoid = tables.load(dev)
    layers = [synthetic.moe_layer(10_000 + i, dev) for i in range(args.layers)]
    torch.cuda.synchronize()

    runner = LayerRunner(layers, args.tokens, dev, silu, sigmoid)
    ms = runner.time_steps(args.steps, args.warmup)
    if int(runner.flags.item()) != 0:
        raise RuntimeError(f'native flags raised: {int(runner.flags.item())}')
    unique = runner.routed_experts_touched()
    bytes_, flops = algorithmic(args.tokens, unique)
    layer_gbs = bytes_ / (ms * 1e-3) / 1e9

    per_tokens = {}
    for t in [int(v) for v in args.extra_tokens.split(',') if v]:
        r = LayerRunner(layers, t, dev, silu, sigmoid)
        tms = r.time_steps(max(args.layers, 40), 0)
        u = r.routed_experts_touched()
        b, f = algorithmic(t, u)
        per_tokens[str(t)] = dict(tokens_per_s=t / (tms * 1e-3), us_per_layer=tms * 1e3, unique_experts=u,
                                  hbm_frac=b / (tms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                  mfma_bf16_frac=f / (tms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS)
        del r
    per_tokens[str(args.tokens)] = dict(tokens_per_s=args.tokens / (ms * 1e-3), us_per_layer=ms * 1e3,
                                        unique_experts=unique, hbm_frac=layer_gbs / HBM_PEAK_GBS)

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
        'roofline': {'bound': 'hbm', 'achieved': layer_gbs, 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': layer_gbs / HBM_PEAK_GBS, 'traffic': None, 'kernel': 'whole layer'},
        'per_tokens': per_tokens,
    }
    if not args.no_cpu_baseline:
        result['cpu_baseline'] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result))


if __name__ == '__main__':
    main()
