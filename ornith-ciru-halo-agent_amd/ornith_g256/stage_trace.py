"""Stage timeline of the single-token layer kernel across its 256 blocks.

Needs the stage-trace build (python -m ornith_g256._build --stage-trace),
which records, per block and call, the steady clock (100 MHz) at each stage
of layer1_kernel (include/ornith_timing.h lists the stages).  The layer runs
as in the benchmark: a captured graph of L calls on L distinct synthetic
layers (their weights exceed the 256 MB MALL), replayed R times.  For every
call the stamps are taken relative to the call's first block start; the
table gives, per stage, the median over calls of the p50, p90 and maximum
over blocks, in microseconds, plus the spacing of consecutive calls (last
output stored -> next call's first block start).

    python -m ornith_g256.stage_trace [--layers 40] [--rounds 5] [--json]

ORNITH_G256_TRACE_DIR names another directory holding a stage-trace build
(to compare two builds on one machine).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
from pathlib import Path

import numpy as np
import torch

from . import _build, native, synthetic

STAGES = ['block start', 'router row published', 'all logits seen', 'experts selected',
          'routed gate-up dots done', 'routed middle published', 'middle of slot 0 seen (down)',
          'middle of slot 7 seen (down)', 'shared middle seen (down)', 'down dots of slot 0 done',
          'output columns stored', 'shared middle published', 'speculative picks published',
          'shared gate logit seen (down)', 'gate-up dots of all four waves done']
CALLS, BLOCKS, SLOTS = 64, 256, 16


def _slot_of_block():
    """Routed slot of each block's gate-up unit (the kernel's XCD pairing:
    block L = 16q + 8h + x takes unit 2(8q + x) + h, slot = unit / 32)."""
    L = np.arange(BLOCKS)
    x, h, q = L & 7, (L >> 3) & 1, L >> 4
    return (2 * (8 * q + x) + h) >> 5


SLOT_OF_BLOCK = _slot_of_block()
TICK_US = 0.01                          # 100 MHz steady clock


def _calls(trace, seqs):
    """{seq: [256, 16] tick array (nan = stage not reached)} for the given seqs."""
    t = trace.reshape(CALLS, BLOCKS, SLOTS)
    out = {}
    for seq in seqs:
        slot = t[seq % CALLS]
        tag = (slot >> np.uint64(52)).astype(np.int64)
        ticks = (slot & np.uint64((1 << 52) - 1)).astype(np.float64)
        ok = (slot != 0) & (tag == (seq & 0xFFF))
        out[seq] = np.where(ok, ticks, np.nan)
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument('--layers', type=int, default=40)
    ap.add_argument('--rounds', type=int, default=5)
    ap.add_argument('--json', action='store_true')
    args = ap.parse_args(argv)
    if args.layers > CALLS:
        raise SystemExit(f'at most {CALLS} calls per replay')
    native.LIB_DIR = Path(os.environ.get('ORNITH_G256_TRACE_DIR', _build.TRACE_DIR))
    h = native.lib()
    dev = torch.device('cuda', 0)
    probe = torch.zeros(CALLS * BLOCKS * SLOTS, dtype=torch.int64, device=dev)
    st = h.ornith_mi355x_stage_trace_read(native.ptr(probe), probe.numel(), native.stream(probe))
    if st != 0:
        raise SystemExit(f'{native.library_path()} records no stage trace (status {st}); '
                         'build it with python -m ornith_g256._build --stage-trace')
    from .tables import load
    silu, sigmoid = load(dev)
    layers = [synthetic.moe_layer(10_000 + i, dev) for i in range(args.layers)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(1001)
    x = torch.randn((1, 2048), generator=gen, device=dev).to(torch.bfloat16)
    ws = torch.zeros(native.routed_layout(1, 'layer').workspace_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty((1, 2048), dtype=torch.bfloat16, device=dev)
    tw = torch.empty((1, 8), dtype=torch.float32, device=dev)
    ti = torch.empty((1, 8), dtype=torch.int32, device=dev)
    sl = torch.empty((1,), dtype=torch.bfloat16, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)

    def step(i):
        L = layers[i]
        native.moe_layer(x, L['router'], None, L['gate'], *L['w13'], *L['w2'], *L['s13'], *L['s2'], silu, sigmoid,
                         ws, tw, ti, sl, out, flags, 1)

    for i in range(args.layers):
        step(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(args.layers):
            step(i)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(graph):
        for i in range(args.layers):
            step(i)
    graph.replay()
    torch.cuda.synchronize()
    seq = 3 * args.layers                  # calls made so far on this workspace
    per_stage = [[] for _ in STAGES]
    per_slot = {}
    spacing, spans, replay_ms = [], [], []
    for _ in range(args.rounds):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        replay_ms.append(start.elapsed_time(end))
        h.ornith_mi355x_stage_trace_read(native.ptr(probe), probe.numel(), native.stream(probe))
        torch.cuda.synchronize()
        trace = probe.cpu().numpy().view(np.uint64)
        seqs = list(range(seq, seq + args.layers))
        seq += args.layers
        calls = _calls(trace, seqs)
        prev_end = None
        for q in seqs:
            c = calls[q]
            t0 = np.nanmin(c[:, 0])
            rel = (c - t0) * TICK_US
            for k in range(len(STAGES)):
                v = rel[:, k]
                v = v[~np.isnan(v)]
                if v.size:
                    per_stage[k].append((np.percentile(v, 50), np.percentile(v, 90), v.max(), v.size))
            for slot in range(8):
                sel = SLOT_OF_BLOCK == slot
                for k in (4, 14, 5):
                    v = rel[sel, k]
                    v = v[~np.isnan(v)]
                    if v.size:
                        per_slot.setdefault((slot, k), []).append((np.percentile(v, 50), v.max()))
            last = np.nanmax(c[:, 10])
            spans.append((last - t0) * TICK_US)
            if prev_end is not None:
                spacing.append((t0 - prev_end) * TICK_US)
            prev_end = last
    if int(flags.item()):
        raise SystemExit(f'native flags raised: {int(flags.item())}')
    rows = []
    for k, name in enumerate(STAGES):
        a = np.array(per_stage[k]) if per_stage[k] else np.zeros((0, 4))
        med = np.median(a, axis=0) if len(a) else [np.nan] * 4
        rows.append({'stage': k, 'name': name, 'p50_us': float(med[0]), 'p90_us': float(med[1]),
                     'max_us': float(med[2]), 'blocks': int(med[3]) if len(a) else 0})
    slots = {f'slot{sl}': {STAGES[k]: [float(x) for x in np.median(np.array(per_slot[(sl, k)]), axis=0)]
                           for k in (4, 14, 5) if (sl, k) in per_slot} for sl in range(8)}
    res = {'calls': len(spans), 'us_per_call_graph': float(np.median(replay_ms)) * 1e3 / args.layers,
           'kernel_span_us_median': float(np.median(spans)),
           'call_spacing_us_median': float(np.median(spacing)) if spacing else None, 'stages': rows,
           'per_slot_p50_max_us': slots}
    if args.json:
        print(json.dumps(res))
        return res
    print(f"calls {res['calls']}; graph time per call {res['us_per_call_graph']:.2f} us; "
          f"first block start -> last output stored {res['kernel_span_us_median']:.2f} us (median); "
          f"last output of a call -> first block of the next {res['call_spacing_us_median']:.2f} us")
    print('| stage | p50 (us) | p90 (us) | max (us) | blocks |')
    print('|---|---:|---:|---:|---:|')
    for r in rows:
        print(f"| {r['stage']} {r['name']} | {r['p50_us']:.2f} | {r['p90_us']:.2f} | {r['max_us']:.2f} | {r['blocks']} |")
    print()
    print('| routed slot | gate-up dots of wave 0 p50 / max (us) | of all four waves | middle published |')
    print('|---|---:|---:|---:|')
    for sl in range(8):
        d = slots[f'slot{sl}']
        cells = [d.get(STAGES[k], [np.nan] * 2) for k in (4, 14, 5)]
        print(f'| {sl} | ' + ' | '.join(f'{c[0]:.2f} / {c[1]:.2f}' for c in cells) + ' |')
    return res


if __name__ == '__main__':
    sys.exit(0 if main() else 1)
