"""bench.py pieces that need no GPU: the single-GPU guard and the algorithmic
byte counts the rooflines divide by."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / 'bench.py'), '--gpus', '2'], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode != 0
    assert 'one GPU' in (r.stdout + r.stderr)


def test_single_token_algorithmic_bytes():
    import bench
    # one N=1 layer: 8 routed banks + the shared expert, A8 activations,
    # fp32 middle rows, bf16 output (the figures the N=1 roofline divides by)
    _, gateup, _, unit = bench.kernel_cost('gateup1', 1, 8)
    _, down, _, _ = bench.kernel_cost('down1', 1, 8)
    assert unit == 'GB/s'
    assert gateup == 9 * 1_081_344 + 2048 + 9 * 512 * 4 == 9_752_576
    assert down == 9 * 540_672 + 9 * 512 * 4 + 2048 * 2 == 4_888_576
    # the one-launch single-token layer: every byte the layer must read or
    # write once (9 expert banks, router + shared gate row, x in, out)
    _, whole, _, unit = bench.kernel_cost('layer1', 1, 8)
    assert unit == 'GB/s'
    assert whole == 9 * (1_081_344 + 540_672) + 256 * 2048 * 2 + 2048 * 2 + 2048 * 2 * 2 == 15_659_008
    assert whole == bench.algorithmic(1, 8)[0]
    # prefill gate-up: at 1120 tokens the bytes bind (97 banks of codes, the
    # A8 input, the fp32 middle rows: 129 MB = 16.1 us at 8 TB/s against
    # 42.3 G int8 ops = 8.5 us at 5 POP/s); at 8192 the matrix cores
    # (2 ops per MAC over 9 routes per token)
    bound, nbytes, _, unit = bench.kernel_cost('gateup_mfma', 1120, 96)
    assert (bound, unit) == ('hbm', 'GB/s')
    assert nbytes == 97 * 1_081_344 + 1120 * 2048 + 9 * 1120 * 512 * 4
    bound, ops, _, unit = bench.kernel_cost('gateup_mfma', 8192, 101)
    assert (bound, unit) == ('mfma', 'TFLOP/s') and ops == 2 * 9 * 8192 * 1024 * 2048
    # the down projection writes fp32 route rows: bytes bind at both sizes
    assert bench.kernel_cost('down_mfma', 8192, 101)[0] == 'hbm'
