"""The permutation scratch, read back from the workspace after a layer call.

The prefill path (T > 32) sorts the routes into bank segments
(routed_storage_n32_prefill.h:19-42 computes the same counts, offsets and
per-expert route lists; its list order is atomic, this library's is stable).
Here the scratch the kernels wrote is compared with the oracle's ``permute``
on the ids the kernels themselves produced (the layer entry's router + top-8,
and the routed entry's caller ids with duplicates and invalid entries):

  * per-16-token-block running counts per bank (the scan's output);
  * per-bank counts and the exclusive offsets (bank 256 = shared expert);
  * the permuted route list: ascending route index within each bank, the
    shared routes R + t after the routed ones;
  * the segment table {bank, first, count, tile_base} of the non-empty
    banks and the number of segments;
  * the 64-route m-tile descriptors {bank, first route, rows, tile in
    segment} and their number.

The workspace offsets follow the library's workspace plan: the permutation
scratch starts at the first 256-byte boundary after ``final_f32`` (T x 2048
fp32) and is carved into 256-byte aligned arrays in the order above.
"""
import numpy as np
import pytest

from _ornith import bf16_normal, from_dev, moe_weights, random_routing, to_dev
from oracle import ornith_oracle as O

pytestmark = pytest.mark.gpu

E, BANKS, TOP, PERM_TOKENS, TILE_ROWS = 256, 257, 8, 16, 64


def _a256(n):
    return (n + 255) & ~255


def _carve(ws, base, Tcap, shared):
    """Views of the permutation scratch inside the workspace bytes."""
    rcap = Tcap * TOP
    rall = rcap + (Tcap if shared else 0)
    blocks = (Tcap + PERM_TOKENS - 1) // PERM_TOKENS
    sizes = [('block_counts', blocks * E), ('counts', BANKS), ('offsets', BANKS + 1), ('routes', rall),
             ('segments', BANKS * 4), ('meta', 4), ('tiles', (rall // TILE_ROWS + BANKS + 10) * 4)]
    out, off = {}, base
    for name, n in sizes:
        out[name] = ws[off:off + 4 * n].view(np.int32)
        off += _a256(4 * n)
    return out


def _expected(ids, T, shared):
    R = T * TOP
    ids = np.asarray(ids, np.int32).reshape(-1)
    counts, offsets, routes = O.permute(ids)
    s = T if shared else 0
    counts = np.append(counts, s).astype(np.int32)
    offsets = np.append(offsets, offsets[-1] + s).astype(np.int32)
    routes = np.concatenate([routes, R + np.arange(s, dtype=np.int32)])
    # segments of the non-empty banks, with each bank's first m-tile
    ntile = (counts + TILE_ROWS - 1) // TILE_ROWS
    tile_base = np.concatenate([[0], np.cumsum(ntile)]).astype(np.int32)
    segs = [(b, offsets[b], counts[b], tile_base[b]) for b in range(BANKS) if counts[b] > 0]
    tiles = [(b, offsets[b] + k * TILE_ROWS, min(TILE_ROWS, counts[b] - k * TILE_ROWS), k)
             for b in range(BANKS) for k in range(ntile[b])]
    # running count of each bank over the earlier 16-token blocks
    nblocks = (T + PERM_TOKENS - 1) // PERM_TOKENS
    valid = (ids >= 0) & (ids < E)
    per_block = np.zeros((nblocks, E), np.int64)
    np.add.at(per_block, (np.arange(R)[valid] // (PERM_TOKENS * TOP), ids[valid]), 1)
    before = (np.cumsum(per_block, axis=0) - per_block).astype(np.int32)
    return counts, offsets, routes, np.array(segs, np.int32).reshape(-1, 4), \
        np.array(tiles, np.int32).reshape(-1, 4), before


def _check_scratch(p, ids, T, shared):
    counts, offsets, routes, segs, tiles, before = _expected(ids, T, shared)
    nblocks = before.shape[0]
    np.testing.assert_array_equal(p['counts'], counts)
    np.testing.assert_array_equal(p['offsets'], offsets)
    live = int(offsets[-1])
    np.testing.assert_array_equal(p['routes'][:live], routes)
    assert int(p['meta'][0]) == len(segs)
    np.testing.assert_array_equal(p['segments'][:4 * len(segs)].reshape(-1, 4), segs)
    assert int(p['meta'][1]) == len(tiles)
    np.testing.assert_array_equal(p['tiles'][:4 * len(tiles)].reshape(-1, 4), tiles)
    np.testing.assert_array_equal(p['block_counts'][:nblocks * E].reshape(nblocks, E), before)
    return counts


def _zipf_bias(s, seed):
    rank = np.random.default_rng(seed).permutation(256).astype(np.float64) + 1.0
    return (-s * np.log(rank)).astype(np.float32)


@pytest.fixture(scope='module')
def banks(device):
    w = moe_weights(1234)
    d = {k: (to_dev(w[k].codes, device), to_dev(w[k].meta, device)) for k in ('w13', 'w2', 's13', 's2')}
    return w, d


@pytest.mark.parametrize('T,zipf', [(33, None), (300, None), (300, 1.3), (1120, 1.1)])
def test_layer_permutation_scratch_matches_oracle(device, banks, shared_tables, T, zipf):
    import torch
    from ornith_g256 import native
    w, d = banks
    silu, sigmoid = shared_tables
    print(f'permutation scratch: layer T={T} zipf={zipf}', flush=True)
    rng = np.random.default_rng(9100 + T)
    x = to_dev(bf16_normal(rng, (T, 2048)), device)
    bias = None if zipf is None else to_dev(_zipf_bias(zipf, 11), device)
    layout = native.routed_layout(T, 'layer')
    ws = torch.full((layout.workspace_bytes,), 0xA5, dtype=torch.uint8, device=device)   # no stale zeros
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((T, 8), dtype=torch.float32, device=device)
    ti = torch.empty((T, 8), dtype=torch.int32, device=device)
    sl = torch.empty((T,), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    native.moe_layer(x, to_dev(w['router'], device), bias, to_dev(w['gate'][0], device),
                     d['w13'][0], d['w13'][1], d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1],
                     d['s2'][0], d['s2'][1], to_dev(silu, device), to_dev(sigmoid, device),
                     ws, tw, ti, sl, out, flags, T)
    torch.cuda.synchronize()
    assert int(flags.item()) == 0
    ids = from_dev(ti)
    p = _carve(from_dev(ws), _a256(layout.final_f32 + T * 2048 * 4), T, shared=True)
    counts = _check_scratch(p, ids, T, shared=True)
    if zipf is not None:
        assert counts[:E].max() > TILE_ROWS      # a bank with several m-tiles
    print(f'  banks used {int((counts[:E] > 0).sum())}, top bank {int(counts[:E].max())} routes', flush=True)


def test_routed_entry_permutation_with_edge_ids(device, banks):
    """Caller ids: duplicates within a token, padding (-1) and out-of-range
    ids (skipped and flagged), one bank with more than 64 routes."""
    import torch
    from ornith_g256 import native
    w, d = banks
    T = 70
    print(f'permutation scratch: routed entry T={T} edge ids', flush=True)
    rng = np.random.default_rng(9177)
    x = to_dev(bf16_normal(rng, (T, 2048)), device)
    rw, ids = random_routing(rng, T)
    ids[ids == 3] = 4                                  # bank 3 only in slot 0: > 64 routes
    ids[:, 0] = 3
    ids[2, :] = 9                                      # a token naming one expert eight times
    ids[4, 5] = -1                                     # padding
    ids[6, 2] = 300                                    # invalid: skipped, flag 4
    ids[8, 7] = -2                                     # invalid: skipped, flag 4
    layout = native.routed_layout(T)
    ws = torch.full((layout.workspace_bytes,), 0x5A, dtype=torch.uint8, device=device)
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    st = native.lib().ornith_routed_direct_launch(
        *[native.ptr(t) for t in (x, to_dev(rw, device), to_dev(ids, device), d['w13'][0], d['w13'][1],
                                  d['w2'][0], d['w2'][1], ws)],
        ws.numel(), native.ptr(out), native.ptr(flags), T, T, native.stream(x))
    assert st == 0
    torch.cuda.synchronize()
    assert int(flags.item()) & 4
    p = _carve(from_dev(ws), _a256(layout.final_f32 + T * 2048 * 4), T, shared=False)
    counts = _check_scratch(p, ids, T, shared=False)
    assert counts[3] > TILE_ROWS and counts[9] >= 8
