"""GPU: the plain scan as one index space over every row (scan_flat.hip).

Plain scans of >= 2 rows (dsa_indexer_scan, the first launch of a
large-batch layer) take every row's 64-token batches as one space cut in
equal workgroup shares, waves taking batches from an LDS counter.  The
per-token arithmetic is the per-row scan's, in the same order, so the two
forms must give the same bits; both are checked against the oracle
(rel 1e-4 of the row's max |score|, 5e-4 with the alternative MFMA form's
summation order; exact -inf past each row's length).
Cases: ragged rows with empty ones, many tiny rows (a share spanning
dozens of rows), the 1024-row maximum and 1025 rows (per-row form), every
index-head count and the alternative MFMA form, invalid page entries, a
slab that is not a multiple of 64, C4's 32 rows (sampled pages).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _cases as C
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _lib():
    from lagged_indexer_dsa_amd import _lib
    return _lib.load()


def _scan(d, slab, flat, variant=0):
    from lagged_indexer_dsa_amd import ops

    lib = _lib()
    lib.dsa_internal_set_flat_scan(flat)
    lib.dsa_internal_set_scan_variant(variant)
    try:
        out = ops.indexer_scan(d["q"], d["w"], d["pages"], d["pt"], d["lens"], slab)
        torch.cuda.synchronize()
    finally:
        lib.dsa_internal_set_flat_scan(1)
        lib.dsa_internal_set_scan_variant(0)
    return out.cpu().numpy()


def _check_oracle(case, got, slab, tol=1e-4):
    ref = O.indexer_scores(case["q"], case["w"], case["pages"], np.where(case["pt"] < 0, 0, case["pt"]),
                           case["lens"], slab)
    for b, n in enumerate(case["lens"]):
        n = int(min(n, slab))
        assert np.all(np.isneginf(got[b, n:])), f"row {b}: tail not -inf"
        if n:
            assert C.rel_err(got[b, :n].astype(np.float64), ref[b, :n]) < tol, f"row {b}"


CASES = [
    ("ragged", [1000, 64, 1, 0, 4099, 17, 0, 20000], 64, 0),
    ("tiny_rows", [int(x) for x in np.random.default_rng(3).integers(0, 200, 300)], 64, 0),
    ("max_rows", [100] * 1024, 64, 0),
    ("over_max_rows", [50] * 1025, 64, 0),
    ("hidx16", [3000, 5000, 70], 16, 0),
    ("hidx32", [3000, 5000, 70], 32, 0),
    ("hidx48_v1", [3000, 5000, 70], 48, 1),
    ("hidx64_v1", [9000, 1, 640], 64, 1),
]


@pytest.mark.parametrize("name,lens,hidx,variant", CASES, ids=[c[0] for c in CASES])
def test_flat_scan_equals_per_row_and_oracle(dev, name, lens, hidx, variant):
    print(f"[scan-flat] {name} rows={len(lens)} hidx={hidx} variant={variant}", flush=True)
    case = C.index_case(seed=len(lens) + hidx, lens=lens, hidx=hidx)
    slab = case["pt"].shape[1] * 64
    d = C.to_dev(case, dev)
    flat = _scan(d, slab, 1, variant)
    rows = _scan(d, slab, 0, variant)
    assert np.array_equal(flat.view(np.uint32), rows.view(np.uint32)), "flat and per-row scans differ"
    # the alternative MFMA form sums four 32-wide fp32 partials per head
    # (another order than the oracle's fp64 sums): 5e-4 of a row's max
    _check_oracle(case, flat, slab, 1e-4 if variant == 0 else 5e-4)


def test_flat_scan_invalid_pages_and_odd_slab(dev):
    lens = [300, 200, 0, 130]
    print(f"[scan-flat] invalid pages lens={lens}", flush=True)
    case = C.index_case(seed=7, lens=lens, hidx=64, pt_stride=8)
    slab = 455  # not a multiple of 64
    case["pt"][1, 1] = case["pages"].shape[0] + 10  # outside the pool: -inf, never read
    case["pt"][3, 0] = -1
    d = C.to_dev(case, dev)
    flat = _scan(d, slab, 1)
    rows = _scan(d, slab, 0)
    assert np.array_equal(flat.view(np.uint32), rows.view(np.uint32))
    assert np.all(np.isneginf(flat[1, 64:128])) and np.all(np.isneginf(flat[3, 0:64]))
    for b, n in enumerate(lens):
        assert np.all(np.isneginf(flat[b, n:]))


def test_flat_scan_c4_rows(dev):
    """C4's 32 rows (bench.py's draw): flat == per-row bitwise, 8 random
    pages of every row against the oracle."""
    from lagged_indexer_dsa_amd import ops
    from lagged_indexer_dsa_amd import synthetic as S

    g = torch.Generator().manual_seed(4000)
    lens = torch.randint(16384, 131073, (32,), generator=g).tolist()
    print(f"[scan-flat] C4 sum={sum(lens)}", flush=True)
    pt, num_pages = S.make_page_table(lens, seed=1000, device=dev)
    L = S.make_decode_layer(lens, seed=3000, device=dev, page_table=pt, num_pages=num_pages)
    lib = _lib()
    outs = []
    for flat in (1, 0):
        lib.dsa_internal_set_flat_scan(flat)
        try:
            L.scores.fill_(7.0)
            ops.indexer_scan(L.q_fp8, L.w, L.index_k, L.page_table, L.seq_lens, L.slab_stride, out=L.scores)
            torch.cuda.synchronize()
            outs.append(L.scores.cpu().numpy().copy())
        finally:
            lib.dsa_internal_set_flat_scan(1)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    sc = outs[0]
    rng = np.random.default_rng(5)
    for b, n in enumerate(lens):
        assert np.all(np.isneginf(sc[b, n:])), f"row {b}: tail"
        pg = np.sort(rng.choice(n // 64, size=8, replace=False))
        pages = L.index_k[L.page_table[b, torch.from_numpy(pg).to(dev)].long()].cpu().numpy()
        ref = O.indexer_scores(L.q_fp8[b:b + 1].cpu().numpy(), L.w[b:b + 1].cpu().numpy(), pages,
                               np.arange(pg.size, dtype=np.int32)[None, :], np.array([64 * pg.size]),
                               64 * pg.size)[0]
        pos = (64 * pg[:, None] + np.arange(64)[None, :]).reshape(-1)
        assert C.rel_err(sc[b, pos].astype(np.float64), ref) < 1e-4, f"row {b}"


def test_flat_scan_output_not_16_byte_aligned(dev):
    """A score slab starting 4 bytes past a 16-byte boundary (a view one
    float into a buffer): every row start is then off the 16-byte grid, so
    the staged runs go out as 4-byte stores; the same bits as an aligned
    slab, -inf tails included, and the float before the slab untouched."""
    from lagged_indexer_dsa_amd import ops

    lens = [300, 1000, 64, 0, 777]
    print(f"[scan-flat] unaligned output lens={lens}", flush=True)
    case = C.index_case(seed=11, lens=lens, hidx=64)
    slab = case["pt"].shape[1] * 64
    d = C.to_dev(case, dev)
    ref = _scan(d, slab, 1)
    big = torch.full((len(lens) * slab + 1,), 7.0, device=dev)
    out = big[1:].view(len(lens), slab)
    assert out.data_ptr() % 16 == 4
    ops.indexer_scan(d["q"], d["w"], d["pages"], d["pt"], d["lens"], slab, out=out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert big[0].item() == 7.0

