"""GPU parity: exact top-k select (dsa_topk) vs the oracle, bit-exact.

Given identical fp32 scores the selected indices must be identical, with
the lower index winning ties (the path's bar for index work).  Cases cover
the reference's select contract (attention_core.py:66-91): rows shorter
than k (sentinel/pad), non-finite scores, forced ties at the threshold,
all-equal rows (the threshold bin overflows the on-chip candidate buffer),
-0.0/+0.0, and the longest supported rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _gpu_topk(scores, lens, k, sorted_, pad=-1, pt=None, dev="cuda"):
    from lagged_indexer_dsa_amd import ops

    s = torch.from_numpy(np.ascontiguousarray(scores, dtype=np.float32)).to(dev)
    l = torch.from_numpy(np.asarray(lens, dtype=np.int32)).to(dev)
    p = None if pt is None else torch.from_numpy(pt).to(dev)
    out = ops.topk(s, l, k, sorted=sorted_, pad_value=pad, page_table=p)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check(scores, lens, k, sorted_, dev, pad=-1, pt=None):
    got = _gpu_topk(scores, lens, k, sorted_, pad, pt, dev)
    ref = O.topk_select(scores, np.asarray(lens), k, sorted_=sorted_, pad=pad, page_table=pt)
    bad = np.nonzero((got != ref).any(axis=1))[0]
    assert bad.size == 0, f"rows {bad[:5]} differ (first: got {got[bad[0]][:8]} ref {ref[bad[0]][:8]})"


@pytest.mark.parametrize("sorted_", [False, True])
def test_topk_random_ragged(dev, sorted_):
    rng = np.random.default_rng(1)
    lens = [8192, 2048, 2047, 100, 0, 1, 5000, 3000]
    print(f"[topk] random ragged sorted={sorted_}", flush=True)
    s = rng.standard_normal((len(lens), 8192)).astype(np.float32)
    _check(s, lens, 2048, sorted_, dev)


@pytest.mark.parametrize("sorted_", [False, True])
def test_topk_forced_ties(dev, sorted_):
    rng = np.random.default_rng(2)
    print(f"[topk] forced ties sorted={sorted_}", flush=True)
    # few distinct values: thousands of ties straddle the threshold
    s = rng.integers(-20, 20, (4, 20000)).astype(np.float32) * 0.25
    s[1] = np.round(rng.standard_normal(20000) * 8) / 8
    s[2, ::3] = -0.0
    s[2, 1::3] = 0.0
    _check(s, [20000, 19999, 20000, 7000], 2048, sorted_, dev)


@pytest.mark.parametrize("sorted_", [False, True])
def test_topk_all_equal_rows_overflow_path(dev, sorted_):
    print(f"[topk] all equal sorted={sorted_}", flush=True)
    s = np.full((3, 50000), 1.5, dtype=np.float32)
    s[1] = 0.0
    s[2, :] = 2.0
    s[2, 40000:] = 3.0   # 10000 above, the rest tied
    _check(s, [50000, 50000, 50000], 2048, sorted_, dev)


@pytest.mark.parametrize("sorted_", [False, True])
def test_topk_nonfinite(dev, sorted_):
    rng = np.random.default_rng(3)
    print(f"[topk] non-finite sorted={sorted_}", flush=True)
    s = rng.standard_normal((4, 6000)).astype(np.float32)
    s[0, rng.integers(0, 6000, 50)] = np.inf
    s[0, rng.integers(0, 6000, 50)] = np.nan
    s[1, 1000:] = -np.inf                   # fewer finite than k -> pads
    s[2, :] = -np.inf
    s[3, rng.integers(0, 6000, 3000)] = -np.inf
    _check(s, [6000] * 4, 2048, sorted_, dev, pad=6000)


def test_topk_page_slot_mapping(dev):
    rng = np.random.default_rng(4)
    print("[topk] slot mapping", flush=True)
    lens = [9000, 70000]
    s = rng.standard_normal((2, 70016)).astype(np.float32)
    pt = np.stack([rng.permutation(5000)[:1094] for _ in range(2)]).astype(np.int32)
    _check(s, lens, 2048, False, dev, pt=pt)


@pytest.mark.parametrize("k", [1, 7, 2048, 4096])
def test_topk_sizes_sorted(dev, k):
    rng = np.random.default_rng(5 + k)
    print(f"[topk] k={k}", flush=True)
    s = rng.standard_normal((2, 30000)).astype(np.float32)
    _check(s, [30000, 4000], k, True, dev)
    _check(s, [30000, 4000], k, False, dev)


@pytest.mark.parametrize("ctx", [131072, 196608, 262144])
def test_topk_max_sizes(dev, ctx):
    rng = np.random.default_rng(ctx)
    print(f"[topk] ctx={ctx}", flush=True)
    s = rng.standard_normal((2, ctx)).astype(np.float32)
    _check(s, [ctx, ctx - 5], 2048, False, dev)
    _check(s, [ctx, ctx - 5], 2048, True, dev)


def test_topk_rejects_bad_args(dev):
    from lagged_indexer_dsa_amd import ops
    from lagged_indexer_dsa_amd._lib import DsaError

    s = torch.zeros(1, 100, device=dev)
    l = torch.full((1,), 100, dtype=torch.int32, device=dev)
    with pytest.raises(DsaError):
        ops.topk(s, l, 5000, sorted=True)
    with pytest.raises(DsaError):
        ops.topk(s, l, 0)


def test_topk_undersized_buffers_rejected_before_launch(dev):
    from lagged_indexer_dsa_amd import ops

    print("[topk] undersized buffers", flush=True)
    sc = torch.zeros(2, 8192, device=dev)
    lens = torch.full((2,), 8192, dtype=torch.int32, device=dev)
    small = ops.topk_scratch(2, 4096, dev)
    with pytest.raises(RuntimeError):
        ops.topk(sc, lens, 2048, scratch=small)
    with pytest.raises(RuntimeError):
        ops.topk(sc, lens, 2048, out=torch.empty(2, 1024, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()


@pytest.mark.parametrize("k", [1, 2047, 8192])
def test_topk_position_order_large_k_and_lengths_past_slab(dev, k):
    """Position order runs the cooperative select: k up to its maximum, rows
    whose seq_len exceeds the slab (clamped) or is negative (empty)."""
    rng = np.random.default_rng(11 + k)
    print(f"[topk] position order k={k}", flush=True)
    s = rng.standard_normal((5, 40000)).astype(np.float32)
    s[3] = np.round(s[3] * 4) / 4           # ties at the threshold
    _check(s, [40000, 90000, 8192, 39999, -3], k, False, dev, pad=-5)


@pytest.mark.parametrize("k", [4096, 8192])
def test_topk_position_order_one_row_wide_lists(dev, k):
    """One long row with a large k: every workgroup of the launch holds a
    list too long for the 4-uint4 union, so the launch carries only the
    8-uint4 form of the cooperative select; ties at the threshold too."""
    rng = np.random.default_rng(29 + k)
    print(f"[topk] one row k={k}", flush=True)
    s = rng.standard_normal((1, 131072)).astype(np.float32)
    _check(s, [131072], k, False, dev)
    s[0] = np.round(s[0] * 8) / 8
    _check(s, [131072], k, False, dev)


@pytest.mark.parametrize("B", [64, 65, 300])
def test_topk_position_order_many_rows(dev, B):
    """64 rows (per-row workgroup plan), 65 and 300 rows (uniform split)."""
    rng = np.random.default_rng(B)
    print(f"[topk] position order B={B}", flush=True)
    s = rng.standard_normal((B, 6000)).astype(np.float32)
    lens = rng.integers(0, 6001, B)
    lens[: B // 4] = 6000
    pt = rng.integers(0, 100000, (B, 94)).astype(np.int32)
    _check(s, lens, 2048, False, dev)
    _check(s, lens, 2048, False, dev, pt=pt)


def test_topk_position_and_sorted_share_scratch(dev):
    """Alternating the two orders over one scratch buffer: each call leaves
    the scratch ready for the next."""
    from lagged_indexer_dsa_amd import ops

    rng = np.random.default_rng(21)
    print("[topk] shared scratch", flush=True)
    B, slab, k = 3, 50000, 2048
    lens = np.array([50000, 20000, 1000], dtype=np.int32)
    scratch = ops.topk_scratch(B, slab, dev)
    l = torch.from_numpy(lens).to(dev)
    for it in range(6):
        sorted_ = it % 2 == 1
        s = rng.standard_normal((B, slab)).astype(np.float32)
        out = ops.topk(torch.from_numpy(s).to(dev), l, k, sorted=sorted_, scratch=scratch)
        torch.cuda.synchronize()
        ref = O.topk_select(s, lens, k, sorted_=sorted_)
        assert np.array_equal(out.cpu().numpy(), ref), f"call {it} sorted={sorted_}"


@pytest.mark.parametrize("step", [1 / 8, 1 / 32, 1 / 128, 1 / 1024])
def test_topk_position_order_rounded_scores_long_rows(dev, step):
    """Scores rounded to a grid: the workgroups' list bins and their
    256-way sub-bins hold runs of exact ties, so a list bound may have to
    start above a whole sub-bin or bin (position order, long rows)."""
    rng = np.random.default_rng(int(1 / step))
    print(f"[topk] rounded scores step={step}", flush=True)
    s = (np.round(rng.standard_normal((3, 131072)) / step) * step).astype(np.float32)
    pt = np.stack([rng.permutation(4096)[:2048] for _ in range(3)]).astype(np.int32)
    _check(s, [131072, 100000, 65536], 2048, False, dev)
    _check(s, [131072, 100000, 65536], 2048, False, dev, pt=pt)


@pytest.mark.parametrize("k", [1000, 2000])
@pytest.mark.parametrize("ties", [False, True])
def test_topk_position_order_list_publish_forms(dev, k, ties):
    """More rows than the per-row workgroup plan takes (64), so every row
    has one workgroup and its own-key count is the row length: lengths that
    straddle the switch between the two list-publish forms (per-thread runs
    up to 2048 own keys, wave segments above), with and without ties at the
    threshold."""
    rng = np.random.default_rng(41 + k + ties)
    print(f"[topk] publish forms k={k} ties={ties}", flush=True)
    base = [2047, 2048, 2049, 2050, 2303, 4097, 9001, 16384]
    lens = (base * 38)[:300]
    s = rng.standard_normal((len(lens), 16384)).astype(np.float32)
    if ties:
        s = np.round(s * 4) / 4
    _check(s, lens, k, False, dev)


@pytest.mark.parametrize("sorted_", [False, True])
def test_topk_top_keys_packed_in_one_window(dev, sorted_):
    """The largest scores packed into one contiguous window of positions (a
    recent-token window), distinct values: the workgroup over the window
    holds far more selected keys than its list can carry, so the row must
    be resolved by the single-workgroup fallback; the window also straddles
    two workgroups' ranges and sits at the row's end."""
    rng = np.random.default_rng(77)
    print(f"[topk] packed window sorted={sorted_}", flush=True)
    lens = [131072, 131072, 100000]
    s = rng.standard_normal((3, 131072)).astype(np.float32)
    s[0, 50000:54000] += 10.0                          # one window
    s[1, 16384 - 1500:16384 + 1500] += 10.0            # straddles a workgroup edge
    s[2, 100000 - 3000:100000] += 10.0                 # the row's last positions
    _check(s, lens, 2048, sorted_, dev)
