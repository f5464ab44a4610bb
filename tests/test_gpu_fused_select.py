"""GPU: the top-k select fused into the decode launch's scan workgroups.

The layer composite (scan + select in one launch, no attend set) must give
the oracle's top-k of the scores it produced, mapped to KV slots, bit-exact
(reference select_topk, attention_core.py:66-91, ties to the lower index).
Covered: the cooperative select (all scan workgroups of a row; default) and
the single-workgroup select, fused into the scan launch (< 8 rows) and as a
select launch over the scan's scores (>= 8 rows), on ragged rows, rows of
<= topk tokens, rows
with many equal scores at the threshold, and rows whose threshold bin
overflows the candidate list (every score equal).  No group wait may expire.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _lib():
    from lagged_indexer_dsa_amd import _lib
    return _lib.load()


def _layer(dev, lens, seed, pattern=None):
    from lagged_indexer_dsa_amd import synthetic as S

    pt, num_pages = S.make_page_table(lens, seed=seed, device=dev)
    L = S.make_decode_layer(lens, seed=seed + 1, device=dev, page_table=pt, num_pages=num_pages)
    pages = L.index_k.view(num_pages, -1)
    if pattern in ("dup", "dup64"):  # every page repeats one of 8 (64) pages: many equal scores
        nsrc = 8 if pattern == "dup" else 64
        src = pages[:nsrc].clone()
        for p in range(num_pages):
            pages[p] = src[p % nsrc]
    elif pattern == "equal":  # every key and scale identical: all scores equal
        pages[:, :8192] = pages[0, :128].repeat(64)
        pages[:, 8192:].view(torch.float32).fill_(1.0)
    elif pattern is not None and pattern.startswith("window"):
        # a window of each row scores far above the rest: "window" 3000
        # tokens from len/3; "window_end" the last 4096 tokens (recent
        # tokens); "window_small" 1000 tokens (the rest of the top-K spread
        # over the row); "window_dup" the window over repeated pages (many
        # equal scores at the threshold)
        if pattern == "window_dup":
            src = pages[:8].clone()
            for p in range(num_pages):
                pages[p] = src[p % 8]
        scales = pages[:, 8192:].view(torch.float32)  # [page][token in page]
        ptc = pt.cpu().numpy()
        for r, n in enumerate(lens):
            a, w = {"window_end": (max(0, n - 4096), 4096), "window_small": (n // 2, 1000)}.get(pattern, (n // 3, 3000))
            for pos in range(a, min(n, a + w)):
                scales[int(ptc[r, pos // 64]), pos % 64] *= 50.0
    return L, pt


def _check(L, pt, lens):
    torch.cuda.synchronize()
    sc = L.scores.cpu().numpy()
    ref = O.topk_select(sc, np.array(lens), L.topk, page_table=pt.cpu().numpy())
    got = L.next_idx.cpu().numpy()
    assert np.array_equal(got, ref), f"first mismatch rows {np.nonzero((got != ref).any(1))[0][:4]}"


CASES = [
    ([131072], 0, None),
    ([5000, 3100, 70], 1, None),
    ([2048, 2049, 1], 2, None),
    ([20000, 9000], 3, "dup"),
    ([6000, 4097], 4, "equal"),
    # >= 8 rows: the indexer runs as a scan launch, then a select launch that
    # loads the scores; ragged, with rows at or below topk
    ([40000, 300, 2048, 17000, 1, 9000, 31000, 2049, 12000, 500, 26000, 4000], 5, None),
    ([9000, 7000, 3000, 12000, 2500, 8000, 6000, 11000, 5000], 6, "dup"),
    # zero-length rows (the length plan still gives each row a workgroup)
    ([0, 5000, 0, 3000], 7, None),
    # >= 8 rows, all scores equal: the score-loading select's histogram form
    ([9000] * 8 + [0], 8, "equal"),
    # 64 rows (the largest batch the length plan covers) and 65 (uniform)
    ([int(x) for x in np.random.default_rng(9).integers(1, 20000, 64)], 9, None),
    ([int(x) for x in np.random.default_rng(10).integers(1, 5000, 65)], 10, None),
    # long rows of repeated pages: runs of equal keys in the workgroups' list
    # bins and sub-bins
    ([131072], 11, "dup"),
    ([131072, 70000], 12, "dup64"),
    # the selected keys packed into one window of each row (a recent-token
    # window): the workgroups over it hold more than their lists carry, so
    # the cooperative select must find that and fall back
    ([131072], 13, "window"),
    ([131072, 70000, 9000], 14, "window"),
    ([20000] * 9, 15, "window"),
    ([131072], 16, "window_end"),
    ([131072, 65536], 17, "window_small"),
    ([131072], 18, "window_dup"),
    ([100000, 3000, 50000], 19, "window_end"),
    ([30000] * 10, 20, "window_small"),
]


@pytest.mark.parametrize("lens,seed,pattern", CASES)
@pytest.mark.parametrize("coop", [1, 0])
def test_fused_select_matches_oracle(dev, lens, seed, pattern, coop):
    lib = _lib()
    print(f"[fused-select] lens={lens} pattern={pattern} coop={coop}", flush=True)
    lib.dsa_internal_group_wait_timeouts(1)
    lib.dsa_internal_set_coop_select(coop)
    try:
        L, pt = _layer(dev, lens, 100 + seed, pattern)
        for rep in range(3):  # the scratch re-arms itself between calls
            L.next_idx.fill_(-7)
            L.run(attend_idx=None)
            _check(L, pt, lens)
    finally:
        lib.dsa_internal_set_coop_select(1)
    assert lib.dsa_internal_group_wait_timeouts(1) == 0


def test_fused_select_coop_equals_single(dev):
    lib = _lib()
    print("[fused-select] coop == single workgroup", flush=True)
    lens = [70000, 1500, 33000]
    L, pt = _layer(dev, lens, 7)
    lib.dsa_internal_set_coop_select(0)
    try:
        L.run(attend_idx=None)
        torch.cuda.synchronize()
        single = L.next_idx.clone()
        out_single = L.out.clone()
    finally:
        lib.dsa_internal_set_coop_select(1)
    L.next_idx.fill_(-7)
    L.run(attend_idx=None)
    torch.cuda.synchronize()
    assert torch.equal(single, L.next_idx)
    assert torch.equal(out_single.view(torch.int16), L.out.view(torch.int16))
    _check(L, pt, lens)
