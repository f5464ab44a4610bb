"""GPU: large-batch layers whose attention rides in the scan launch.

From 8 rows a layer attending a set it does not produce runs its attention
in the plain scan's grid (scan_flat.hip, about a quarter of the CUs, 2-8
splits per (row, head group)) when the rows' capacity is large next to
B * topk; the select follows as its own launch.  Checked here against the
oracle and against the standalone attention, bitwise, at the split count
the launch used (one of 2, 4, 8): 16 and 32 heads (one and two head
groups), 8 and 16 rows, a short row among long ones, an empty row and a
row shorter than top-k, an attend set with padding (-1) entries, two
replays of the same layer (the scratch re-arms itself), every score the
same bits as the plain scan launch's (the scores start as NaN), selections
bit-exact against the oracle's top-k of the scores.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _cases import rel_err
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _oracle_attention_row(L, b, att):
    sl = att[b].long()
    valid = (sl >= 0) & (sl < L.kv_pool.shape[0])
    rows = L.kv_pool[sl[valid]].cpu().numpy()
    idx = np.arange(rows.shape[0], dtype=np.int32)[None, :]
    q = L.q_bf16[b:b + 1].float().cpu().numpy()
    return O.sparse_mla_decode(q, rows, idx, L.sm_scale)[0]


CASES = [
    ("b8_h16", [100000, 90000, 120000, 85000, 131072, 95000, 110000, 3000], 16),
    ("b8_h32", [100000, 90000, 120000, 85000, 131072, 95000, 110000, 99000], 32),
    ("b16_h16", [int(x) for x in np.random.default_rng(16).integers(60000, 131073, 16)], 16),
    # an empty row and a row shorter than top-k among long ones
    ("b8_empty_short", [120000, 0, 131072, 1500, 100000, 110000, 125000, 90000], 16),
]


@pytest.mark.parametrize("name,lens,heads", CASES, ids=[c[0] for c in CASES])
def test_riding_attention_matches_oracle(dev, name, lens, heads):
    from lagged_indexer_dsa_amd import _lib, ops
    from lagged_indexer_dsa_amd import synthetic as S

    print(f"[ride] {name} rows={len(lens)} heads={heads}", flush=True)
    _lib.sync_timeouts(reset=True)
    pt, num_pages = S.make_page_table(lens, seed=51, device=dev)
    L = S.make_decode_layer(lens, seed=52, device=dev, page_table=pt, num_pages=num_pages, heads=heads)
    att = S.random_selection(lens, 2048, pt, seed=53, device=dev)
    att[0, -100:] = -1  # padding entries in the attended set
    plain = ops.indexer_scan(L.q_fp8, L.w, L.index_k, L.page_table, L.seq_lens, L.slab_stride).view(torch.int32)
    for rep in range(2):
        L.out.zero_()
        L.next_idx.fill_(-7)
        L.scores.fill_(float("nan"))
        L.run(attend_idx=att)
        torch.cuda.synchronize()
        assert _lib.sync_timeouts() == 0, "a group wait expired"
        # every score written, the same bits as the plain scan launch
        assert torch.equal(L.scores.view(torch.int32), plain), f"rep {rep}: scores"
        ref_sel = O.topk_select(L.scores.cpu().numpy(), np.array(lens), L.topk, page_table=pt.cpu().numpy())
        assert np.array_equal(L.next_idx.cpu().numpy(), ref_sel), f"rep {rep}: selection"
        got = L.out.view(torch.int16)
        assert any(torch.equal(ops.sparse_mla_decode(L.q_bf16, L.kv_pool, att, nsplit=ns).view(torch.int16), got)
                   for ns in (2, 4, 8)), f"rep {rep}: not the standalone attention at 2, 4 or 8 splits"
        out = L.out.float().cpu().numpy()
        for b in range(len(lens)):
            err = rel_err(out[b], _oracle_attention_row(L, b, att))
            assert err < 2e-2, f"rep {rep} row {b}: attention rel err {err:.2e}"
