"""GPU: decode-layer composite and the MLI lag schedule (eager and hipGraph).

Invariants (the reference's tests/test_equivalence.py:45-64 gate, fused ==
reference with identical index sets, carried over to streams and graphs):
  * the schedule (eager and captured) equals the
    serial composition of the standalone kernels, bitwise, outputs and selections;
  * layer i attends exactly layer i-1's selection (lag), layer 0 the given set;
  * at lag depth k and under IndexCache patterns each layer attends the
    selection the oracle's depth-k FIFO names;
  * replaying the graph with eager work in between reproduces it bitwise;
  * the composite's selection equals the oracle top-k of its own scores,
    mapped to KV slots.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

LENS = [5000, 3100, 70]


def _stack(dev, n_layers=3, indexer_every=1):
    from lagged_indexer_dsa_amd import synthetic as S

    pt, num_pages = S.make_page_table(LENS, seed=1, device=dev)
    # a fixed split count: the shared launch and the standalone attention
    # would otherwise pick their own (the split count is part of the rounding)
    layers = [S.make_decode_layer(LENS, seed=10 + i, device=dev, page_table=pt, num_pages=num_pages,
                                  indexer=(i % indexer_every == 0), nsplit=16)
              for i in range(n_layers)]
    first = S.random_selection(LENS, 2048, pt, seed=99, device=dev)
    return layers, first, pt


def _serial(layers, first):
    """Reference composition on one stream with the standalone ops."""
    from lagged_indexer_dsa_amd import ops

    outs, sels = [], []
    carried = first
    for i, L in enumerate(layers):
        att = first if i == 0 else carried
        if L.has_indexer:
            sc = ops.indexer_scan(L.q_fp8, L.w, L.index_k, L.page_table, L.seq_lens, L.slab_stride)
            sel = ops.topk(sc, L.seq_lens, L.topk, page_table=L.page_table)
            sels.append(sel)
            new_carried = sel
        else:
            sels.append(None)
            new_carried = carried
        outs.append(ops.sparse_mla_decode(L.q_bf16, L.kv_pool, att, nsplit=L.nsplit))
        carried = new_carried
    torch.cuda.synchronize()
    return outs, sels


def _snap(layers):
    torch.cuda.synchronize()
    return ([L.out.clone() for L in layers],
            [L.next_idx.clone() if L.has_indexer else None for L in layers])


def _eq(a, b):
    return torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b)


def test_decode_layer_composite_matches_ops_and_oracle(dev):
    from lagged_indexer_dsa_amd import ops

    print("[mli] composite", flush=True)
    layers, first, pt = _stack(dev, n_layers=1)
    L = layers[0]
    L.run(attend_idx=None)          # baseline DSA: attend own fresh selection
    torch.cuda.synchronize()
    sc = L.scores.cpu().numpy()
    ref_sel = O.topk_select(sc, np.array(LENS), 2048, page_table=pt.cpu().numpy())
    assert np.array_equal(L.next_idx.cpu().numpy(), ref_sel)
    out = ops.sparse_mla_decode(L.q_bf16, L.kv_pool, L.next_idx, nsplit=L.nsplit)
    torch.cuda.synchronize()
    assert _eq(out, L.out)


@pytest.mark.parametrize("indexer_every", [1, 2])
def test_mli_eager_and_graph_equal_serial(dev, indexer_every):
    from lagged_indexer_dsa_amd.decode import MLISchedule

    print(f"[mli] eager/graph indexer_every={indexer_every}", flush=True)
    layers, first, pt = _stack(dev, n_layers=4, indexer_every=indexer_every)
    ref_out, ref_sel = _serial(layers, first)

    sched = MLISchedule(layers, first)
    for L in layers:
        L.out.zero_(); L.next_idx.fill_(-7)
    sched.run_eager()
    e_out, e_sel = _snap(layers)
    for i in range(len(layers)):
        assert _eq(e_out[i], ref_out[i]), f"eager layer {i} output"
        if ref_sel[i] is not None:
            assert _eq(e_sel[i], ref_sel[i]), f"eager layer {i} selection"

    # many replays: the split merge and the fused top-k hand data between
    # workgroups of one launch; every replay must reproduce the serial result
    for rep in range(20):
        for L in layers:
            L.out.zero_(); L.next_idx.fill_(-7)
        torch.cuda.synchronize()
        print(f"[mli] graph replay {rep}", flush=True)
        sched.replay()
        g_out, g_sel = _snap(layers)
        for i in range(len(layers)):
            assert _eq(g_out[i], ref_out[i]), f"graph replay {rep} layer {i} output"
            if ref_sel[i] is not None:
                assert _eq(g_sel[i], ref_sel[i]), f"graph replay {rep} layer {i} selection"
        _ = torch.randn(1000, device=dev).sum().item()   # eager work between replays
    sched.close()


def test_mli_layer_attends_previous_selection(dev):
    from lagged_indexer_dsa_amd import ops
    from lagged_indexer_dsa_amd.decode import MLISchedule

    print("[mli] lag consumption", flush=True)
    layers, first, pt = _stack(dev, n_layers=3)
    MLISchedule(layers, first).run_eager()
    torch.cuda.synchronize()
    for i in range(1, 3):
        o = ops.sparse_mla_decode(layers[i].q_bf16, layers[i].kv_pool, layers[i - 1].next_idx, nsplit=16)
        torch.cuda.synchronize()
        assert _eq(o, layers[i].out)
    o0 = ops.sparse_mla_decode(layers[0].q_bf16, layers[0].kv_pool, first, nsplit=16)
    torch.cuda.synchronize()
    assert _eq(o0, layers[0].out)


@pytest.mark.parametrize("depth,pattern,cold", [(1, "FFSFSFF", False), (2, "FFFFFF", True),
                                                 (2, "FFSFSFFS", False), (3, "FSFFSSFF", True)])
def test_mli_lag_depth_and_indexcache_pattern(dev, depth, pattern, cold):
    """Each layer's output equals the standalone attention over the selection
    the oracle's depth-k FIFO names for it (P:1835-1904, P:3020-3100), eager
    and in a replayed graph; the selections equal the serial ones."""
    from lagged_indexer_dsa_amd import ops
    from lagged_indexer_dsa_amd import synthetic as S
    from lagged_indexer_dsa_amd.decode import MLISchedule

    print(f"[mli] depth={depth} pattern={pattern} cold={cold}", flush=True)
    pt, num_pages = S.make_page_table(LENS, seed=1, device=dev)
    layers = [S.make_decode_layer(LENS, seed=40 + i, device=dev, page_table=pt, num_pages=num_pages,
                                  indexer=(c == "F"), nsplit=16)
              for i, c in enumerate(pattern)]
    first = layers[0].next_idx if cold else S.random_selection(LENS, 2048, pt, seed=98, device=dev)
    src = O.mli_attend_sources([c == "F" for c in pattern], 0 if cold else -1, depth)
    sched = MLISchedule(layers, first, lag_depth=depth)
    for mode in ("eager", "graph", "graph"):
        for L in layers:
            L.out.zero_(); L.next_idx.fill_(-7)
        torch.cuda.synchronize()
        sched.run_eager() if mode == "eager" else sched.replay()
        outs, sels = _snap(layers)
        for i, L in enumerate(layers):
            if L.has_indexer:
                sc = ops.indexer_scan(L.q_fp8, L.w, L.index_k, L.page_table, L.seq_lens, L.slab_stride)
                ref_sel = ops.topk(sc, L.seq_lens, L.topk, page_table=L.page_table)
                torch.cuda.synchronize()
                assert _eq(sels[i], ref_sel), f"{mode} layer {i} selection"
            att = first if src[i] == -1 else sels[src[i]]
            ref = ops.sparse_mla_decode(L.q_bf16, L.kv_pool, att, nsplit=L.nsplit)
            torch.cuda.synchronize()
            assert _eq(outs[i], ref), f"{mode} layer {i} attends layer {src[i]}"
    sched.close()


def test_mli_large_batch_layers_equal_serial(dev):
    """>= 8 rows: each indexer layer is a scan launch, a select launch and an
    attention launch; outputs and selections equal the standalone ops."""
    from lagged_indexer_dsa_amd import synthetic as S
    from lagged_indexer_dsa_amd.decode import MLISchedule

    print("[mli] 8-row batch", flush=True)
    lens = [9000, 3000, 2048, 70, 5000, 12000, 800, 4097]
    pt, num_pages = S.make_page_table(lens, seed=3, device=dev)
    # a fixed split count: the shared launch would otherwise pick its own
    # (fewer splits per row at this batch), which rounds differently
    layers = [S.make_decode_layer(lens, seed=60 + i, device=dev, page_table=pt, num_pages=num_pages, nsplit=8)
              for i in range(3)]
    first = S.random_selection(lens, 2048, pt, seed=97, device=dev)
    ref_out, ref_sel = _serial(layers, first)
    sched = MLISchedule(layers, first)
    for mode in ("eager", "graph", "graph"):
        for L in layers:
            L.out.zero_(); L.next_idx.fill_(-7)
        torch.cuda.synchronize()
        sched.run_eager() if mode == "eager" else sched.replay()
        outs, sels = _snap(layers)
        for i in range(len(layers)):
            assert _eq(outs[i], ref_out[i]), f"{mode} layer {i} output"
            assert _eq(sels[i], ref_sel[i]), f"{mode} layer {i} selection"
    sched.close()


def test_large_batch_layer_attends_own_selection(dev):
    """>= 8 rows, attend_idx = NULL (baseline DSA): the attention launch
    follows the select launch and reads the fresh selection; the selection
    equals the oracle top-k of the layer's scores, the output equals the
    standalone attention over it at the default split count."""
    from lagged_indexer_dsa_amd import ops
    from lagged_indexer_dsa_amd import synthetic as S

    print("[mli] 9-row own selection", flush=True)
    lens = [9000, 3000, 2048, 70, 5000, 12000, 800, 4097, 1]
    pt, num_pages = S.make_page_table(lens, seed=5, device=dev)
    L = S.make_decode_layer(lens, seed=70, device=dev, page_table=pt, num_pages=num_pages)
    for rep in range(2):
        L.out.zero_(); L.next_idx.fill_(-7)
        L.run(attend_idx=None)
        torch.cuda.synchronize()
        ref_sel = O.topk_select(L.scores.cpu().numpy(), np.array(lens), 2048, page_table=pt.cpu().numpy())
        assert np.array_equal(L.next_idx.cpu().numpy(), ref_sel), f"rep {rep} selection"
        out = ops.sparse_mla_decode(L.q_bf16, L.kv_pool, L.next_idx)
        torch.cuda.synchronize()
        assert _eq(out, L.out), f"rep {rep} output"
