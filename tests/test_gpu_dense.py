"""GPU: dense MLA decode and dense layers in the MLI schedule.

Reference semantics: a full-attention layer, and a DSA layer 0 under the
DENSE cold start, attend every causal key (model.py:51-59, 104-114;
attention_core.py:142-160).  Under the lag, layer L runs an indexer iff
layer L+1 is a DSA layer (model.py:61-71), so the last full layer of a dense
prefix carries the boundary indexer that seeds the first DSA layer.

Checked:
  * dsa_dense_mla_decode against the oracle's attention over every slot of
    the row (rel 2e-2 of max |out|), on ragged rows with a random page table,
    including rows longer than the old 16384-key limit;
  * dense_mla_core (the drop-in) beyond 16384 keys against float64 closed form;
  * a dense-prefix stack (2 full + 4 DSA layers at 32K) and a DENSE cold
    start, eager and as a replayed graph: dense layers against the oracle,
    DSA layers bitwise against the standalone attention over the previous
    layer's selection, every selection bit-exact against the oracle top-k,
    and the layers that run an indexer exactly O.lagged_indexer_layers.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

from _cases import rel_err

pytestmark = pytest.mark.gpu


def _all_slots(pt_row: np.ndarray, n: int) -> np.ndarray:
    return O.slot_of(pt_row, np.arange(n)).astype(np.int64)


def _oracle_dense_row(L, b: int, n: int) -> np.ndarray:
    slots = torch.from_numpy(_all_slots(L.page_table[b].cpu().numpy(), n)).to(L.kv_pool.device)
    rows = L.kv_pool[slots].cpu().numpy()
    q = L.q_bf16[b:b + 1].float().cpu().numpy()
    return O.sparse_mla_decode(q, rows, np.arange(n, dtype=np.int32)[None, :], L.sm_scale)[0]


@pytest.mark.parametrize("lens,nsplit", [([32768, 5000, 70], 0), ([20000, 1, 0], 7), ([131072], 0)])
def test_dense_mla_decode_matches_oracle(dev, lens, nsplit):
    from lagged_indexer_dsa_amd import ops
    from lagged_indexer_dsa_amd import synthetic as S

    print(f"[dense] lens={lens} nsplit={nsplit}", flush=True)
    pt, num_pages = S.make_page_table([max(n, 1) for n in lens], seed=31, device=dev)
    L = S.make_decode_layer([max(n, 1) for n in lens], seed=32, device=dev, page_table=pt, num_pages=num_pages,
                            indexer=False)
    seq = torch.tensor(lens, dtype=torch.int32, device=dev)
    for rep in range(2):  # the workspace's barriers re-arm themselves
        out = ops.dense_mla_decode(L.q_bf16, L.kv_pool, pt, seq, nsplit=nsplit, workspace=L.workspace)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        for b, n in enumerate(lens):
            if n == 0:
                assert np.all(got[b] == 0), "an empty row gives 0"
                continue
            err = rel_err(got[b], _oracle_dense_row(L, b, n))
            assert err < 2e-2, f"rep {rep} row {b} (len {n}): rel err {err:.2e}"


def test_dense_mla_core_beyond_16k(dev):
    """The drop-in dense op on 40000 keys (two decode-position query rows)
    against the float64 closed form of the fp32 reference op."""
    from lagged_indexer_dsa_amd import attention_core as ac

    print("[dense] dense_mla_core 40000 keys", flush=True)
    g = torch.Generator().manual_seed(23)
    B, S, H, Skv = 1, 2, 16, 40000
    q = torch.randn(B, S, H, 576, generator=g)
    kv = torch.randn(B, Skv, 576, generator=g)
    got = ac.dense_mla_core(q.to(dev), kv.to(dev), 512).cpu().double().numpy()
    qd, kd = q.double().numpy(), kv.double().numpy()
    for s in range(S):
        n = Skv - S + s + 1
        sc = qd[0, s] @ kd[0, :n].T * 576 ** -0.5
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        ref = (p / p.sum(axis=1, keepdims=True)) @ kd[0, :n, :512]
        # e4m3 latent rows against the fp32 reference: the drop-in tolerance
        assert rel_err(got[0, s], ref) < 6e-2


@pytest.mark.parametrize("case", ["dense_prefix", "dense_cold_start", "eager_cold_start", "dense_prefix_b8"])
def test_mli_stack_with_dense_layers(dev, case):
    """The step built from a config by MLISchedule.for_config.
    dense_prefix_b8: 8 ragged rows, where each layer runs as three launches
    (scan, select, then the attention at its own split count), with a dense
    layer that produces a selection (layer 1) and one that does not (layer
    0).  eager_cold_start: layer 0 attends its own fresh selection."""
    from lagged_indexer_dsa_amd import _lib, ops
    from lagged_indexer_dsa_amd import synthetic as S
    from lagged_indexer_dsa_amd.config import AttentionType, ColdStartPolicy, dense_prefix_attention_types
    from lagged_indexer_dsa_amd.decode import MLISchedule, lagged_layer_plan

    lens = [9000, 3000, 12000, 500, 7000, 2048, 16000, 4097] if case == "dense_prefix_b8" else [32768]
    if case.startswith("dense_prefix"):
        types = dense_prefix_attention_types(6, 2)   # F F D D D D
    else:
        types = (AttentionType.DSA,) * 4
    cold = ColdStartPolicy.EAGER if case == "eager_cold_start" else ColdStartPolicy.DENSE
    plan = lagged_layer_plan(types, cold)
    produces = [p.indexer for p in plan]
    dense = [p.dense for p in plan]
    is_dsa = [t is AttentionType.DSA for t in types]
    assert produces[1:] == O.lagged_indexer_layers(is_dsa)[1:]
    print(f"[dense] MLI {case} produces={produces} dense={dense}", flush=True)
    _lib.sync_timeouts(reset=True)
    pt, num_pages = S.make_page_table(lens, seed=41, device=dev)
    nsplit = 0 if case == "dense_prefix_b8" else 16
    sched = MLISchedule.for_config(
        types, lambda i, idx: S.make_decode_layer(lens, seed=420 + i, device=dev, page_table=pt,
                                                  num_pages=num_pages, indexer=idx, nsplit=nsplit),
        cold_start=cold)
    layers = sched.layers
    # the set a sparse layer attends: the previous layer's fresh selection
    # (layer 0 under EAGER: its own)
    src = [None if dense[i] else (0 if plan[i].attends_own else i - 1) for i in range(len(types))]
    assert all(s is None or produces[s] for s in src), "every sparse layer's source runs an indexer"
    for mode in ("eager", "graph", "graph"):
        for L in layers:
            L.out.zero_(); L.next_idx.fill_(-7)
        torch.cuda.synchronize()
        sched.run_eager() if mode == "eager" else sched.replay()
        torch.cuda.synchronize()
        assert _lib.sync_timeouts() == 0
        sels = [L.next_idx.clone() for L in layers]
        for i, L in enumerate(layers):
            if produces[i]:
                ref_sel = O.topk_select(L.scores.cpu().numpy(), np.array(lens), L.topk,
                                        page_table=pt.cpu().numpy())
                assert np.array_equal(sels[i].cpu().numpy(), ref_sel), f"{mode} layer {i} selection"
            if dense[i]:
                got = L.out.float().cpu().numpy()
                for b, n in enumerate(lens):
                    err = rel_err(got[b], _oracle_dense_row(L, b, n))
                    assert err < 2e-2, f"{mode} dense layer {i} row {b}: rel err {err:.2e}"
            else:
                # the standalone attention over the set the schedule names,
                # bitwise, at the layer's split count or (from 8 rows, when
                # the attention rides in the scan launch) the launch's own
                # count of splits
                got = L.out.view(torch.int16)
                ok = False
                for ns in (L.nsplit, 1, 2, 4, 8):
                    ref = ops.sparse_mla_decode(L.q_bf16, L.kv_pool, sels[src[i]], nsplit=ns)
                    torch.cuda.synchronize()
                    if torch.equal(ref.view(torch.int16), got):
                        ok = True
                        break
                assert ok, f"{mode} layer {i}"
    sched.close()
