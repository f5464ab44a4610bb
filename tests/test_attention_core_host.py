"""CPU: the drop-in core ops' argument contract (same ValueErrors as the
reference's attention_core.py:27-160) and their installation into a module
that imported the reference names (dsa_layer.py:21-27).  No kernel runs."""

from __future__ import annotations

import types

import pytest
import torch


def _ac():
    from lagged_indexer_dsa_amd import attention_core as ac
    return ac


def test_shape_errors_match_reference():
    ac = _ac()
    with pytest.raises(ValueError):
        ac.indexer_logits(torch.zeros(1, 2, 3), torch.zeros(1, 4, 128), torch.zeros(1, 2, 3))
    with pytest.raises(ValueError):
        ac.indexer_logits(torch.zeros(1, 1, 4, 128), torch.zeros(4, 128), torch.zeros(1, 1, 4))
    with pytest.raises(ValueError):
        ac.indexer_logits(torch.zeros(1, 1, 16, 64), torch.zeros(1, 4, 64), torch.zeros(1, 1, 16))
    with pytest.raises(ValueError):
        ac.select_topk(torch.zeros(4, 8), 2)
    with pytest.raises(ValueError):
        ac.sparse_mla_core(torch.zeros(1, 1, 16, 576), torch.zeros(1, 8, 576), torch.zeros(1, 1, 4), 256)
    with pytest.raises(ValueError):
        ac.sparse_mla_core(torch.zeros(1, 1, 8, 576), torch.zeros(1, 8, 576), torch.zeros(1, 1, 4), 512)


def test_pad_index_is_skv():
    assert _ac().pad_index(8192) == 8192


def test_install_rebinds_reference_names():
    ac = _ac()
    mod = types.SimpleNamespace(indexer_logits=None, select_topk=None, sparse_mla_core=None,
                                dense_mla_core=None, apply_causal_mask=None, unrelated=1)
    ac.install(mod)
    assert mod.indexer_logits is ac.indexer_logits
    assert mod.select_topk is ac.select_topk
    assert mod.sparse_mla_core is ac.sparse_mla_core
    assert mod.dense_mla_core is ac.dense_mla_core
    assert mod.apply_causal_mask is ac.apply_causal_mask
    assert mod.unrelated == 1
    assert not hasattr(mod, "pad_index")


def test_indexcache_pattern_equals_oracle():
    import json
    import pathlib

    from lagged_indexer_dsa_amd.decode import indexcache_pattern
    from oracle import dsa_oracle as O

    g = json.loads((pathlib.Path(__file__).parent / "golden" / "indexcache_patterns.json").read_text())
    cases = [dict(freq=f) for f in (None, 1, 2, 3, 4, 7)]
    cases += [dict(refresh_layers=r) for r in ([], [3, 9], "2,4, 60", [0])]
    cases += [dict(pattern=v["pattern"]) for v in g["patterns"].values()]
    cases += [dict(pattern="FS", freq=3), dict(pattern="", refresh_layers=[4])]
    for c in cases:
        for n in (0, 1, 13, 78):
            want = "".join("F" if p else "S" for p in O.indexcache_produces(n, **c))
            assert indexcache_pattern(n, **c) == want, (c, n)
    with pytest.raises(ValueError):
        indexcache_pattern(4, pattern="FX")
    with pytest.raises(ValueError):
        indexcache_pattern(4, freq=0)


def test_lagged_layer_plan_follows_the_reference_schedule():
    """lagged_layer_plan restates DSAModel.forward LAGGED_FUSED (model.py:
    61-71, 104-136): a layer produces iff the next layer is DSA; FULL layers
    and a DSA layer 0 under the DENSE cold start attend densely; under EAGER
    layer 0 runs its own indexer for its own attention."""
    from lagged_indexer_dsa_amd.config import (AttentionType, ColdStartPolicy, DSAConfig,
                                               dense_prefix_attention_types)
    from lagged_indexer_dsa_amd.decode import LayerPlan, lagged_layer_plan
    from oracle import dsa_oracle as O

    F, D = AttentionType.FULL, AttentionType.DSA
    for types in ([F, F, D, D, D, D], [D, D, D], [D, F, D, F], [F, F], [D], [D, F, F, D]):
        for cold in ColdStartPolicy:
            plan = lagged_layer_plan(tuple(types), cold)
            prod = O.lagged_indexer_layers([t is D for t in types])
            for i, (p, t) in enumerate(zip(plan, types)):
                eager0 = i == 0 and t is D and cold is ColdStartPolicy.EAGER
                assert p.indexer == (prod[i] or eager0)
                assert p.dense == (t is F or (i == 0 and t is D and cold is ColdStartPolicy.DENSE))
                assert p.attends_own == eager0
    cfg = DSAConfig(num_hidden_layers=6, attention_layer_types=dense_prefix_attention_types(6, 2))
    assert lagged_layer_plan(cfg) == [LayerPlan(True, False), LayerPlan(True, True)] + \
        [LayerPlan(False, True)] * 3 + [LayerPlan(False, False)]
    assert lagged_layer_plan(DSAConfig(num_hidden_layers=3), "eager") == \
        [LayerPlan(False, True, True), LayerPlan(False, True), LayerPlan(False, False)]
