"""Pin the CPU oracle (oracle/dsa_oracle.py) before trusting it.

Every check here is independent of the oracle's own formula: library
routines (torch's float8_e4m3fn / bfloat16 casts, torch.topk), brute-force
Python loops, closed forms and invariants chosen so that a dropped term, a
wrong index or a transposed operand fails.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O


# ---------------------------------------------------------------- fp8 / bf16

def test_e4m3_decode_all_codes_match_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_decode(codes.numpy())
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    m = ~np.isnan(ref)
    assert np.array_equal(ref[m], got[m])


def test_e4m3_encode_matches_torch_on_random_and_ties():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000) * 40,
        rng.uniform(-448, 448, 50000),
        rng.standard_normal(50000) * 2.0 ** -8,        # subnormal range
    ]).astype(np.float32)
    # exact midpoints between neighbouring codes (round-half-even cases)
    vals = O.E4M3_TABLE[:0x7F]
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    x = np.clip(np.concatenate([x, mids, -mids, [0.0, -0.0, 448.0, -448.0]]), -448, 448).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.e4m3_encode(x)
    assert np.array_equal(ref, got)


def test_bf16_rn_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-20, 20, 200000))).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.bf16_rn(x), ref)


def test_latent_dequant_rule_all_codes_sample_scales():
    # bf16_rn(f32(e4m3) * scale) for every code and a spread of scales, vs torch
    codes = np.arange(256, dtype=np.uint8)
    codes = codes[~np.isnan(O.E4M3_TABLE)]
    for scale in [1.0, 0.0123, 3.7e-3, 1 / 448.0, 2.5, 1e-5]:
        s = np.float32(scale)
        ref = (torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float() * float(s)).to(torch.bfloat16).float().numpy()
        got = O.bf16_rn((O.e4m3_decode(codes) * s).astype(np.float32))
        assert np.array_equal(ref, got), scale


def test_quantize_rowwise_round_trip_bound_and_exactness():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    codes, scale = O.quantize_rowwise(x)
    deq = O.e4m3_decode(codes) * scale[:, None]
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 for normals, plus
    # the subnormal absolute step 2^-10 * scale
    err = np.abs(deq - x)
    assert np.all(err <= np.abs(x) / 16 + scale[:, None] * 2.0 ** -10 + 1e-7)
    # the row maximum maps to +-448 exactly
    assert np.all(np.abs(O.e4m3_decode(codes)).max(axis=1) == 448.0)
    # values that are exactly e4m3 * 2^k with amax 448 round-trip exactly
    exact = O.E4M3_TABLE[rng.integers(0, 0x7E, (8, 128))].astype(np.float32)
    exact[:, 0] = 448.0
    c2, s2 = O.quantize_rowwise(exact)
    assert np.all(s2 == np.float32(1.0))
    assert np.array_equal(O.e4m3_decode(c2), exact)


# ---------------------------------------------------------------- indexer

def _rand_index_case(rng, B, H, lens, num_pages_extra=3):
    n_pages = [(n + 63) // 64 for n in lens]
    num_pages = sum(n_pages) + num_pages_extra
    perm = rng.permutation(num_pages)
    pt = np.full((B, max(n_pages)), -1, dtype=np.int32)
    o = 0
    for b, npg in enumerate(n_pages):
        pt[b, :npg] = perm[o:o + npg]
        o += npg
    pages = np.zeros((num_pages, O.INDEX_PAGE_BYTES), dtype=np.uint8)
    keys = []
    for b, n in enumerate(lens):
        k = rng.standard_normal((n, 128)).astype(np.float32)
        c, s = O.quantize_rowwise(k)
        keys.append((c, s))
        p = O.pack_index_pages(c, s, pt[b], num_pages)
        for lp in range(n_pages[b]):
            pages[pt[b, lp]] = p[pt[b, lp]]
    qc, sq = O.quantize_rowwise(rng.standard_normal((B, H, 128)).astype(np.float32))
    w = (rng.standard_normal((B, H)) / 8).astype(np.float32) * sq
    return qc, w.astype(np.float32), pages, pt, keys


def test_indexer_scores_brute_force():
    rng = np.random.default_rng(3)
    lens = [70, 5, 64]
    qc, w, pages, pt, keys = _rand_index_case(rng, 3, 4, lens)
    slab = 200
    got = O.indexer_scores(qc, w, pages, pt, np.array(lens), slab)
    for b, n in enumerate(lens):
        kc, ks = keys[b]
        for g in range(n):
            acc = 0.0
            for h in range(4):
                dot = 0.0
                for d in range(128):
                    dot += float(O.E4M3_TABLE[qc[b, h, d]]) * float(O.E4M3_TABLE[kc[g, d]])
                acc += float(w[b, h]) * max(dot, 0.0)
            assert math.isclose(got[b, g], acc * float(ks[g]), rel_tol=1e-12, abs_tol=1e-12)
        assert np.all(np.isneginf(got[b, n:]))


def test_indexer_scores_closed_forms_and_invariants():
    rng = np.random.default_rng(4)
    lens = [300, 129]
    qc, w, pages, pt, keys = _rand_index_case(rng, 2, 8, lens)
    seq = np.array(lens)
    base = O.indexer_scores(qc, w, pages, pt, seq, 320)
    # w = 0 -> 0 on the prefix
    z = O.indexer_scores(qc, np.zeros_like(w), pages, pt, seq, 320)
    assert np.all(z[0, :300] == 0) and np.all(z[1, :129] == 0)
    # linear in w
    w2 = (rng.standard_normal(w.shape)).astype(np.float32)
    s2 = O.indexer_scores(qc, w2, pages, pt, seq, 320)
    s12 = O.indexer_scores(qc, w.astype(np.float64) + w2.astype(np.float64), pages, pt, seq, 320)
    m = np.isfinite(base)
    assert np.allclose(s12[m], base[m] + s2[m], rtol=1e-9, atol=1e-9)
    # one head: w * relu(q.k) * s
    one = O.indexer_scores(qc[:, :1], w[:, :1], pages, pt, seq, 320)
    kc, ks = keys[0]
    dot = O.e4m3_decode(kc).astype(np.float64) @ O.e4m3_decode(qc[0, 0]).astype(np.float64)
    assert np.allclose(one[0, :300], w[0, 0] * np.maximum(dot, 0) * ks, rtol=1e-12)
    # physical page placement is invisible: move every page elsewhere
    perm = rng.permutation(pages.shape[0])
    pages2 = np.empty_like(pages)
    pages2[perm] = pages
    pt2 = np.where(pt >= 0, perm[np.maximum(pt, 0)], -1).astype(np.int32)
    assert np.array_equal(O.indexer_scores(qc, w, pages2, pt2, seq, 320), base)


def test_fp8_scores_equal_fp32_indexer_on_decoded_values():
    # the fp8 score is the reference fp32 indexer_logits (AC:27-49) applied
    # to the decoded fp8 values, times the per-key scale
    rng = np.random.default_rng(5)
    lens = [150]
    qc, w, pages, pt, keys = _rand_index_case(rng, 1, 16, lens)
    got = O.indexer_scores(qc, w, pages, pt, np.array(lens), 150)[0]
    kc, ks = keys[0]
    q = O.e4m3_decode(qc).astype(np.float64)[:, None]           # [B=1, S=1, H, D]
    k = O.e4m3_decode(kc).astype(np.float64)[None]               # [1, n, D]
    ref = O.indexer_logits_fp32(q, k, w.astype(np.float64)[:, None])[0, 0] * ks
    assert np.allclose(got, ref, rtol=1e-12, atol=0)


def test_indexer_logits_fp32_matches_reference_test_port():
    # the reference's own check (tests/test_attention_core.py:20-29, 67-76)
    torch.manual_seed(0)
    b, s, h, d, skv = 2, 12, 8, 16, 12
    q = torch.randn(b, s, h, d)
    k = torch.randn(b, skv, d)
    wt = torch.randn(b, s, h)
    score = torch.einsum("bmhd,bnd->bhmn", q, k)
    expected = (score.relu() * wt.unsqueeze(-1).transpose(1, 2)).sum(dim=1)
    got = O.indexer_logits_fp32(q.numpy(), k.numpy(), wt.numpy())
    assert np.allclose(got, expected.numpy(), atol=1e-5, rtol=1e-4)


# ---------------------------------------------------------------- top-k

def _brute_topk(row, n, k, sorted_, pad):
    vals = [(row[i], i) for i in range(n)]

    def rank(v):
        if math.isnan(v):
            return (3, 0.0)
        if math.isinf(v):
            return (2, 0.0) if v > 0 else (0, 0.0)
        return (1, float(v))
    vals.sort(key=lambda t: (tuple(-x for x in rank(t[0])), t[1]))
    pick = vals[:k]
    fin = [(v, i) for v, i in pick if math.isfinite(v)]
    if sorted_:
        res = [i if math.isfinite(v) else pad for v, i in pick]
    else:
        res = sorted(i for _, i in fin)
    return res + [pad] * (k - len(res))


@pytest.mark.parametrize("sorted_", [False, True])
def test_topk_brute_force_with_ties_and_specials(sorted_):
    rng = np.random.default_rng(6)
    for trial in range(60):
        n = int(rng.integers(0, 80))
        k = int(rng.integers(1, 40))
        row = rng.integers(-4, 5, 90).astype(np.float32)          # heavy ties
        if trial % 3 == 0:
            row = rng.standard_normal(90).astype(np.float32)
        if trial % 5 == 0 and n > 3:
            row[rng.integers(0, n, 3)] = [np.inf, -np.inf, np.nan]
        if trial % 7 == 0:
            row[rng.integers(0, 90, 10)] = -0.0
        got = O.topk_select(row[None], np.array([n]), k, sorted_=sorted_, pad=-7)[0]
        assert list(got) == _brute_topk(list(row), n, k, sorted_, -7), trial


def test_topk_sorted_values_equal_torch_topk():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4, 5000)).astype(np.float32)
    got = O.topk_select(x, np.full(4, 5000), 2048, sorted_=True)
    ref_vals, _ = torch.topk(torch.from_numpy(x), 2048, dim=-1)
    assert np.array_equal(np.take_along_axis(x, got.astype(np.int64), 1), ref_vals.numpy())


def test_topk_zero_signs_tie_and_lower_index_wins():
    row = np.array([1.0, -0.0, 0.0, -1.0, 0.0], dtype=np.float32)
    # -0.0 == +0.0: among the three zeros the two lowest indices win
    assert list(O.topk_select(row[None], np.array([5]), 3, sorted_=True)[0]) == [0, 1, 2]
    assert list(O.topk_select(row[None], np.array([5]), 3)[0]) == [0, 1, 2]


def test_select_topk_reference_semantics_sentinel():
    # AC:66-91: slots without a finite score carry the sentinel S_kv
    logits = np.array([[[3.0, -np.inf, 1.0, -np.inf]]], dtype=np.float32)
    got = O.select_topk_reference(logits, 3)
    assert got.tolist() == [[[0, 2, 4]]]
    got = O.select_topk_reference(logits, 6)
    assert got.tolist() == [[[0, 2, 4, 4, 4, 4]]]


def test_topk_page_slot_mapping():
    pt = np.array([[5, 2]], dtype=np.int32)
    row = np.zeros(128, dtype=np.float32)
    row[[3, 70, 64]] = [3.0, 2.0, 1.0]
    got = O.topk_select(row[None], np.array([128]), 3, page_table=pt)[0]
    assert list(got) == [5 * 64 + 3, 2 * 64 + 0, 2 * 64 + 6]


# ---------------------------------------------------------------- sparse MLA

def _mla_case(rng, n_rows=300, B=2, H=3):
    lat = rng.standard_normal((n_rows, 576)).astype(np.float32)
    rows = O.pack_latent_rows(lat[:, :512], lat[:, 512:])
    q = O.bf16_rn(rng.standard_normal((B, H, 576)).astype(np.float32))
    return rows, q


def test_pack_latent_rows_layout():
    rng = np.random.default_rng(8)
    lat = rng.standard_normal((3, 576)).astype(np.float32)
    rows = O.pack_latent_rows(lat[:, :512], lat[:, 512:])
    assert rows.shape == (3, 656)
    deq = O.dequant_latent_rows(rows)
    # rope is the bf16 of the input, stored at bytes 528..656
    assert np.array_equal(deq[:, 512:], O.bf16_rn(lat[:, 512:]))
    # group scale g covers dims 128g..128g+127 and lives at byte 512 + 4g
    sc = rows[:, 512:528].copy().view(np.float32)
    for g in range(4):
        amax = np.abs(lat[:, 128 * g:128 * (g + 1)]).max(axis=1)
        assert np.allclose(sc[:, g], amax / 448, rtol=1e-6)
    assert np.allclose(deq[:, :512], lat[:, :512], rtol=0.07, atol=0.02)


def test_sparse_mla_brute_force():
    rng = np.random.default_rng(9)
    rows, q = _mla_case(rng, n_rows=40, B=1, H=2)
    idx = np.array([[3, 17, -1, 39, 40, 5]])
    got = O.sparse_mla_decode(q, rows, idx, 0.05)
    kv = O.dequant_latent_rows(rows).astype(np.float64)
    valid = [3, 17, 39, 5]
    for h in range(2):
        sc = [0.05 * sum(float(q[0, h, d]) * kv[j, d] for d in range(576)) for j in valid]
        mx = max(sc)
        e = [math.exp(s - mx) for s in sc]
        tot = sum(e)
        ref = sum(e[i] / tot * kv[j, :512] for i, j in enumerate(valid))
        assert np.allclose(got[0, h], ref, rtol=1e-10, atol=1e-12)


def test_sparse_mla_invariants():
    rng = np.random.default_rng(10)
    rows, q = _mla_case(rng)
    idx = rng.permutation(300)[:64][None].repeat(2, 0)
    base = O.sparse_mla_decode(q, rows, idx, 576 ** -0.5)
    perm = O.sparse_mla_decode(q, rows, idx[:, ::-1].copy(), 576 ** -0.5)
    assert np.allclose(base, perm, rtol=1e-12, atol=1e-12)
    # one key: output is that row's value
    one = O.sparse_mla_decode(q, rows, np.array([[7], [7]]), 576 ** -0.5)
    assert np.allclose(one[0, 0], O.dequant_latent_rows(rows[7:8])[0, :512])
    # nothing valid -> 0
    none = O.sparse_mla_decode(q, rows, np.array([[-1, 300], [-5, 999]]), 576 ** -0.5)
    assert np.all(none == 0)


def test_split_lse_merge_equals_one_pass():
    rng = np.random.default_rng(11)
    rows, q = _mla_case(rng)
    kv = O.dequant_latent_rows(rows[:200]).astype(np.float64)
    qh = q[0].astype(np.float64)
    ref = O.sparse_mla_decode(q[:1], rows, np.arange(200)[None], 0.1)[0]
    for nsplit in [1, 3, 16, 64, 300]:
        merged = O.lse_merge(O.split_partials(qh, kv, 0.1, nsplit))
        assert np.allclose(merged, ref, rtol=1e-10, atol=1e-12), nsplit


def test_sparse_mla_equals_reference_masked_dense_form():
    # AC:94-118: scatter a membership mask over all S_kv keys, then a dense
    # masked softmax -- a different computation of the same quantity
    rng = np.random.default_rng(12)
    rows, q = _mla_case(rng, n_rows=120, B=1, H=4)
    sel = rng.permutation(120)[:30]
    kv = O.dequant_latent_rows(rows).astype(np.float64)
    mask = np.zeros(121, dtype=bool)
    mask[np.minimum(sel, 120)] = True
    score = q[0].astype(np.float64) @ kv.T
    score = np.where(mask[None, :120], score, -np.inf) * 576 ** -0.5
    p = np.exp(score - score.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ref = p @ kv[:, :512]
    got = O.sparse_mla_decode(q, rows, sel[None], 576 ** -0.5)[0]
    assert np.allclose(got, ref, rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------- schedule

def test_lagged_indexer_layers_reference_cases():
    # model.py:61-71: layer i emits iff layer i+1 is DSA
    assert O.lagged_indexer_layers([True] * 5) == [True, True, True, True, False]
    assert O.lagged_indexer_layers([False, False, True, True]) == [False, True, True, False]
    assert O.lagged_indexer_layers([True, False, True]) == [False, True, False]
    assert O.mli_attend_sources([True, True, False]) == [-1, 0, 1]
    assert O.mli_attend_sources([True, False, False, False, True, False]) == [-1, 0, 0, 0, 0, 4]


def test_lag_depth_matches_overlay_invariants():
    """P:3020-3060: with the cold start (R_0 attends its own fresh set),
    refresh layer R_n attends the set produced k refresh layers back from
    R_k on, and R_1..R_{k-1} attend the incoming carry (R_0's set)."""
    for k in range(1, 6):
        src = O.mli_attend_sources([True] * 12, first_attend=0, depth=k)
        assert src[0] == 0
        for n in range(1, 12):
            assert src[n] == (n - k if n >= k else 0), (k, n)
    # depth 1 is the certified one-layer lag, whatever the pattern
    rng = np.random.default_rng(3)
    for _ in range(50):
        prod = list(rng.random(15) < 0.4)
        assert O.mli_attend_sources(prod, depth=1) == O.mli_attend_sources(prod)
    with pytest.raises(ValueError):
        O.mli_attend_sources([True], depth=0)


def test_lag_depth_with_indexcache_reuse():
    """Reuse layers copy: the FRESH set of the producer before them at depth
    1 (P:3050-3052), the producer's ATTENDED set at depth >= 2 (P:3040-3046)."""
    prod = [True, False, True, False, True, False, True, False]
    assert O.mli_attend_sources(prod, -1, 1) == [-1, 0, 0, 2, 2, 4, 4, 6]
    assert O.mli_attend_sources(prod, -1, 2) == [-1, -1, -1, -1, 0, 0, 2, 2]
    assert O.mli_attend_sources(prod, 0, 2) == [0, 0, 0, 0, 0, 0, 2, 2]
    # brute force over producers: at depth k every layer attends the fresh
    # set of the producer k producers before the latest producer at or
    # before it, clamped to the cold start
    for k in (2, 3, 4):
        rng = np.random.default_rng(k)
        for _ in range(40):
            prod = [True] + list(rng.random(20) < 0.5)
            src = O.mli_attend_sources(prod, 0, k)
            R = [i for i, p in enumerate(prod) if p]
            for i in range(len(prod)):
                n = max(j for j, r in enumerate(R) if r <= i)
                assert src[i] == (R[n - k] if n >= k else 0), (k, i)


def test_indexcache_published_patterns_and_precedence():
    import json
    import pathlib

    g = json.loads((pathlib.Path(__file__).parent / "golden" / "indexcache_patterns.json").read_text())
    for v in g["patterns"].values():
        prod = O.indexcache_produces(g["num_layers"], freq=4, pattern=v["pattern"], refresh_layers=[5])
        assert sum(prod) == v["full_layers"]          # pattern wins over freq and refresh_layers
        assert prod[0] and prod[1]
    assert O.indexcache_produces(5, pattern="FS") == [True, False, True, True, True]
    assert O.indexcache_produces(6, freq=2, refresh_layers="3, 5") == [True, False, False, True, False, True]
    assert O.indexcache_produces(6, refresh_layers=[]) == [True] + [False] * 5
    assert O.indexcache_produces(9, freq=4) == [True, False, False, False, True, False, False, False, True]
    assert O.indexcache_produces(3, freq=None) == [True] * 3
