"""GPU: the drop-in core ops (lagged_indexer_dsa_amd.attention_core) against
the reference's semantics (src/lagged_indexer_dsa/attention_core.py:27-160)
restated in oracle/.

Tolerances: scores and attention outputs within
max-abs 2e-2 relative to the reference's scale; top-k bit-exact on the
same fp32 logits with the lower-index tie rule.  The indexer's 2e-2 gate is
against the reference's fp8 semantics (its GPU gate K:3105 compares with
ref_indexer_logits_fp8, K:2990-2992: the same e4m3 operands); against the
fp32 CPU op the e4m3 rounding of both q and k (3 mantissa bits) leaves
about 4% of max-abs, so that comparison uses K:3105's correlation gate
(1 - corr < 1e-3) and an fp8 bound of 6e-2.  Likewise attention: the 2e-2
gate is against the same fp8 latent rows (the reference's GPU gate K:3104
compares with ref_sparse_mla on the dequantised rows); against fp32 rows
the e4m3 values leave a few percent, bounded by 6e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2
FP8_VS_FP32 = 6e-2


def _ac():
    from lagged_indexer_dsa_amd import attention_core as ac
    return ac


def _rel(got: np.ndarray, ref: np.ndarray) -> float:
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def test_indexer_logits_matches_fp32_reference(dev):
    ac = _ac()
    print("[ac] indexer_logits", flush=True)
    g = torch.Generator().manual_seed(11)
    for (B, S, H, Skv) in [(2, 3, 64, 5000), (1, 1, 32, 130), (1, 2, 16, 64)]:
        q = torch.randn(B, S, H, 128, generator=g)
        k = torch.randn(B, Skv, 128, generator=g)
        w = torch.randn(B, S, H, generator=g) * H ** -0.5
        got = ac.indexer_logits(q.to(dev), k.to(dev), w.to(dev))
        assert got.shape == (B, S, Skv) and got.dtype == torch.float32
        ref = O.indexer_logits_fp32(q.double().numpy(), k.double().numpy(), w.double().numpy())
        g_ = got.cpu().double().numpy()
        assert _rel(g_, ref) < FP8_VS_FP32, (B, S, H, Skv)
        if Skv >= 1000:
            assert 1.0 - np.corrcoef(g_.ravel(), ref.ravel())[0, 1] < 1e-3, (B, S, H, Skv)


def test_indexer_logits_exact_on_quantised_operands(dev):
    """The fp8 path computes s_k * sum_h w' ReLU(q8.k8) exactly up to fp32
    accumulation (oracle indexer_scores on the same codes)."""
    from lagged_indexer_dsa_amd import formats as F

    ac = _ac()
    g = torch.Generator().manual_seed(12)
    B, S, H, Skv = 1, 2, 64, 3000
    q = torch.randn(B, S, H, 128, generator=g)
    k = torch.randn(B, Skv, 128, generator=g)
    w = torch.randn(B, S, H, generator=g) / 8
    got = ac.indexer_logits(q.to(dev), k.to(dev), w.to(dev)).cpu().numpy()
    kc, ks = F.quantize_rowwise(k[0].to(dev))          # the op's own (device) quantisation
    q8, wq = F.quantize_index_query(q[0].to(dev), w[0].to(dev))
    npg = (Skv + 63) // 64
    pages = O.pack_index_pages(kc.cpu().numpy(), ks.cpu().numpy(), np.arange(npg), npg)
    ref = O.indexer_scores(q8.cpu().numpy(), wq.cpu().numpy(), pages, np.tile(np.arange(npg), (S, 1)),
                           np.full(S, Skv), npg * 64)[:, :Skv]
    assert _rel(got[0], ref) < 1e-4   # fp32 accumulation vs float64


def test_apply_causal_mask_aligned_and_decode(dev):
    ac = _ac()
    x = torch.randn(2, 5, 5, device=dev)
    m = ac.apply_causal_mask(x).cpu()
    tri = torch.tril(torch.ones(5, 5, dtype=torch.bool))
    assert torch.equal(torch.isfinite(m[0]), tri)           # S == S_kv: reference rule
    d = ac.apply_causal_mask(torch.randn(1, 1, 9, device=dev)).cpu()
    assert torch.isfinite(d).all()                           # decode row: whole prefix


@pytest.mark.parametrize("B,S,Skv,topk", [(2, 2, 9000, 2048), (1, 1, 1500, 2048), (1, 3, 4096, 7)])
def test_select_topk_bit_exact(dev, B, S, Skv, topk):
    ac = _ac()
    print(f"[ac] select_topk {B}x{S}x{Skv} k={topk}", flush=True)
    g = torch.Generator().manual_seed(Skv)
    x = torch.randn(B, S, Skv, generator=g)
    x = torch.round(x * 8) / 8                               # many ties
    x[..., ::7] = float("-inf")
    x[0, 0, 3] = float("nan")
    x[..., 5] = -0.0
    got = ac.select_topk(x.to(dev), topk).cpu().numpy()
    ref = O.select_topk_reference(x.numpy(), topk)
    assert got.dtype == np.int64
    assert np.array_equal(got, ref)


def _mla_ref(q: np.ndarray, kv: np.ndarray, idx_sets, sm: float) -> np.ndarray:
    """Float64 closed form: softmax over each row's admissible key set."""
    B, S, H, _ = q.shape
    out = np.zeros((B, S, H, 512))
    for b in range(B):
        for s in range(S):
            keys = np.array(sorted(idx_sets[b][s]), dtype=np.int64)
            if keys.size == 0:
                continue
            k = kv[b, keys]
            sc = (q[b, s] @ k.T) * sm
            sc -= sc.max(axis=1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(axis=1, keepdims=True)
            out[b, s] = p @ k[:, :512]
    return out


def _mla_ref_quantised(ac, q, kv, idx_sets, sm: float, dev) -> np.ndarray:
    """Oracle sparse MLA over the op's own fp8 latent rows and bf16 q."""
    B, S, H, _ = q.shape
    Skv = kv.shape[1]
    rows = ac._pool_rows(kv.to(dev)).cpu().numpy()
    qb = q.to(torch.bfloat16).float().numpy()
    out = np.zeros((B, S, H, 512))
    for b in range(B):
        for s in range(S):
            slots = np.array([b * Skv + j for j in sorted(idx_sets[b][s])], dtype=np.int64)
            out[b, s] = O.sparse_mla_decode(qb[b, s][None], rows, slots[None], sm)[0]
    return out


def test_sparse_mla_core_matches_reference(dev):
    ac = _ac()
    print("[ac] sparse_mla_core", flush=True)
    g = torch.Generator().manual_seed(21)
    B, S, H, Skv, K = 2, 2, 16, 6000, 2048
    q = torch.randn(B, S, H, 576, generator=g)
    kv = torch.randn(B, Skv, 576, generator=g)
    idx = torch.stack([torch.stack([torch.randperm(Skv, generator=g)[:K] for _ in range(S)]) for _ in range(B)])
    idx[0, 0, :100] = Skv          # sentinel
    idx[1, 1, 10:20] = idx[1, 1, 0]  # duplicates count once
    idx[1, 0, 7] = Skv - 1         # after row 0's position (S_kv - 2): masked
    got = ac.sparse_mla_core(q.to(dev), kv.to(dev), idx.to(dev), 512).cpu().double().numpy()
    sets = [[{int(j) for j in idx[b, s] if 0 <= j <= Skv - S + s} for s in range(S)] for b in range(B)]
    ref8 = _mla_ref_quantised(ac, q, kv, sets, 576 ** -0.5, dev)
    assert _rel(got, ref8) < TOL
    ref = _mla_ref(q.double().numpy(), kv.double().numpy(), sets, 576 ** -0.5)
    assert _rel(got, ref) < FP8_VS_FP32


def test_dense_mla_core_aligned_prefill(dev):
    ac = _ac()
    g = torch.Generator().manual_seed(22)
    B, S, H, Skv = 1, 6, 16, 300
    q = torch.randn(B, S, H, 576, generator=g)
    kv = torch.randn(B, Skv, 576, generator=g)
    got = ac.dense_mla_core(q.to(dev), kv.to(dev), 512).cpu().double().numpy()
    sets = [[set(range(Skv - S + s + 1)) for s in range(S)]]
    ref8 = _mla_ref_quantised(ac, q, kv, sets, 576 ** -0.5, dev)
    assert _rel(got, ref8) < TOL
    ref = _mla_ref(q.double().numpy(), kv.double().numpy(), sets, 576 ** -0.5)
    assert _rel(got, ref) < FP8_VS_FP32


def test_select_then_attend_pipeline_decode_row(dev):
    """indexer_logits -> select_topk -> sparse_mla_core on one C1 decode row
    (oracle cpu_reference_path operands).  The fp8 scores pick almost the
    same top-2048 as the fp32 path; the output over the picked set matches
    the float64 closed form."""
    from oracle.cpu_reference_path import decode_layer_fp32, make_inputs

    ac = _ac()
    inp = make_inputs(8192, seed=0)
    ref_idx, _ = decode_layer_fp32(*inp, topk=2048)
    iq, ik, w, q, kv = inp[:5]
    logits = ac.indexer_logits(iq.to(dev), ik.to(dev), w.to(dev))
    idx = ac.select_topk(logits, 2048)
    got = ac.sparse_mla_core(q.to(dev), kv.to(dev), idx, 512).cpu().double().numpy()
    picked = set(idx[0, 0].cpu().tolist())
    overlap = len(picked & set(ref_idx[0, 0].tolist())) / 2048
    assert overlap > 0.9, overlap
    ref = _mla_ref(q.double().numpy(), kv.double().numpy(), [[picked]], 576 ** -0.5)
    assert _rel(got, ref) < FP8_VS_FP32


def test_cpu_tensors_rejected():
    ac = _ac()
    with pytest.raises(RuntimeError):
        ac.select_topk(torch.zeros(1, 1, 8), 4)
