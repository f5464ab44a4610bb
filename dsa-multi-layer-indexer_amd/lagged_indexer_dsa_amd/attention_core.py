"""Drop-in for the reference's core DSA ops on the MI355X path.

Same names, argument shapes, return shapes and argument errors (ValueError)
as the reference's plain-PyTorch ops (src/lagged_indexer_dsa/
attention_core.py:23-160), so ``DSALayer`` and ``DSAModel`` (dsa_layer.py,
model.py) can call them unchanged -- see :func:`install`.  Every op takes
GPU (HIP) tensors and runs the hand-written kernels of this package; there is
no CPU path (a CPU tensor raises).

Numerics are those of the reference's GPU decode path, which the HIP kernels
implement:

* :func:`indexer_logits` quantises the keys per token and the queries per
  head to OCP e4m3 (scale = amax / 448, the query scale folded into the head
  weight; K:2969-2974, K:2984-2985) and contracts them on fp8 MFMA:
  ``I[g] = s_k[g] * sum_h w'[h] * ReLU(q8[h] . k8[g])`` (K:2990-2992).
* :func:`select_topk` is exact on the fp32 logits it is given: rank by
  value (-0.0 == +0.0, NaN above +inf), ties to the LOWER index (the tie
  order torch.topk leaves open), non-finite selections and missing slots
  -> the sentinel ``S_kv`` (attention_core.py:66-91).
* :func:`sparse_mla_core` quantises the latent rows to the 656-byte fp8
  format (512 e4m3 + 4 fp32 per-128 scales + 64 bf16 rope; K:1181-1197)
  and the queries to bf16, and runs the split-K sparse MLA kernel.  A row
  with no admissible key returns 0 (the GPU kernels' rule, K:1038-1042;
  the dense CPU op would return NaN there).

Causality follows the GPU kernels' convention: query row s of S sits at
position ``S_kv - S + s`` (K:245).  For S == S_kv (aligned prefill) that is
the reference CPU ops' rule; for a decode row (S == 1) it admits the whole
prefix, which is what the reference's decode kernels do.
"""

from __future__ import annotations

import torch

from . import formats, ops
from ._lib import INDEX_DIM, LATENT_DIM, PAGE_TOKENS, QK_DIM, TOPK_MAX_CTX

def _gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("lagged_indexer_dsa_amd.attention_core runs on GPU (HIP) tensors only")


def pad_index(seq_len_kv: int) -> int:
    """The out-of-range index sentinel: ``S_kv`` (attention_core.py:21-23)."""
    return seq_len_kv


def _q_pos(S: int, Skv: int, device) -> torch.Tensor:
    return torch.arange(Skv - S, Skv, device=device)


def indexer_logits(index_q: torch.Tensor, index_k: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """Lightning-indexer scores ``[B, S, S_kv]`` (attention_core.py:27-49).

    index_q ``[B, S, H_idx, 128]``, index_k ``[B, S_kv, 128]``, weights
    ``[B, S, H_idx]``; H_idx one of 16, 32, 48, 64.  No causal masking
    (apply it with :func:`apply_causal_mask`, as the reference does).
    """
    if index_q.dim() != 4:
        raise ValueError(f"index_q must be [B,S,H,D], got {tuple(index_q.shape)}")
    if index_k.dim() != 3:
        raise ValueError(f"index_k must be [B,S_kv,D], got {tuple(index_k.shape)}")
    B, S, H, D = index_q.shape
    if index_k.shape[0] != B or index_k.shape[2] != D or tuple(weights.shape) != (B, S, H):
        raise ValueError("index_q, index_k and weights disagree in B, S, H or D")
    if D != INDEX_DIM:
        raise ValueError(f"the fp8 indexer contracts D = {INDEX_DIM}, got {D}")
    _gpu(index_q, index_k, weights)
    dev = index_q.device
    Skv = index_k.shape[1]
    npg = max(1, (Skv + PAGE_TOKENS - 1) // PAGE_TOKENS)
    # identity paging: batch b's page p is physical page b * npg + p; every
    # key of the batch quantized in one call and laid out page by page
    pt = (torch.arange(B, dtype=torch.int32, device=dev)[:, None] * npg
          + torch.arange(npg, dtype=torch.int32, device=dev)[None, :])
    codes, sc = formats.quantize_rowwise(index_k.reshape(B * Skv, D))
    kpad = torch.zeros(B, npg * PAGE_TOKENS, D, dtype=torch.uint8, device=dev)
    kpad[:, :Skv] = codes.reshape(B, Skv, D)
    spad = torch.zeros(B, npg * PAGE_TOKENS, dtype=torch.float32, device=dev)
    spad[:, :Skv] = sc.reshape(B, Skv)
    pages = torch.cat([kpad.reshape(B * npg, PAGE_TOKENS * D),
                       spad.reshape(B * npg, PAGE_TOKENS).view(torch.uint8)], dim=1).contiguous()
    q8, wq = formats.quantize_index_query(index_q.reshape(B * S, H, D), weights.reshape(B * S, H))
    rows_pt = pt.repeat_interleave(S, dim=0).contiguous()
    seq = torch.full((B * S,), Skv, dtype=torch.int32, device=dev)
    scores = ops.indexer_scan(q8, wq, pages, rows_pt, seq, npg * PAGE_TOKENS)
    return scores[:, :Skv].reshape(B, S, Skv)


def apply_causal_mask(logits: torch.Tensor) -> torch.Tensor:
    """Scores of keys after each query's position -> -inf
    (attention_core.py:52-63; query row s is at position S_kv - S + s)."""
    _gpu(logits)
    S, Skv = logits.shape[1], logits.shape[2]
    k_pos = torch.arange(Skv, device=logits.device)[None, :]
    causal = k_pos <= _q_pos(S, Skv, logits.device)[:, None]
    return logits.masked_fill(~causal.unsqueeze(0), float("-inf"))


def select_topk(logits: torch.Tensor, topk: int) -> torch.Tensor:
    """Top-``topk`` key indices per query, int64 ``[B, S, topk]``, ordered by
    score (attention_core.py:66-91); non-finite or missing -> ``S_kv``."""
    if logits.dim() != 3:
        raise ValueError(f"logits must be [B,S,S_kv], got {tuple(logits.shape)}")
    _gpu(logits)
    B, S, Skv = logits.shape
    if Skv > TOPK_MAX_CTX:
        raise ValueError(f"S_kv {Skv} above the select's limit {TOPK_MAX_CTX}")
    rows = logits.reshape(B * S, Skv).float().contiguous()
    seq = torch.full((B * S,), Skv, dtype=torch.int32, device=logits.device)
    idx = ops.topk(rows, seq, topk, sorted=True, pad_value=pad_index(Skv))
    return idx.to(torch.int64).reshape(B, S, topk)


def _pool_rows(kv: torch.Tensor) -> torch.Tensor:
    """[B, S_kv, 576] -> the 656-byte fp8 latent rows, batch-major slots."""
    B, Skv, _ = kv.shape
    flat = kv.reshape(B * Skv, QK_DIM)
    return formats.pack_latent_rows(flat[:, :LATENT_DIM], flat[:, LATENT_DIM:]).contiguous()


def _attend_rows(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, sm_scale: float) -> torch.Tensor:
    """q [B,S,H,576], kv [B,S_kv,576], idx [B,S,n] int64 (admissible key
    positions or -1) -> [B,S,H,512] in q's dtype."""
    B, S, H, _ = q.shape
    Skv = kv.shape[1]
    # a selection is a set: a repeated index counts once (the reference's
    # scatter mask, attention_core.py:94-103)
    srt, _ = torch.sort(idx, dim=-1)
    dup = torch.zeros_like(srt, dtype=torch.bool)
    dup[..., 1:] = (srt[..., 1:] == srt[..., :-1]) & (srt[..., 1:] >= 0)
    srt = srt.masked_fill(dup, -1)
    base = (torch.arange(B, device=q.device) * Skv)[:, None, None]
    slots = torch.where(srt >= 0, srt + base, torch.full_like(srt, -1))
    n = slots.shape[-1]
    qb = q.reshape(B * S, H, QK_DIM).to(torch.bfloat16).contiguous()
    out = ops.sparse_mla_decode(qb, _pool_rows(kv), slots.reshape(B * S, n).to(torch.int32).contiguous(),
                                sm_scale=sm_scale)
    return out.reshape(B, S, H, LATENT_DIM).to(q.dtype)


def _check_mla(q: torch.Tensor, kv: torch.Tensor, value_dim: int) -> None:
    if q.dim() != 4 or kv.dim() != 3:
        raise ValueError(f"q must be [B,S,H,D] and kv [B,S_kv,D], got {tuple(q.shape)}, {tuple(kv.shape)}")
    if q.shape[0] != kv.shape[0] or q.shape[3] != kv.shape[2]:
        raise ValueError("q and kv disagree in B or D")
    if q.shape[3] != QK_DIM or value_dim != LATENT_DIM:
        raise ValueError(f"the fp8 latent format is D_qk = {QK_DIM}, value_dim = {LATENT_DIM}")
    if q.shape[2] % 16:
        raise ValueError("the head count must be a multiple of 16")
    _gpu(q, kv)


def sparse_mla_core(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor, value_dim: int,
                    sm_scale: float | None = None) -> torch.Tensor:
    """Sparse MLA over the selected and causal keys, ``[B, S, H, value_dim]``
    (attention_core.py:121-139).  indices ``[B, S, topk]``; out-of-range
    entries (the sentinel ``S_kv``, negatives) and keys after the query's
    position are not attended."""
    _check_mla(q, kv, value_dim)
    if indices.dim() != 3 or indices.shape[:2] != q.shape[:2]:
        raise ValueError(f"indices must be [B,S,topk], got {tuple(indices.shape)}")
    _gpu(indices)
    S, Skv = q.shape[1], kv.shape[1]
    if sm_scale is None:
        sm_scale = q.shape[-1] ** -0.5
    idx = indices.long()
    q_pos = _q_pos(S, Skv, q.device)[None, :, None]
    ok = (idx >= 0) & (idx < Skv) & (idx <= q_pos)
    return _attend_rows(q, kv, torch.where(ok, idx, torch.full_like(idx, -1)), float(sm_scale))


def dense_mla_core(q: torch.Tensor, kv: torch.Tensor, value_dim: int,
                   sm_scale: float | None = None) -> torch.Tensor:
    """Dense causal MLA (full-attention layers and the DENSE cold start,
    attention_core.py:142-160): query row s attends keys 0 .. S_kv - S + s,
    on the dense MLA kernel (no limit on S_kv).  The latent rows are packed
    to the fp8 format once, batch b's into pages of its own; every query row
    is a decode row over its causal prefix of those pages."""
    _check_mla(q, kv, value_dim)
    B, S, H, _ = q.shape
    Skv = kv.shape[1]
    if sm_scale is None:
        sm_scale = q.shape[-1] ** -0.5
    dev = q.device
    npg = max(1, (Skv + PAGE_TOKENS - 1) // PAGE_TOKENS)
    rows = torch.zeros(B, npg * PAGE_TOKENS, QK_DIM, dtype=kv.dtype, device=dev)
    rows[:, :Skv] = kv
    pool = _pool_rows(rows)  # slot of (b, j) = b * npg * 64 + j
    pt = (torch.arange(B, dtype=torch.int32, device=dev)[:, None] * npg
          + torch.arange(npg, dtype=torch.int32, device=dev)[None, :])
    pt_rows = pt.repeat_interleave(S, dim=0).contiguous()
    lens = (_q_pos(S, Skv, dev) + 1).clamp(min=0).to(torch.int32).repeat(B).contiguous()
    qb = q.reshape(B * S, H, QK_DIM).to(torch.bfloat16).contiguous()
    out = ops.dense_mla_decode(qb, pool, pt_rows, lens, sm_scale=float(sm_scale))
    return out.reshape(B, S, H, LATENT_DIM).to(q.dtype)


_NAMES = ("pad_index", "indexer_logits", "apply_causal_mask", "select_topk", "sparse_mla_core",
          "dense_mla_core")


def install(module) -> None:
    """Rebind the core-op names a reference module imported (for instance
    ``lagged_indexer_dsa.dsa_layer``, which binds them at import time,
    dsa_layer.py:21-27) to these GPU ops."""
    for name in _NAMES:
        if hasattr(module, name):
            setattr(module, name, globals()[name])
