"""CPU restatement of the reference's fp32 decode-row path -- TEST / BASELINE
INFRASTRUCTURE ONLY (imported by tests and by bench.py's cpu_baseline leg).

One DSA decode layer exactly as ``dsa_layer.py`` computes it for the last
query row, in torch fp32 on the host:
  indexer_logits   attention_core.py:27-49   einsum + ReLU + weighted head sum
  select_topk      attention_core.py:66-91   torch.topk, non-finite -> sentinel
  _selection_mask  attention_core.py:94-103  scatter into S_kv+1 columns
  _attend          attention_core.py:112-118 dense masked softmax over S_kv
At decode the query sits at position S_kv-1, so every key is causal and
no causal mask is applied (the GPU kernels' q_pos = seq_len-1, K:245).
"""

from __future__ import annotations

import torch


def decode_layer_fp32(index_q: torch.Tensor, index_k: torch.Tensor, weights: torch.Tensor,
                      q: torch.Tensor, kv: torch.Tensor, topk: int, value_dim: int = 512,
                      sm_scale: float | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """index_q [B,1,Hi,Di], index_k [B,Skv,Di], weights [B,1,Hi], q [B,1,H,Dqk],
    kv [B,Skv,Dqk] -> (indices [B,1,topk] int64, out [B,1,H,value_dim])."""
    skv = kv.shape[1]
    score = torch.einsum("bshd,bnd->bshn", index_q, index_k)
    logits = (torch.relu(score) * weights.unsqueeze(-1)).sum(dim=2)            # [B,1,Skv]
    k_eff = min(topk, skv)
    values, indices = torch.topk(logits, k_eff, dim=-1)
    indices = indices.masked_fill(~torch.isfinite(values), skv)
    if k_eff < topk:
        pad = torch.full((*indices.shape[:2], topk - k_eff), skv, dtype=indices.dtype)
        indices = torch.cat([indices, pad], dim=-1)
    mask = torch.zeros(*indices.shape[:2], skv + 1, dtype=torch.bool)
    mask.scatter_(2, indices.clamp(max=skv), True)
    mask = mask[..., :skv]
    if sm_scale is None:
        sm_scale = q.shape[-1] ** -0.5
    s = torch.einsum("bshd,bnd->bshn", q, kv)
    s = s.masked_fill(~mask.unsqueeze(2), float("-inf")) * sm_scale
    p = torch.softmax(s, dim=-1)
    out = torch.einsum("bshn,bnd->bshd", p, kv[..., :value_dim])
    return indices, out


def make_inputs(ctx: int, seed: int = 0, hidx: int = 64, didx: int = 128, heads: int = 16,
                dqk: int = 576):
    """C1 operands: N(0,1) everywhere, head weights x 1/sqrt(hidx), seed 0."""
    g = torch.Generator().manual_seed(seed)
    iq = torch.randn(1, 1, hidx, didx, generator=g)
    ik = torch.randn(1, ctx, didx, generator=g)
    w = torch.randn(1, 1, hidx, generator=g) * hidx ** -0.5
    q = torch.randn(1, 1, heads, dqk, generator=g)
    kv = torch.randn(1, ctx, dqk, generator=g)
    return iq, ik, w, q, kv
