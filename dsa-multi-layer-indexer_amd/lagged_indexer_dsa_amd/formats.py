"""HBM data formats of the decode path and torch builders for them.

* index-K page (8448 B): [64 keys x 128 e4m3][64 x f32 per-key scale]
  (reference K:540-546, K:630, K:2428; serving index-K buffer P:339-342).
* latent KV row (656 B): [512 e4m3][4 x f32 scale, one per 128 dims]
  [64 x bf16 rope] (K:1114, K:1355-1395; SGLang fp8 KV layout P:800-803).
* page table: int32 [B, pt_stride]; token g of row b is in physical page
  page_table[b, g // 64], slot g % 64; its latent row is KV slot
  page_table[b, g // 64] * 64 + g % 64 (hp_page_to_slot, K:1142-1144).

The quantisers follow the reference harness (K:2969-2974): per row,
scale = max(amax, 1e-6) / 448, code = e4m3(clamp(x / scale, +-448)).
They are torch ops that run on whatever device the input lives on: they
build caches, they are not part of the per-step hot path.
"""

from __future__ import annotations

import torch

from ._lib import INDEX_DIM, INDEX_PAGE_BYTES, LATENT_DIM, LATENT_ROW_BYTES, PAGE_TOKENS, ROPE_DIM

E4M3_MAX = 448.0


def quantize_rowwise(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row (last dim) e4m3 quantisation -> (uint8 codes, float32 scale).

    The two fp32 divisions are IEEE-rounded on every device: they are done in
    float64 and rounded once to float32 (exact for a quotient of two fp32
    values), since a GPU's fp32 division in torch need not be correctly
    rounded."""
    x = x.float()
    amax = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-6)
    scale = (amax.double() / E4M3_MAX).float()
    q = (x.double() / scale.double()).float().clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), scale.squeeze(-1)


def quantize_index_query(q: torch.Tensor, w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Indexer query [B,H,128] -> e4m3 codes with the per-head scale folded
    into the head weight: wp = w * q_scale (K:2984-2985; transformer.py:1143-1144)."""
    codes, sq = quantize_rowwise(q)
    return codes.contiguous(), (w.float() * sq).contiguous()


def random_page_table(seq_lens: list[int], pt_stride: int, num_pages: int,
                      generator: torch.Generator | None = None) -> torch.Tensor:
    """Distinct physical pages for every row's logical pages, drawn as one
    seeded permutation of the pool (CPU int32 [B, pt_stride], unused = -1)."""
    need = [(n + PAGE_TOKENS - 1) // PAGE_TOKENS for n in seq_lens]
    if sum(need) > num_pages:
        raise ValueError(f"pool of {num_pages} pages cannot hold {sum(need)}")
    if max(need, default=0) > pt_stride:
        raise ValueError("pt_stride too small for the longest row")
    perm = torch.randperm(num_pages, generator=generator).to(torch.int32)
    pt = torch.full((len(seq_lens), pt_stride), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(need):
        pt[b, :n] = perm[o:o + n]
        o += n
    return pt


def write_index_keys(pages: torch.Tensor, page_table_row: torch.Tensor,
                     codes: torch.Tensor, scale: torch.Tensor, start: int = 0) -> None:
    """Store keys (codes [n,128] uint8, scale [n] f32) of tokens start..start+n."""
    n = codes.shape[0]
    dev = pages.device
    g = torch.arange(start, start + n, device=dev)
    pid = page_table_row.to(dev).long()[g // PAGE_TOKENS]
    slot = g % PAGE_TOKENS
    cols = (slot * INDEX_DIM)[:, None] + torch.arange(INDEX_DIM, device=dev)[None, :]
    pages[pid[:, None], cols] = codes.to(dev)
    sbytes = scale.float().contiguous().view(torch.uint8).view(n, 4).to(dev)
    scols = (PAGE_TOKENS * INDEX_DIM + 4 * slot)[:, None] + torch.arange(4, device=dev)[None, :]
    pages[pid[:, None], scols] = sbytes


def pack_latent_rows(latent: torch.Tensor, rope: torch.Tensor) -> torch.Tensor:
    """[n,512] latent + [n,64] rope -> [n,656] uint8 rows (per-128 e4m3 quant)."""
    n = latent.shape[0]
    codes, scales = quantize_rowwise(latent.float().reshape(n, 4, 128))
    rows = torch.empty(n, LATENT_ROW_BYTES, dtype=torch.uint8, device=latent.device)
    rows[:, :LATENT_DIM] = codes.reshape(n, LATENT_DIM)
    rows[:, LATENT_DIM:LATENT_DIM + 16] = scales.float().contiguous().view(torch.uint8).reshape(n, 16)
    rows[:, LATENT_DIM + 16:] = rope.to(torch.bfloat16).contiguous().view(torch.uint8).reshape(n, 2 * ROPE_DIM)
    return rows


def write_latent_rows(pool: torch.Tensor, page_table_row: torch.Tensor, rows: torch.Tensor,
                      start: int = 0) -> None:
    """Store packed latent rows of tokens start..start+n at their KV slots."""
    n = rows.shape[0]
    dev = pool.device
    g = torch.arange(start, start + n, device=dev)
    slots = page_table_row.to(dev).long()[g // PAGE_TOKENS] * PAGE_TOKENS + g % PAGE_TOKENS
    pool[slots] = rows.to(dev)


def positions_to_slots(page_table: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """Token positions [B,K] -> KV slots (negative positions stay -1)."""
    valid = idx >= 0
    g = idx.clamp_min(0).long()
    slot = torch.gather(page_table.long(), 1, g // PAGE_TOKENS) * PAGE_TOKENS + g % PAGE_TOKENS
    return torch.where(valid, slot, torch.full_like(slot, -1)).to(torch.int32)


def new_index_pool(num_pages: int, device) -> torch.Tensor:
    return torch.zeros(num_pages, INDEX_PAGE_BYTES, dtype=torch.uint8, device=device)


def new_latent_pool(num_pages: int, device) -> torch.Tensor:
    return torch.zeros(num_pages * PAGE_TOKENS, LATENT_ROW_BYTES, dtype=torch.uint8, device=device)
