"""Seeded synthetic decode layers of the V3.2 shape (benchmarks, tests).

The workload configs draw every operand N(0,1) (head weights additionally
scaled by 1/sqrt(64)), quantise keys per token and the latent per 128-dim
group to e4m3, and place tokens through a seeded random page table of
64-token pages.  Generation runs on the target device with a seeded device
generator; page tables come from a seeded CPU generator.
"""

from __future__ import annotations

import torch

from . import formats
from ._lib import PAGE_TOKENS
from .decode import DecodeLayer


def pages_for(seq_lens: list[int]) -> int:
    return sum((n + PAGE_TOKENS - 1) // PAGE_TOKENS for n in seq_lens)


def make_page_table(seq_lens: list[int], seed: int, device, pt_stride: int | None = None,
                    num_pages: int | None = None) -> tuple[torch.Tensor, int]:
    need = max((n + PAGE_TOKENS - 1) // PAGE_TOKENS for n in seq_lens)
    pt_stride = pt_stride or need
    num_pages = num_pages or pages_for(seq_lens)
    gen = torch.Generator().manual_seed(seed)
    pt = formats.random_page_table(seq_lens, pt_stride, num_pages, generator=gen)
    return pt.to(device), num_pages


def make_decode_layer(seq_lens: list[int], *, seed: int, device, page_table: torch.Tensor,
                      num_pages: int, hidx: int = 64, heads: int = 16, topk: int = 2048,
                      slab_stride: int | None = None, indexer: bool = True,
                      nsplit: int = 0) -> DecodeLayer:
    """One layer: own caches and queries, shared page table."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    B = len(seq_lens)
    slab_stride = slab_stride or page_table.shape[1] * PAGE_TOKENS
    pt_cpu = page_table.cpu()
    index_k = formats.new_index_pool(num_pages, dev) if indexer else None
    kv_pool = formats.new_latent_pool(num_pages, dev)
    for b, n in enumerate(seq_lens):
        if indexer:
            keys = torch.randn(n, 128, generator=g, device=dev)
            codes, sc = formats.quantize_rowwise(keys)
            formats.write_index_keys(index_k, pt_cpu[b], codes, sc)
            del keys, codes, sc
        lat = torch.randn(n, 576, generator=g, device=dev)
        rows = formats.pack_latent_rows(lat[:, :512], lat[:, 512:])
        formats.write_latent_rows(kv_pool, pt_cpu[b], rows)
        del lat, rows
    q_fp8 = w = None
    if indexer:
        q_idx = torch.randn(B, hidx, 128, generator=g, device=dev)
        w_raw = torch.randn(B, hidx, generator=g, device=dev) * (hidx ** -0.5)
        q_fp8, w = formats.quantize_index_query(q_idx, w_raw)
    q_mla = torch.randn(B, heads, 576, generator=g, device=dev).to(torch.bfloat16)
    seq = torch.tensor(seq_lens, dtype=torch.int32, device=dev)
    return DecodeLayer(q_fp8=q_fp8, w=w, index_k=index_k, q_bf16=q_mla, kv_pool=kv_pool,
                       page_table=page_table, seq_lens=seq, slab_stride=slab_stride, topk=topk,
                       nsplit=nsplit)


def random_selection(seq_lens: list[int], topk: int, page_table: torch.Tensor, seed: int,
                     device) -> torch.Tensor:
    """A seeded top-k-shaped set of distinct KV slots per row (cold-start /
    previous-step selection for the first layer of a lagged stack)."""
    gen = torch.Generator().manual_seed(seed)
    B = len(seq_lens)
    pos = torch.full((B, topk), -1, dtype=torch.int64)
    for b, n in enumerate(seq_lens):
        k = min(topk, n)
        pos[b, :k] = torch.randperm(n, generator=gen)[:k].sort().values
    return formats.positions_to_slots(page_table.cpu(), pos).to(device)
