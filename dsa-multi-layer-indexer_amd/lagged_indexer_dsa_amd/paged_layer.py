"""Decode-time adapter of a ``DSALayer``: persistent paged fp8 caches and the
fused layer launch.

The reference's ``DSALayer.fused_attention_and_indices`` (dsa_layer.py:173-192)
recomputes the whole key set on every call.  At decode time the keys of the
prefix never change, so :class:`PagedDSALayer` keeps them where the serving
path keeps them -- the paged index-K cache and the 656-byte fp8 latent pool
of one layer -- appends each new token once (the HIP quantizers of
``ops.append_index_keys`` / ``ops.append_latent_rows``), and answers a decode
row with ONE ``dsa_decode_layer`` launch: the attention over the given
(lagged) selection and this layer's indexer scan and top-k side by side.

It wraps any module with the reference layer's projection methods
(``q_latent``, ``_mla_qkv``, ``_indexer_qkw``, ``_project_output`` and a
``config`` with ``index_topk``); the projections stay in torch, outside the
timed hot path.  Shapes the kernels accept: kv_lora_rank 512, rope 64
(576-wide absorbed queries), index_head_dim 128, index_n_heads 16/32/48/64,
attention heads a multiple of 16.

Index convention: selections cross this API as token positions, int64
``[B, 1, topk]`` like ``select_topk`` returns them, with the sentinel
``S_kv`` (the row length) for unused entries.  They come back in ascending
position order -- the decode kernels' order -- where ``select_topk`` orders by
score; both are the same set, which is all ``sparse_mla_core`` reads.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib, ops
from ._lib import INDEX_DIM, LATENT_DIM, PAGE_TOKENS, QK_DIM, LayerArgs


class PagedDSALayer:
    """Paged caches of one layer for ``batch`` rows of up to ``max_ctx``
    tokens each (identity paging: row b owns pages [b*npg, (b+1)*npg))."""

    def __init__(self, layer, batch: int, max_ctx: int, device=None, nsplit: int = 0) -> None:
        cfg = layer.config
        if cfg.kv_lora_rank + cfg.qk_rope_head_dim != QK_DIM or cfg.kv_lora_rank != LATENT_DIM:
            raise ValueError("the fp8 latent format needs kv_lora_rank 512 and qk_rope_head_dim 64")
        if cfg.index_head_dim != INDEX_DIM or cfg.index_n_heads not in (16, 32, 48, 64):
            raise ValueError("the fp8 indexer needs index_head_dim 128 and 16/32/48/64 index heads")
        if cfg.num_attention_heads % 16:
            raise ValueError("the attention heads must be a multiple of 16")
        dev = torch.device(device) if device is not None else next(layer.parameters()).device
        self.layer, self.B, self.topk = layer, int(batch), int(cfg.index_topk)
        self.H, self.Hidx = cfg.num_attention_heads, cfg.index_n_heads
        self.npg = max(1, -(-int(max_ctx) // PAGE_TOKENS))
        self.cap = self.npg * PAGE_TOKENS
        B = self.B
        self.page_table = (torch.arange(B, dtype=torch.int32, device=dev)[:, None] * self.npg
                           + torch.arange(self.npg, dtype=torch.int32, device=dev)[None, :]).contiguous()
        self.index_k = torch.zeros(B * self.npg, _lib.INDEX_PAGE_BYTES, dtype=torch.uint8, device=dev)
        self.kv_pool = torch.zeros(B * self.cap, _lib.LATENT_ROW_BYTES, dtype=torch.uint8, device=dev)
        self.seq_lens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.length = 0
        self.scores = torch.empty(B, self.cap, dtype=torch.float32, device=dev)
        self.topk_scratch = ops.topk_scratch(B, self.cap, dev)
        self.next_idx = torch.full((B, self.topk), -1, dtype=torch.int32, device=dev)
        self.attend = torch.full((B, self.topk), -1, dtype=torch.int32, device=dev)
        self.nsplit = int(nsplit)
        self.workspace = ops.sparse_mla_workspace(B, self.H, self.nsplit, dev)
        self.out = torch.zeros(B, self.H, LATENT_DIM, dtype=torch.bfloat16, device=dev)
        self.q_fp8 = torch.empty(B, self.Hidx, INDEX_DIM, dtype=torch.uint8, device=dev)
        self.w = torch.empty(B, self.Hidx, dtype=torch.float32, device=dev)
        self._rows = torch.arange(B, dtype=torch.int32, device=dev)
        self._base = (torch.arange(B, dtype=torch.int64, device=dev) * self.cap)[:, None]

    # ---- cache maintenance ----
    def _append(self, index_k: torch.Tensor, kv: torch.Tensor) -> None:
        """Store keys [B,S,128] and latent rows [B,S,576] of the next S tokens."""
        B, S = kv.shape[0], kv.shape[1]
        if self.length + S > self.cap:
            raise ValueError(f"context {self.length + S} above the cache's {self.cap} tokens")
        pos = torch.arange(self.length, self.length + S, dtype=torch.int32, device=kv.device)
        rows = self._rows.repeat_interleave(S)
        posb = pos.repeat(B)
        ops.append_index_keys(self.index_k, self.page_table, rows, posb,
                              index_k.reshape(B * S, INDEX_DIM).to(torch.bfloat16).contiguous())
        slots = (rows.long() * self.cap + posb.long()).to(torch.int32)
        ops.append_latent_rows(self.kv_pool, slots, kv.reshape(B * S, QK_DIM).to(torch.bfloat16).contiguous())
        self.length += S
        self.seq_lens.fill_(self.length)

    def append(self, x_norm: torch.Tensor, rope) -> None:
        """Project and store the keys of S new tokens ([B, S, hidden], rope
        caches for their positions) without attending (prompt prefill)."""
        c_q = self.layer.q_latent(x_norm)
        _, kv = self.layer._mla_qkv(x_norm, c_q, rope)
        _, index_k, _ = self.layer._indexer_qkw(x_norm, c_q, rope)
        self._append(index_k, kv)

    # ---- index conventions ----
    def _to_slots(self, indices: torch.Tensor) -> torch.Tensor:
        """[B,1,topk] positions (sentinel / negatives unused) -> int32 KV slots."""
        idx = indices.reshape(self.B, -1).long()
        if idx.shape[1] != self.topk:
            raise ValueError(f"indices must be [B, 1, {self.topk}], got {tuple(indices.shape)}")
        ok = (idx >= 0) & (idx < self.length)
        return torch.where(ok, idx + self._base, torch.full_like(idx, -1)).to(torch.int32)

    def _to_positions(self, slots: torch.Tensor) -> torch.Tensor:
        s = slots.long()
        return torch.where(s >= 0, s - self._base, torch.full_like(s, self.length)).reshape(self.B, 1, self.topk)

    # ---- the decode row ----
    def fused_attention_and_indices(self, x_norm: torch.Tensor, rope, attn_indices: torch.Tensor | None,
                                    produce_indexer: bool = True):
        """The decode row at position ``length`` ([B, 1, hidden], rope caches
        for that position): its key and latent row are appended first (a row
        attends itself), then one launch attends ``attn_indices`` (dense when
        None) and, if asked, runs this layer's indexer.  Returns (attention
        hidden output [B, 1, hidden], next indices [B, 1, topk] or None)
        (dsa_layer.py:173-192)."""
        if x_norm.dim() != 3 or x_norm.shape[:2] != (self.B, 1):
            raise ValueError(f"x_norm must be [{self.B}, 1, hidden] (one decode row per request)")
        lay = self.layer
        c_q = lay.q_latent(x_norm)
        q, kv = lay._mla_qkv(x_norm, c_q, rope)
        index_q = index_k = weights = None
        if produce_indexer:
            index_q, index_k, weights = lay._indexer_qkw(x_norm, c_q, rope)
        else:
            _, index_k, _ = lay._indexer_qkw(x_norm, c_q, rope)
        self._append(index_k, kv)
        q_bf16 = q.reshape(self.B, self.H, QK_DIM).to(torch.bfloat16).contiguous()
        if produce_indexer:
            ops.quantize_index_query(index_q.reshape(self.B, self.Hidx, INDEX_DIM).to(torch.bfloat16).contiguous(),
                                     weights.reshape(self.B, self.Hidx).float().contiguous(),
                                     out_q=self.q_fp8, out_w=self.w)
        a = LayerArgs()
        if produce_indexer:
            a.q_fp8, a.w = self.q_fp8.data_ptr(), self.w.data_ptr()
            a.index_k, a.num_idx_pages = self.index_k.data_ptr(), self.index_k.shape[0]
            a.Hidx = self.Hidx
        a.scores, a.topk_scratch, a.next_idx = (self.scores.data_ptr(), self.topk_scratch.data_ptr(),
                                                self.next_idx.data_ptr())
        a.q_bf16, a.kv_pool, a.kv_rows = q_bf16.data_ptr(), self.kv_pool.data_ptr(), self.kv_pool.shape[0]
        a.workspace, a.out_bf16 = self.workspace.data_ptr(), self.out.data_ptr()
        if attn_indices is None:
            a.dense = 1
        else:
            self.attend.copy_(self._to_slots(attn_indices))
            a.attend_idx = self.attend.data_ptr()
        a.page_table, a.seq_lens = self.page_table.data_ptr(), self.seq_lens.data_ptr()
        a.B, a.H, a.topk, a.nsplit = self.B, self.H, self.topk, self.nsplit
        a.pt_stride, a.slab_stride = self.npg, self.cap
        a.sm_scale = QK_DIM ** -0.5
        _lib.call("dsa_decode_layer", ctypes.byref(a), torch.cuda.current_stream().cuda_stream)
        o_latent = self.out.float().reshape(self.B, 1, self.H, LATENT_DIM).to(x_norm.dtype)
        hidden = lay._project_output(o_latent)
        nxt = self._to_positions(self.next_idx) if produce_indexer else None
        return hidden, nxt
