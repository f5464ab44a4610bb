"""GPU: the decode-time DSALayer adapter (PagedDSALayer) reaches the fused
launch and matches the reference's fused_attention_and_indices
(dsa_layer.py:173-192) on a decode row.

The wrapped layer is a small module with the reference layer's projection
methods (q_latent, _mla_qkv, _indexer_qkw, _project_output) and random
weights.  A 5000-token prefix is appended, then decode rows run through
``fused_attention_and_indices``:
  * the produced set equals the oracle's top-k of the fp8-semantics scores
    over the adapter's caches, bit-exact, and overlaps the fp32 reference
    op's set by > 0.9 (the drop-in's stated agreement with the fp32 path);
  * the attention output equals the oracle's sparse MLA over the attended
    set (rel 2e-2 before the output projection) and the fp32 reference
    computation within the drop-in tolerance 6e-2;
  * attn_indices=None attends densely; produce_indexer=False returns None;
  * lagging: the set one row produces is what the next row attends.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
from torch import nn

from oracle import dsa_oracle as O

from _cases import rel_err

pytestmark = pytest.mark.gpu


class _Cfg:
    hidden_size = 256
    num_attention_heads = 16
    q_lora_rank = 96
    kv_lora_rank = 512
    qk_nope_head_dim = 32
    qk_rope_head_dim = 64
    v_head_dim = 32
    index_n_heads = 64
    index_head_dim = 128
    index_topk = 2048


class _Layer(nn.Module):
    """Projection methods of the reference layer's shape (no rope: the
    adapter hands the rope caches through untouched)."""

    def __init__(self, g: torch.Generator) -> None:
        super().__init__()
        c = self.config = _Cfg()
        h = c.num_attention_heads

        def p(*shape, fan):
            return nn.Parameter(torch.randn(*shape, generator=g) / fan ** 0.5)
        self.wqa = p(c.hidden_size, c.q_lora_rank, fan=c.hidden_size)
        self.wqb = p(c.q_lora_rank, h * (c.qk_nope_head_dim + c.qk_rope_head_dim), fan=c.q_lora_rank)
        self.wkva = p(c.hidden_size, c.kv_lora_rank + c.qk_rope_head_dim, fan=c.hidden_size)
        self.wuk = p(h, c.qk_nope_head_dim, c.kv_lora_rank, fan=c.qk_nope_head_dim)
        self.wuv = p(h, c.v_head_dim, c.kv_lora_rank, fan=c.kv_lora_rank)
        self.wo = p(h * c.v_head_dim, c.hidden_size, fan=h * c.v_head_dim)
        self.wiq = p(c.q_lora_rank, c.index_n_heads * c.index_head_dim, fan=c.q_lora_rank)
        self.wik = p(c.hidden_size, c.index_head_dim, fan=c.hidden_size)
        self.wiw = p(c.q_lora_rank, c.index_n_heads, fan=c.q_lora_rank * c.index_n_heads)

    def q_latent(self, x):
        y = x @ self.wqa
        return y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + 1e-6)

    def _mla_qkv(self, x, c_q, rope):
        c = self.config
        b, s, _ = x.shape
        q = (c_q @ self.wqb).view(b, s, c.num_attention_heads, -1)
        q_nope, q_rope = q[..., :c.qk_nope_head_dim], q[..., c.qk_nope_head_dim:]
        q_abs = torch.einsum("bshd,hdl->bshl", q_nope, self.wuk)
        kv = x @ self.wkva
        return torch.cat([q_abs, q_rope], -1), kv

    def _indexer_qkw(self, x, c_q, rope):
        c = self.config
        b, s, _ = x.shape
        return ((c_q @ self.wiq).view(b, s, c.index_n_heads, c.index_head_dim), x @ self.wik, c_q @ self.wiw)

    def _project_output(self, o_latent):
        b, s = o_latent.shape[:2]
        return torch.einsum("bshl,hdl->bshd", o_latent, self.wuv).reshape(b, s, -1) @ self.wo


def _fp32_reference(layer, xs, x_row, attn_set):
    """The reference ops' fp32 decode row: indexer logits over every key,
    top-k set; attention over attn_set (a set of positions); row at the end."""
    x_all = torch.cat([xs, x_row], dim=1)                   # [1, n, hid]
    c_q = layer.q_latent(x_row)
    q, _ = layer._mla_qkv(x_row, c_q, None)
    _, kv_all = layer._mla_qkv(x_all, layer.q_latent(x_all), None)
    iq, _, w = layer._indexer_qkw(x_row, c_q, None)
    _, ik_all, _ = layer._indexer_qkw(x_all, layer.q_latent(x_all), None)
    d = torch.einsum("hd,nd->hn", iq[0, 0].double(), ik_all[0].double())
    logits = (torch.relu(d) * w[0, 0].double()[:, None]).sum(0)
    top = set(torch.topk(logits, layer.config.index_topk).indices.tolist())
    sel = torch.tensor(sorted(attn_set), dtype=torch.long)
    kvs = kv_all[0, sel].double()
    s = q[0, 0].double() @ kvs.T * 576 ** -0.5
    o = torch.softmax(s, -1) @ kvs[:, :512]
    hidden = layer._project_output(o[None, None].float())
    return top, o.numpy(), hidden


def test_paged_layer_fused_decode_rows(dev):
    from lagged_indexer_dsa_amd import _lib
    from lagged_indexer_dsa_amd.paged_layer import PagedDSALayer

    print("[paged-layer] fused decode rows", flush=True)
    g = torch.Generator().manual_seed(5)
    layer = _Layer(g)
    n0 = 5000
    xs = torch.randn(1, n0, 256, generator=g)
    rows = [torch.randn(1, 1, 256, generator=g) for _ in range(3)]
    layer_cpu = copy.deepcopy(layer)
    layer_d = layer.to(dev)
    with torch.no_grad():
        pl = PagedDSALayer(layer_d, batch=1, max_ctx=8192, device=dev)
        pl.append(xs.to(dev), None)
        _lib.sync_timeouts(reset=True)
        # row 0: dense cold start + its own indexer
        h0, sel0 = pl.fused_attention_and_indices(rows[0].to(dev), None, None, produce_indexer=True)
        torch.cuda.synchronize()
        n = pl.length
        sel0_pos = sel0[0, 0].cpu().numpy()
        # bit-exact against the oracle's fp8 scores over the adapter's caches
        sc = O.indexer_scores(pl.q_fp8.cpu().numpy(), pl.w.cpu().numpy(), pl.index_k.cpu().numpy(),
                              pl.page_table.cpu().numpy(), np.array([n]), pl.cap)
        assert np.allclose(pl.scores[0, :n].cpu().numpy(), sc[0, :n], rtol=0, atol=1e-4 * np.abs(sc[0, :n]).max())
        ref_pos = O.topk_select(pl.scores.cpu().numpy(), np.array([n]), 2048)[0]
        assert np.array_equal(np.sort(sel0_pos[sel0_pos < n]), ref_pos), "selection vs oracle"
        assert np.all(sel0_pos[2048 - (sel0_pos >= n).sum():] == n), "sentinel pads last"
        top32, o32, hid32 = _fp32_reference(layer_cpu, xs, rows[0], set(range(n)))
        assert len(top32 & set(sel0_pos.tolist())) / 2048 > 0.9
        assert rel_err(h0.cpu().numpy(), hid32.detach().numpy()) < 6e-2, "dense row vs fp32 reference"
        # row 1: lagged -- attends row 0's set while producing its own
        h1, sel1 = pl.fused_attention_and_indices(rows[1].to(dev), None, sel0, produce_indexer=True)
        torch.cuda.synchronize()
        attended = pl.attend[0].long()
        ql = pl.out.float()[0].cpu().numpy()
        kv_rows = pl.kv_pool[attended[attended >= 0]].cpu().numpy()
        qb = layer._mla_qkv(rows[1].to(dev), layer.q_latent(rows[1].to(dev)), None)[0]
        ref_o = O.sparse_mla_decode(qb.reshape(1, 16, 576).to(torch.bfloat16).float().cpu().numpy(), kv_rows,
                                    np.arange(kv_rows.shape[0], dtype=np.int32)[None, :], 576 ** -0.5)[0]
        assert rel_err(ql, ref_o) < 2e-2, "lagged attention vs oracle"
        assert set(attended[attended >= 0].cpu().tolist()) == set(sel0_pos[sel0_pos < n0 + 1].tolist())
        # row 2: no indexer
        h2, none = pl.fused_attention_and_indices(rows[2].to(dev), None, sel1, produce_indexer=False)
        assert none is None
        torch.cuda.synchronize()
        assert _lib.sync_timeouts() == 0
        assert pl.length == n0 + 3
