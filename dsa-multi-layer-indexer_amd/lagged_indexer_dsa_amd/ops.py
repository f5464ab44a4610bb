"""torch-tensor entry points onto the C ABI (one launch sequence each).

Every op requires device (HIP) tensors and runs on torch's current stream;
there is no CPU path.  Shapes/dtypes are checked here; the library re-checks
its own contract and raises :class:`DsaError` (a RuntimeError) on violation.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import (
    DSA_TOPK_POSITION_ORDER,
    DSA_TOPK_SORTED,
    INDEX_DIM,
    INDEX_PAGE_BYTES,
    LATENT_DIM,
    LATENT_ROW_BYTES,
    QK_DIM,
)


def _dev(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise RuntimeError("lagged_indexer_dsa_amd ops need GPU (HIP) tensors; there is no CPU path")
        if not t.is_contiguous():
            raise RuntimeError("lagged_indexer_dsa_amd ops need contiguous tensors")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def _need_bytes(name: str, t: torch.Tensor, nbytes: int) -> None:
    """The C ABI takes raw pointers: a caller buffer smaller than the
    library's size function says would be overrun on the device."""
    if _nbytes(t) < nbytes:
        raise RuntimeError(f"{name} holds {_nbytes(t)} bytes, the call needs {nbytes}")


def _need_shape(name: str, t: torch.Tensor, shape: tuple, dtype) -> None:
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype or not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous {dtype} {tuple(shape)}, got {t.dtype} {tuple(t.shape)}")


def indexer_scan(q_fp8: torch.Tensor, w: torch.Tensor, index_k: torch.Tensor,
                 page_table: torch.Tensor, seq_lens: torch.Tensor, slab_stride: int,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """fp8 lightning-indexer scores over the paged index-K cache.

    q_fp8 [B,Hidx,128] uint8 (e4m3 codes) or float8_e4m3fn; w [B,Hidx] f32
    (q-scale folded in); index_k [P,8448] uint8; page_table [B,pt] int32;
    seq_lens [B] int32  ->  scores [B, slab_stride] f32 (-inf past seq_len).
    Reference: K:2990-2992 ref_indexer_logits_fp8; attention_core.py:27-49.
    """
    q_fp8 = q_fp8.view(torch.uint8) if q_fp8.dtype == torch.float8_e4m3fn else q_fp8
    _dev(q_fp8, w, index_k, page_table, seq_lens)
    B, Hidx, D = q_fp8.shape
    if D != INDEX_DIM or q_fp8.dtype != torch.uint8:
        raise RuntimeError("q_fp8 must be [B, Hidx, 128] e4m3 bytes")
    if w.shape != (B, Hidx) or w.dtype != torch.float32:
        raise RuntimeError("w must be [B, Hidx] float32")
    if index_k.dim() != 2 or index_k.shape[1] != INDEX_PAGE_BYTES or index_k.dtype != torch.uint8:
        raise RuntimeError("index_k must be [pages, 8448] uint8")
    if page_table.dim() != 2 or page_table.shape[0] != B or page_table.dtype != torch.int32:
        raise RuntimeError("page_table must be [B, pt_stride] int32")
    if seq_lens.shape != (B,) or seq_lens.dtype != torch.int32:
        raise RuntimeError("seq_lens must be [B] int32")
    if out is None:
        out = torch.empty(B, slab_stride, dtype=torch.float32, device=q_fp8.device)
    _dev(out)
    if out.shape != (B, slab_stride) or out.dtype != torch.float32:
        raise RuntimeError("out must be [B, slab_stride] float32")
    _lib.call("dsa_indexer_scan", q_fp8.data_ptr(), w.data_ptr(), index_k.data_ptr(),
              index_k.shape[0], page_table.data_ptr(), seq_lens.data_ptr(), out.data_ptr(),
              B, Hidx, page_table.shape[1], slab_stride, _stream())
    return out


def topk_scratch(B: int, slab: int, device) -> torch.Tensor:
    """Zero-filled scratch for :func:`topk` (each call leaves it zeroed)."""
    nbytes = _lib.load().dsa_topk_scratch_bytes(B, slab)
    if nbytes == 0:
        raise RuntimeError(f"bad top-k scratch shape B={B} slab={slab}")
    return torch.zeros(nbytes // 4, dtype=torch.int32, device=device)


def topk(scores: torch.Tensor, seq_lens: torch.Tensor, k: int, sorted: bool = False,
         pad_value: int = -1, page_table: torch.Tensor | None = None,
         out: torch.Tensor | None = None, scratch: torch.Tensor | None = None) -> torch.Tensor:
    """Exact top-k per row (score desc, ties -> lower index), int32 [B, k].

    sorted=False: ascending positions (or KV slots through page_table), pads
    last.  sorted=True: torch.topk order with the lower-index tie rule.
    Non-finite selections and missing slots are ``pad_value``.
    Reference: attention_core.py:66-91 select_topk.
    """
    _dev(scores, seq_lens)
    if scores.dim() != 2 or scores.dtype != torch.float32:
        raise RuntimeError("scores must be [B, slab] float32")
    B, slab = scores.shape
    if seq_lens.shape != (B,) or seq_lens.dtype != torch.int32:
        raise RuntimeError("seq_lens must be [B] int32")
    if page_table is not None:
        _dev(page_table)
    if out is None:
        out = torch.empty(B, k, dtype=torch.int32, device=scores.device)
    if scratch is None:
        scratch = topk_scratch(B, slab, scores.device)
    _dev(out, scratch)
    _need_shape("out", out, (B, k), torch.int32)
    _need_bytes("top-k scratch", scratch, _lib.load().dsa_topk_scratch_bytes(B, slab))
    _lib.call("dsa_topk", scores.data_ptr(), seq_lens.data_ptr(), _ptr(page_table),
              0 if page_table is None else page_table.shape[1], scratch.data_ptr(),
              out.data_ptr(), B, slab, k,
              DSA_TOPK_SORTED if sorted else DSA_TOPK_POSITION_ORDER, pad_value, _stream())
    return out


def sparse_mla_workspace(B: int, H: int, nsplit: int, device) -> torch.Tensor:
    """Zero-filled workspace (split partials + the splits' barriers; every
    call leaves the barriers ready).  nsplit=0 sizes it for any split count."""
    nbytes = _lib.load().dsa_sparse_mla_workspace_bytes(B, H, nsplit)
    if nbytes == 0:
        raise RuntimeError(f"bad sparse MLA workspace shape B={B} H={H} nsplit={nsplit}")
    return torch.zeros(nbytes // 4, dtype=torch.float32, device=device)


def sparse_mla_decode(q: torch.Tensor, kv_pool: torch.Tensor, idx: torch.Tensor,
                      sm_scale: float | None = None, nsplit: int = 0,
                      workspace: torch.Tensor | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Split-K sparse MLA over the fp8 656-byte latent pool.

    q [B,H,576] bf16; kv_pool [rows,656] uint8; idx [B,topk] int32 KV slots
    (out-of-range = masked)  ->  out [B,H,512] bf16.
    Reference: attention_core.py:121-146 sparse_mla_core; K:2950-2966.
    """
    _dev(q, kv_pool, idx)
    if q.dim() != 3 or q.shape[2] != QK_DIM or q.dtype != torch.bfloat16:
        raise RuntimeError("q must be [B, H, 576] bfloat16")
    B, H, _ = q.shape
    if kv_pool.dim() != 2 or kv_pool.shape[1] != LATENT_ROW_BYTES or kv_pool.dtype != torch.uint8:
        raise RuntimeError("kv_pool must be [rows, 656] uint8")
    if idx.dim() != 2 or idx.shape[0] != B or idx.dtype != torch.int32:
        raise RuntimeError("idx must be [B, topk] int32")
    if sm_scale is None:
        sm_scale = QK_DIM ** -0.5
    if workspace is None:
        workspace = sparse_mla_workspace(B, H, nsplit, q.device)
    if out is None:
        out = torch.empty(B, H, LATENT_DIM, dtype=torch.bfloat16, device=q.device)
    _dev(workspace, out)
    _need_shape("out", out, (B, H, LATENT_DIM), torch.bfloat16)
    # sized for this nsplit (nsplit=0, the library's choice: the largest size)
    _need_bytes("sparse MLA workspace", workspace, _lib.load().dsa_sparse_mla_workspace_bytes(B, H, nsplit))
    _lib.call("dsa_sparse_mla_decode", q.data_ptr(), kv_pool.data_ptr(), kv_pool.shape[0],
              idx.data_ptr(), workspace.data_ptr(), out.data_ptr(), B, H, idx.shape[1], nsplit,
              float(sm_scale), _stream())
    return out


def dense_mla_decode(q: torch.Tensor, kv_pool: torch.Tensor, page_table: torch.Tensor, seq_lens: torch.Tensor,
                     sm_scale: float | None = None, nsplit: int = 0,
                     workspace: torch.Tensor | None = None,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Dense MLA of each decode row over its first seq_lens[b] tokens, their
    latent rows found through the page table (64-token pages).

    q [B,H,576] bf16; kv_pool [rows,656] uint8; page_table [B,pt] int32;
    seq_lens [B] int32  ->  out [B,H,512] bf16.
    Reference: attention_core.py:142-160 dense_mla_core; model.py:104-114.
    """
    _dev(q, kv_pool, page_table, seq_lens)
    if q.dim() != 3 or q.shape[2] != QK_DIM or q.dtype != torch.bfloat16:
        raise RuntimeError("q must be [B, H, 576] bfloat16")
    B, H, _ = q.shape
    if kv_pool.dim() != 2 or kv_pool.shape[1] != LATENT_ROW_BYTES or kv_pool.dtype != torch.uint8:
        raise RuntimeError("kv_pool must be [rows, 656] uint8")
    if page_table.dim() != 2 or page_table.shape[0] != B or page_table.dtype != torch.int32:
        raise RuntimeError("page_table must be [B, pt_stride] int32")
    _need_shape("seq_lens", seq_lens, (B,), torch.int32)
    if sm_scale is None:
        sm_scale = QK_DIM ** -0.5
    if workspace is None:
        workspace = sparse_mla_workspace(B, H, nsplit, q.device)
    if out is None:
        out = torch.empty(B, H, LATENT_DIM, dtype=torch.bfloat16, device=q.device)
    _dev(workspace, out)
    _need_shape("out", out, (B, H, LATENT_DIM), torch.bfloat16)
    _need_bytes("sparse MLA workspace", workspace, _lib.load().dsa_sparse_mla_workspace_bytes(B, H, nsplit))
    _lib.call("dsa_dense_mla_decode", q.data_ptr(), kv_pool.data_ptr(), kv_pool.shape[0], page_table.data_ptr(),
              page_table.shape[1], seq_lens.data_ptr(), workspace.data_ptr(), out.data_ptr(), B, H, nsplit,
              float(sm_scale), _stream())
    return out


# ---- decode-step operand preparation (the inputs the decode layer reads) ----

def quantize_index_query(q: torch.Tensor, w: torch.Tensor, out_q: torch.Tensor | None = None,
                         out_w: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Indexer query [B, Hidx, 128] bf16 and head weights [B, Hidx] fp32 ->
    (e4m3 codes uint8 [B, Hidx, 128], folded weights w * scale fp32).
    Per (token, head): scale = max(amax, 1e-6) / 448 (K:2969-2974, K:2984-2985)."""
    _dev(q, w)
    if q.dim() != 3 or q.shape[2] != INDEX_DIM or q.dtype != torch.bfloat16:
        raise RuntimeError("q must be [B, Hidx, 128] bfloat16")
    B, H, _ = q.shape
    _need_shape("w", w, (B, H), torch.float32)
    if out_q is None:
        out_q = torch.empty(B, H, INDEX_DIM, dtype=torch.uint8, device=q.device)
    if out_w is None:
        out_w = torch.empty(B, H, dtype=torch.float32, device=q.device)
    _dev(out_q, out_w)
    _need_shape("out_q", out_q, (B, H, INDEX_DIM), torch.uint8)
    _need_shape("out_w", out_w, (B, H), torch.float32)
    _lib.call("dsa_quantize_index_query", q.data_ptr(), w.data_ptr(), out_q.data_ptr(), out_w.data_ptr(),
              B, H, _stream())
    return out_q, out_w


def append_index_keys(index_k: torch.Tensor, page_table: torch.Tensor, rows: torch.Tensor,
                      pos: torch.Tensor, keys: torch.Tensor) -> None:
    """Quantize keys [n, 128] bf16 (per token, e4m3 + fp32 scale) into the
    paged index cache at token positions pos[i] of rows rows[i] (P:339-342)."""
    _dev(index_k, page_table, rows, pos, keys)
    n = keys.shape[0]
    if keys.dim() != 2 or keys.shape[1] != INDEX_DIM or keys.dtype != torch.bfloat16:
        raise RuntimeError("keys must be [n, 128] bfloat16")
    if index_k.dim() != 2 or index_k.shape[1] != INDEX_PAGE_BYTES or index_k.dtype != torch.uint8:
        raise RuntimeError("index_k must be [pages, 8448] uint8")
    if page_table.dim() != 2 or page_table.dtype != torch.int32:
        raise RuntimeError("page_table must be [B, pt_stride] int32")
    _need_shape("rows", rows, (n,), torch.int32)
    _need_shape("pos", pos, (n,), torch.int32)
    _lib.call("dsa_append_index_keys", keys.data_ptr(), rows.data_ptr(), pos.data_ptr(), n,
              page_table.data_ptr(), page_table.shape[1], index_k.data_ptr(), index_k.shape[0], _stream())


def append_latent_rows(kv_pool: torch.Tensor, slots: torch.Tensor, latent: torch.Tensor) -> None:
    """Pack latent [n, 576] bf16 (512 latent | 64 rope) into 656-byte fp8 rows
    at KV slots slots[i] (per-128 e4m3 + fp32 scales, bf16 rope; K:1114)."""
    _dev(kv_pool, slots, latent)
    n = latent.shape[0]
    if latent.dim() != 2 or latent.shape[1] != QK_DIM or latent.dtype != torch.bfloat16:
        raise RuntimeError("latent must be [n, 576] bfloat16")
    if kv_pool.dim() != 2 or kv_pool.shape[1] != LATENT_ROW_BYTES or kv_pool.dtype != torch.uint8:
        raise RuntimeError("kv_pool must be [rows, 656] uint8")
    _need_shape("slots", slots, (n,), torch.int32)
    _lib.call("dsa_append_latent_rows", latent.data_ptr(), slots.data_ptr(), n, kv_pool.data_ptr(),
              kv_pool.shape[0], _stream())
