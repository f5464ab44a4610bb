"""CPU oracle for the DSA decode hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of the reference's decode path
so the HIP kernels can be checked against it.  It is imported only by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py``, and only as the checker: nothing in the shipped package calls
it, and the package fails loudly when its HIP library is missing.

Every function cites the reference file:line it follows.  Abbreviations:
``K:`` = ``kernels/cuda_fused_sparse_splitk.py``; ``AC:`` =
``src/lagged_indexer_dsa/attention_core.py``; ``ML:`` =
``src/lagged_indexer_dsa/model.py``.

How each function is pinned (tests/test_oracle.py):
  e4m3_decode / e4m3_encode  -- all 256 codes and 2e5 values against torch's
                                float8_e4m3fn (the OCP definition).
  bf16_rn                     -- against torch's float32 -> bfloat16 cast.
  quantize_rowwise            -- round trip bound |x - deq| <= scale/16 *|x|
                                 and exactness on representable inputs.
  indexer_scores              -- brute-force Python loops; w=0 -> 0; one head
                                 closed form; page-permutation invariance;
                                 linearity in w.
  topk_select                 -- brute-force sort on tiny rows; torch.topk
                                 value multiset; forced ties; -inf/NaN rows.
  sparse_mla_decode           -- brute-force loops; permutation invariance;
                                 one-key closed form (output = value row);
                                 split + lse_merge == one pass; masked -> 0.
  lagged_indexer_layers / mli_plan -- the reference's own examples
                                 (ML:61-71 docstring cases).
Nothing here is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

PAGE_TOKENS = 64
INDEX_DIM = 128
INDEX_PAGE_BYTES = PAGE_TOKENS * INDEX_DIM + PAGE_TOKENS * 4  # 8448, K:2428
LATENT_DIM = 512
ROPE_DIM = 64
QK_DIM = LATENT_DIM + ROPE_DIM  # 576, config.py:122-125
LATENT_ROW_BYTES = LATENT_DIM + 4 * 4 + ROPE_DIM * 2  # 656, K:1114
E4M3_MAX = 448.0

# --------------------------------------------------------------------------
# fp8 e4m3fn codec (OCP; the format of torch.float8_e4m3fn and of gfx950's
# fp8 instructions).  Reference uses it via .to(torch.float8_e4m3fn)
# (K:2969-2974) and decodes it exactly (K:123-133).
# --------------------------------------------------------------------------


def _e4m3_table() -> np.ndarray:
    """Value of each of the 256 codes: s eeee mmm, bias 7, 0x7f/0xff NaN."""
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            out[code] = np.nan
        elif e == 0:
            out[code] = s * m * 2.0 ** -9
        else:
            out[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


E4M3_TABLE = _e4m3_table()
_POS_CODES = np.arange(0, 0x7F)  # finite non-negative codes, increasing value
_POS_VALUES = E4M3_TABLE[_POS_CODES]


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values (exact)."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float -> e4m3fn code, round to nearest, ties to even mantissa.

    Inputs are expected in [-448, 448] (callers clamp first, as K:2973 does);
    larger magnitudes saturate to +-448 here, NaN maps to 0x7f.
    """
    x = np.asarray(x, dtype=np.float64)
    a = np.minimum(np.abs(x), E4M3_MAX)
    hi = np.searchsorted(_POS_VALUES, a, side="left")  # first value >= a
    hi = np.clip(hi, 0, len(_POS_VALUES) - 1)
    lo = np.clip(hi - 1, 0, len(_POS_VALUES) - 1)
    d_hi = _POS_VALUES[hi] - a
    d_lo = a - _POS_VALUES[lo]
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((_POS_CODES[hi] & 1) == 0))
    code = np.where(pick_hi, _POS_CODES[hi], _POS_CODES[lo]).astype(np.uint8)
    neg = np.signbit(x)
    code = np.where(neg, code | 0x80, code).astype(np.uint8)
    code = np.where(np.isnan(x), np.uint8(0x7F), code)
    return code.astype(np.uint8)


def bf16_rn(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 (already bf16-representable) -> uint16 bits."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------
# Quantisers (fixture generation).  K:2969-2974 quantize_e4m3_rowwise.
# --------------------------------------------------------------------------


def quantize_rowwise(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric e4m3: scale = max(amax, 1e-6)/448, code = e4m3(x/scale).

    K:2969-2974: amax.clamp_min(1e-6) / 448, (x/scale).clamp(-448, 448).
    Arithmetic in float32 like the reference's torch ops.
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.maximum(np.abs(x).max(axis=-1, keepdims=True), np.float32(1e-6))
    scale = (amax / np.float32(E4M3_MAX)).astype(np.float32)
    y = np.clip(x / scale, -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return e4m3_encode(y), scale[..., 0]


# --------------------------------------------------------------------------
# Paged layouts.  index-K page K:540-546, K:630, K:2428; latent row K:1114,
# K:1355-1395 (656 B: 512 e4m3 | 4 f32 group scales | 64 bf16 rope).
# --------------------------------------------------------------------------


def pack_index_pages(k_codes: np.ndarray, k_scale: np.ndarray, page_ids: np.ndarray,
                     num_pages: int) -> np.ndarray:
    """Scatter one row's keys (token order) into [num_pages, 8448] pages."""
    n = k_codes.shape[0]
    pages = np.zeros((num_pages, INDEX_PAGE_BYTES), dtype=np.uint8)
    for lp in range((n + PAGE_TOKENS - 1) // PAGE_TOKENS):
        g0, g1 = lp * PAGE_TOKENS, min(n, (lp + 1) * PAGE_TOKENS)
        pg = pages[page_ids[lp]]
        pg[: (g1 - g0) * INDEX_DIM] = k_codes[g0:g1].reshape(-1)
        sc = np.zeros(PAGE_TOKENS, dtype=np.float32)
        sc[: g1 - g0] = k_scale[g0:g1]
        pg[PAGE_TOKENS * INDEX_DIM:] = sc.view(np.uint8)
    return pages


def read_index_keys(pages: np.ndarray, page_table_row: np.ndarray, n: int):
    """Gather a row's first n keys back out of the pages: (codes [n,128], scale [n])."""
    codes = np.empty((n, INDEX_DIM), dtype=np.uint8)
    scale = np.empty(n, dtype=np.float32)
    for g0 in range(0, n, PAGE_TOKENS):
        g1 = min(n, g0 + PAGE_TOKENS)
        pg = pages[page_table_row[g0 // PAGE_TOKENS]]
        codes[g0:g1] = pg[: (g1 - g0) * INDEX_DIM].reshape(g1 - g0, INDEX_DIM)
        scale[g0:g1] = pg[PAGE_TOKENS * INDEX_DIM:].view(np.float32)[: g1 - g0]
    return codes, scale


def pack_latent_rows(latent: np.ndarray, rope: np.ndarray) -> np.ndarray:
    """[n,512] f32 latent + [n,64] rope -> [n,656] bytes, per-128 e4m3 quant."""
    n = latent.shape[0]
    codes, scales = quantize_rowwise(np.asarray(latent, np.float32).reshape(n, 4, 128))
    rows = np.zeros((n, LATENT_ROW_BYTES), dtype=np.uint8)
    rows[:, :LATENT_DIM] = codes.reshape(n, LATENT_DIM)
    rows[:, LATENT_DIM:LATENT_DIM + 16] = scales.astype(np.float32).view(np.uint8).reshape(n, 16)
    rows[:, LATENT_DIM + 16:] = bf16_bits(bf16_rn(rope)).view(np.uint8).reshape(n, 128)
    return rows


def dequant_latent_rows(rows: np.ndarray) -> np.ndarray:
    """[n,656] bytes -> [n,576] float32 of bf16 values.

    bf16_rn(f32(e4m3) * scale[d/128]) for d < 512 (K:1181-1197), rope as stored.
    """
    rows = np.asarray(rows, dtype=np.uint8)
    n = rows.shape[0]
    vals = e4m3_decode(rows[:, :LATENT_DIM]).reshape(n, 4, 128)
    scales = rows[:, LATENT_DIM:LATENT_DIM + 16].copy().view(np.float32).reshape(n, 4, 1)
    nope = bf16_rn((vals * scales).astype(np.float32)).reshape(n, LATENT_DIM)
    rope = bf16_from_bits(rows[:, LATENT_DIM + 16:].copy().view(np.uint16))
    return np.concatenate([nope, rope], axis=1).astype(np.float32)


def slot_of(page_table_row: np.ndarray, g: np.ndarray) -> np.ndarray:
    """Token position -> KV slot through the page table (hp_page_to_slot, K:1142-1144)."""
    g = np.asarray(g, dtype=np.int64)
    return page_table_row[g // PAGE_TOKENS].astype(np.int64) * PAGE_TOKENS + g % PAGE_TOKENS


# --------------------------------------------------------------------------
# (1) indexer score.  AC:27-49 (fp32 form), fp8 form K:2990-2992 and
# inference/modeling/kernels.py:285-312: s_k * sum_h wp_h * ReLU(q_h . k).
# --------------------------------------------------------------------------


def indexer_scores(q_codes: np.ndarray, w: np.ndarray, pages: np.ndarray,
                   page_table: np.ndarray, seq_lens: np.ndarray, slab_stride: int) -> np.ndarray:
    """[B,H,128] codes, [B,H] w -> [B, slab_stride] float64 scores, -inf tail."""
    B = q_codes.shape[0]
    out = np.full((B, slab_stride), -np.inf, dtype=np.float64)
    for b in range(B):
        n = int(min(seq_lens[b], slab_stride, page_table.shape[1] * PAGE_TOKENS))
        if n <= 0:
            continue
        kc, ks = read_index_keys(pages, page_table[b], n)
        q = e4m3_decode(q_codes[b]).astype(np.float64)          # [H,128]
        k = e4m3_decode(kc).astype(np.float64)                   # [n,128]
        dots = q @ k.T                                           # [H,n] exact
        out[b, :n] = ks.astype(np.float64) * (np.maximum(dots, 0.0) * w[b].astype(np.float64)[:, None]).sum(0)
    return out


def indexer_logits_fp32(index_q: np.ndarray, index_k: np.ndarray, weights: np.ndarray) -> np.ndarray:
    """AC:27-49 verbatim semantics: [B,S,H,D],[B,Skv,D],[B,S,H] -> [B,S,Skv]."""
    score = np.einsum("bshd,bnd->bshn", index_q, index_k)
    return (np.maximum(score, 0) * weights[..., None]).sum(axis=2)


# --------------------------------------------------------------------------
# (2) top-k.  AC:66-91 select_topk (torch.topk, non-finite -> sentinel) with
# the tie rule "lower index wins"; key transform K:1132-1135.
# --------------------------------------------------------------------------


def rank_key(x: np.ndarray) -> np.ndarray:
    """fp32 -> uint32 order-preserving key; -0 == +0, NaN above +inf."""
    x = np.asarray(x, dtype=np.float32)
    b = x.view(np.uint32).copy()
    b[(b & 0x7FFFFFFF) == 0] = 0
    key = np.where(b & 0x80000000, ~b, b | 0x80000000).astype(np.uint32)
    key[np.isnan(x)] = 0xFFFFFFFF
    return key


def _key_finite(key: np.ndarray) -> np.ndarray:
    return (key > 0x007FFFFF) & (key < 0xFF800000)


def topk_select(scores: np.ndarray, seq_lens: np.ndarray, topk: int, sorted_: bool = False,
                pad: int = -1, page_table: np.ndarray | None = None) -> np.ndarray:
    """[B, slab] f32 -> [B, topk] int32, same contract as dsa_topk."""
    scores = np.asarray(scores, dtype=np.float32)
    B, slab = scores.shape
    out = np.full((B, topk), pad, dtype=np.int64)
    for b in range(B):
        n = int(max(0, min(int(seq_lens[b]), slab)))
        key = rank_key(scores[b, :n])
        order = np.lexsort((np.arange(n), ~key))[: min(topk, n)]   # key desc, idx asc
        fin = _key_finite(key[order])
        if sorted_:
            vals = np.where(fin, order, pad)
            out[b, : len(order)] = vals
        else:
            sel = np.sort(order[fin])
            if page_table is not None:
                sel = slot_of(page_table[b], sel)
            out[b, : len(sel)] = sel
    return out.astype(np.int32)


def select_topk_reference(logits: np.ndarray, topk: int) -> np.ndarray:
    """AC:66-91 on a [B,S,Skv] array: sentinel = Skv pad, selection order
    value-descending with lower index first on ties."""
    B, S, skv = logits.shape
    flat = logits.reshape(B * S, skv)
    idx = topk_select(flat, np.full(B * S, skv), topk, sorted_=True, pad=skv)
    return idx.reshape(B, S, topk).astype(np.int64)


# --------------------------------------------------------------------------
# (3) sparse MLA decode + (5) LSE merge.  AC:94-146, K:2950-2966, K:996-1045.
# --------------------------------------------------------------------------


def sparse_mla_decode(q: np.ndarray, rows: np.ndarray, idx: np.ndarray, sm_scale: float) -> np.ndarray:
    """q [B,H,576] (bf16 values as f32), rows [n,656], idx [B,K] KV slots.

    Softmax over the listed valid slots (0 <= slot < n); float64 math.
    """
    B, H, _ = q.shape
    n = rows.shape[0]
    out = np.zeros((B, H, LATENT_DIM), dtype=np.float64)
    for b in range(B):
        sl = np.asarray(idx[b], dtype=np.int64)
        sl = sl[(sl >= 0) & (sl < n)]
        if sl.size == 0:
            continue
        kv = dequant_latent_rows(rows[sl]).astype(np.float64)        # [m,576]
        s = (q[b].astype(np.float64) @ kv.T) * sm_scale              # [H,m]
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[b] = p @ kv[:, :LATENT_DIM]
    return out


def split_partials(q: np.ndarray, kv: np.ndarray, sm_scale: float, nsplit: int):
    """One head block, dequantised kv [m,576]: per-split (o_unnorm, m, l), natural log."""
    m_tot = kv.shape[0]
    kps = -(-m_tot // nsplit)
    parts = []
    for sp in range(nsplit):
        sub = kv[sp * kps:(sp + 1) * kps]
        if sub.shape[0] == 0:
            parts.append((np.zeros((q.shape[0], LATENT_DIM)), np.full(q.shape[0], -np.inf), np.zeros(q.shape[0])))
            continue
        s = (q @ sub.T) * sm_scale
        m = s.max(axis=1)
        p = np.exp(s - m[:, None])
        parts.append((p @ sub[:, :LATENT_DIM], m, p.sum(axis=1)))
    return parts


def lse_merge(parts) -> np.ndarray:
    """K:996-1045: m* = max m_s, l = sum l_s e^(m_s-m*), o = sum o_s e^(m_s-m*)/l."""
    ms = np.stack([p[1] for p in parts])            # [S,H]
    m = ms.max(axis=0)
    out = np.zeros_like(parts[0][0])
    l = np.zeros_like(m)
    for o_s, m_s, l_s in parts:
        wgt = np.where(np.isfinite(m_s), np.exp(np.where(np.isfinite(m_s), m_s - m, 0.0)), 0.0)
        out += o_s * wgt[:, None]
        l += l_s * wgt
    return np.where(l[:, None] > 0, out / np.where(l > 0, l, 1.0)[:, None], 0.0)


# --------------------------------------------------------------------------
# (4) MLI schedule.  ML:61-71 (_lagged_indexer_layers), ML:109-136.
# --------------------------------------------------------------------------


def lagged_indexer_layers(is_dsa: list[bool]) -> list[bool]:
    """Layer i emits an indexer iff layer i+1 is DSA (ML:61-71)."""
    n = len(is_dsa)
    return [(i + 1 < n and is_dsa[i + 1]) for i in range(n)]


def mli_attend_sources(produces: list[bool], first_attend: int = -1, depth: int = 1) -> list[int]:
    """For each layer, the index of the layer whose fresh selection it
    attends; ``first_attend`` (-1: an externally supplied set) is what the
    first layer attends.

    depth 1 (the certified lag, P:2942-2997): the most recent producer
    strictly before the layer; reuse layers therefore copy the FRESH set of
    the producer before them.

    depth k >= 2 (P:1835-1904 queue, P:3020-3100 dispatch), restated as the
    overlay's FIFO: a producer pushes its fresh set; when the queue already
    holds k entries it first pops the oldest and attends it, otherwise it
    attends the incoming carry.  The carry out of every layer is the set it
    ATTENDED, so reuse layers copy their producer's attended set.
    """
    if depth < 1:
        raise ValueError("depth must be >= 1")
    src = []
    if depth == 1:
        last = first_attend
        for p in produces:
            src.append(last)
            if p:
                last = len(src) - 1
        return src
    queue: list[int] = []
    carry = first_attend
    for i, p in enumerate(produces):
        if p:
            if len(queue) >= depth:
                att = queue.pop(0)
            else:
                att = carry
            queue.append(i)
            if len(queue) > depth:
                raise AssertionError("queue overflow")
        else:
            att = carry
        src.append(att)
        carry = att
    return src


def indexcache_produces(num_layers: int, freq: int | None = 1, pattern: str | None = None,
                        refresh_layers=None) -> list[bool]:
    """Which layers run their indexer (F) and which reuse (S), in the
    precedence of SGLang's dsa_layer_skips_topk as the overlay extends it
    (P:191-201): an explicit ``pattern`` string ("F"/"S" per layer, layers
    past its end are F); else ``refresh_layers`` (a list, or a comma string,
    of F layers, layer 0 always F); else uniform retention 1-in-``freq``.
    The uniform rule (layer % freq == 0, so layer 0 is F) is stock SGLang
    code that the reference does not vendor: parity unpinned for it."""
    if pattern is not None:
        return [not (i < len(pattern) and pattern[i] == "S") for i in range(num_layers)]
    if refresh_layers is not None:
        if isinstance(refresh_layers, str):
            refresh_layers = [int(x) for x in refresh_layers.split(",") if x.strip()]
        keep = set(refresh_layers) | {0}
        return [i in keep for i in range(num_layers)]
    f = 1 if freq is None else int(freq)
    if f < 1:
        raise ValueError("freq must be >= 1")
    return [i % f == 0 for i in range(num_layers)]
