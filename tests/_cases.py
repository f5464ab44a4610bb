"""Seeded input builders shared by the GPU parity tests (numpy -> device)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import dsa_oracle as O


def index_case(seed: int, lens: list[int], hidx: int = 64, extra_pages: int = 5,
               pt_stride: int | None = None):
    """Paged fp8 index-K cache + fp8 queries for rows of the given lengths."""
    rng = np.random.default_rng(seed)
    B = len(lens)
    n_pages = [(n + 63) // 64 for n in lens]
    num_pages = sum(n_pages) + extra_pages
    pt_stride = pt_stride or max(1, max(n_pages))
    perm = rng.permutation(num_pages).astype(np.int32)
    pt = np.full((B, pt_stride), -1, dtype=np.int32)
    pages = np.zeros((num_pages, O.INDEX_PAGE_BYTES), dtype=np.uint8)
    o = 0
    for b, n in enumerate(lens):
        pt[b, :n_pages[b]] = perm[o:o + n_pages[b]]
        o += n_pages[b]
        if n:
            c, s = O.quantize_rowwise(rng.standard_normal((n, 128)).astype(np.float32))
            for lp in range(n_pages[b]):
                g0, g1 = lp * 64, min(n, lp * 64 + 64)
                pg = pages[pt[b, lp]]
                pg[: (g1 - g0) * 128] = c[g0:g1].reshape(-1)
                sc = np.zeros(64, dtype=np.float32)
                sc[: g1 - g0] = s[g0:g1]
                pg[8192:] = sc.view(np.uint8)
    qc, sq = O.quantize_rowwise(rng.standard_normal((B, hidx, 128)).astype(np.float32))
    w = ((rng.standard_normal((B, hidx)) / np.sqrt(hidx)).astype(np.float32) * sq).astype(np.float32)
    return dict(q=qc, w=w, pages=pages, pt=pt, lens=np.array(lens, dtype=np.int32))


def to_dev(case: dict, dev) -> dict:
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in case.items()}


def latent_case(seed: int, n_rows: int, B: int, H: int, topk: int, valid_frac: float = 1.0):
    rng = np.random.default_rng(seed)
    lat = rng.standard_normal((n_rows, 576)).astype(np.float32)
    rows = O.pack_latent_rows(lat[:, :512], lat[:, 512:])
    q = O.bf16_rn(rng.standard_normal((B, H, 576)).astype(np.float32))
    idx = np.stack([rng.permutation(n_rows)[:topk] for _ in range(B)]).astype(np.int32)
    if valid_frac < 1.0:
        drop = rng.random(idx.shape) > valid_frac
        idx[drop] = np.where(rng.random(idx.shape) < 0.5, -1, n_rows + 3)[drop]
    return dict(rows=rows, q=q, idx=idx)


def q_bf16_dev(q: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(O.bf16_bits(q).view(np.int16)).view(torch.bfloat16).to(dev)


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| (the path's stated tolerance metric)."""
    den = float(np.abs(ref).max())
    return float(np.abs(got - ref).max() / (den if den > 0 else 1.0))


def corr_diff(a: np.ndarray, b: np.ndarray) -> float:
    """1 - 2<a,b>/(|a|^2+|b|^2), the reference's corr gate (K:2944-2947)."""
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    n = (a * a + b * b).sum()
    return 0.0 if n == 0 else float(1.0 - 2 * (a * b).sum() / n)
