"""GPU: decode-step operand preparation (quant.hip) against the oracle.

Bit-exact bar: the codes, scales and packed rows equal the oracle's
quantize_rowwise / pack_latent_rows (the reference harness rule,
K:2969-2974) on the same bf16 inputs, and the folded weights equal
w * scale in fp32.  The e4m3 encoder sees every code value and every
midpoint between neighbours exactly (a row whose amax is 448 has scale 1).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _bf16(x: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(O.bf16_bits(O.bf16_rn(x)).view(np.int16)).view(torch.bfloat16).to(dev)


def _f32_of_bf16(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def _encoder_rows() -> np.ndarray:
    """Rows of 128: 448 first (scale = 1), then e4m3 values and midpoints."""
    pos = O.e4m3_decode(np.arange(0x7F, dtype=np.uint8))            # +0 .. 448 (0x7f is NaN)
    mids = (pos[:-1] + pos[1:]) / 2
    vals = np.concatenate([pos, mids, -pos, -mids, [1e-4, -1e-4, 0.0021, 0.0019, 447.9, 300.0]])
    vals = vals.astype(np.float32)
    rows = []
    for i in range(0, len(vals), 127):
        chunk = vals[i:i + 127]
        rows.append(np.concatenate([[448.0], chunk, np.zeros(127 - len(chunk))]).astype(np.float32))
    return np.stack(rows)


def test_quantize_index_query_bit_exact(dev):
    from lagged_indexer_dsa_amd import ops

    print("[prep] index query", flush=True)
    rng = np.random.default_rng(5)
    enc = _encoder_rows()                                             # [r, 128]
    q = rng.standard_normal((3, 64, 128)).astype(np.float32)
    q[0, 1] = 0.0                                                     # all-zero row: scale 1e-6/448
    q[1, 2] *= 1e-5                                                   # tiny values: subnormal codes
    q[2, 3] *= 300.0
    q[2, :enc.shape[0]] = enc
    q = O.bf16_rn(q)
    w = (rng.standard_normal((3, 64)) / 8).astype(np.float32)
    codes, wf = ops.quantize_index_query(_bf16(q, dev), torch.from_numpy(w).to(dev))
    torch.cuda.synchronize()
    ref_c, ref_s = O.quantize_rowwise(q)
    assert np.array_equal(codes.cpu().numpy(), ref_c)
    assert np.array_equal(wf.cpu().numpy(), (w * ref_s).astype(np.float32))


def test_append_index_keys_bit_exact(dev):
    from lagged_indexer_dsa_amd import ops

    print("[prep] index keys", flush=True)
    rng = np.random.default_rng(6)
    lens = [300, 130]
    npg = 8
    pt = np.full((2, 6), -1, dtype=np.int32)
    perm = rng.permutation(npg).astype(np.int32)
    pt[0, :5], pt[1, :3] = perm[:5], perm[5:8]
    n = 200
    rows = rng.integers(0, 2, n).astype(np.int32)
    pos = np.array([rng.integers(0, lens[r]) for r in rows], dtype=np.int32)
    _, first = np.unique(np.stack([rows, pos], 1), axis=0, return_index=True)   # one write per token
    rows, pos = rows[np.sort(first)], pos[np.sort(first)]
    n = len(rows)
    keys = O.bf16_rn((rng.standard_normal((n, 128)) * rng.uniform(0.01, 50, (n, 1))).astype(np.float32))
    keys[0] = 0.0
    pool = torch.full((npg, 8448), 0xAB, dtype=torch.uint8, device=dev)
    ops.append_index_keys(pool, torch.from_numpy(pt).to(dev), torch.from_numpy(rows).to(dev),
                          torch.from_numpy(pos).to(dev), _bf16(keys, dev))
    torch.cuda.synchronize()
    ref = np.full((npg, 8448), 0xAB, dtype=np.uint8)
    codes, scale = O.quantize_rowwise(keys)
    for i in range(n):
        p, s = pt[rows[i], pos[i] // 64], pos[i] % 64
        ref[p, s * 128:(s + 1) * 128] = codes[i]
        ref[p, 8192 + 4 * s:8192 + 4 * s + 4] = np.array([scale[i]], dtype=np.float32).view(np.uint8)
    assert np.array_equal(pool.cpu().numpy(), ref)


def test_append_latent_rows_bit_exact(dev):
    from lagged_indexer_dsa_amd import ops

    print("[prep] latent rows", flush=True)
    rng = np.random.default_rng(7)
    n, kv_rows = 257, 600
    lat = O.bf16_rn((rng.standard_normal((n, 576)) * rng.uniform(0.001, 20, (n, 1))).astype(np.float32))
    lat[3, :128] = 0.0                                               # a zero group
    lat[4, :128] = _encoder_rows()[0]                                # encoder values
    slots = rng.permutation(kv_rows)[:n].astype(np.int32)
    slots[5] = kv_rows + 7                                           # out of range: skipped
    slots[6] = -1
    pool = torch.full((kv_rows, 656), 0x5A, dtype=torch.uint8, device=dev)
    ops.append_latent_rows(pool, torch.from_numpy(slots).to(dev), _bf16(lat, dev))
    torch.cuda.synchronize()
    ref = np.full((kv_rows, 656), 0x5A, dtype=np.uint8)
    packed = O.pack_latent_rows(lat[:, :512], lat[:, 512:])
    for i in range(n):
        if 0 <= slots[i] < kv_rows:
            ref[slots[i]] = packed[i]
    assert np.array_equal(pool.cpu().numpy(), ref)


def test_layer_built_by_the_append_kernels_equals_fixture_layer(dev):
    """Caches and the query prepared by the HIP kernels give the same decode
    layer (scores, selection, output) as the torch fixture builders."""
    from lagged_indexer_dsa_amd import formats as F
    from lagged_indexer_dsa_amd import ops
    from lagged_indexer_dsa_amd import synthetic as S

    print("[prep] layer from appended caches", flush=True)
    lens = [3000, 2200]
    pt, num_pages = S.make_page_table(lens, seed=21, device=dev)
    ref = S.make_decode_layer(lens, seed=22, device=dev, page_table=pt, num_pages=num_pages)
    g = torch.Generator(device=dev).manual_seed(23)
    # the same tensors again, this time through the HIP kernels
    idx_pool = F.new_index_pool(num_pages, dev)
    kv_pool = F.new_latent_pool(num_pages, dev)
    for b, n in enumerate(lens):
        keys = torch.randn(n, 128, generator=g, device=dev).to(torch.bfloat16)
        lat = torch.randn(n, 576, generator=g, device=dev).to(torch.bfloat16)
        rows = torch.full((n,), b, dtype=torch.int32, device=dev)
        pos = torch.arange(n, dtype=torch.int32, device=dev)
        ops.append_index_keys(idx_pool, pt, rows, pos, keys)
        slots = F.positions_to_slots(pt[b:b + 1].cpu(), pos.cpu()[None].long())[0].to(dev)
        ops.append_latent_rows(kv_pool, slots, lat)
        # the fixture path on the same bf16 values
        codes, sc = F.quantize_rowwise(keys.float())
        F.write_index_keys(ref.index_k, pt[b].cpu(), codes, sc)
        F.write_latent_rows(ref.kv_pool, pt[b].cpu(), F.pack_latent_rows(lat[:, :512].float(), lat[:, 512:]))
    torch.cuda.synchronize()
    got_i, ref_i = idx_pool.cpu().numpy(), ref.index_k.cpu().numpy()
    bad = np.argwhere(got_i != ref_i)
    assert bad.size == 0, (f"{len(bad)} index-pool bytes differ, first at (page, byte) {bad[:4].tolist()}: "
                           f"kernel {got_i[tuple(bad[0])]} fixture {ref_i[tuple(bad[0])]}")
    assert torch.equal(kv_pool, ref.kv_pool)
    q = torch.randn(len(lens), 64, 128, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(len(lens), 64, generator=g, device=dev) / 8
    q8, wf = ops.quantize_index_query(q, w)
    rq8, rwf = F.quantize_index_query(q.float(), w)
    torch.cuda.synchronize()
    assert torch.equal(q8, rq8)
    assert torch.equal(wf, rwf)
