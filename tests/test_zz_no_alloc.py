"""GPU: the allocation-free sparse MLA entry point (dsa_sparse_mla_decode_noalloc).

It must give what dsa_sparse_mla_decode gives with a caller workspace at the
same split count, bit for bit, on consecutive calls that share the library's
static scratch -- the second one smaller than the first, and a third back at
the first shape (its barriers must still be armed) -- and it must reject a
shape whose partials exceed the static limit before launching.  Called
through the C ABI.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import _cases as C

pytestmark = pytest.mark.gpu


def _lib():
    from lagged_indexer_dsa_amd import _lib
    return _lib


def _run(fn_name, q, pool, idx, B, H, topk, nsplit, ws=None):
    L = _lib()
    lib = L.load()
    out = torch.full((B, H, 512), 7.0, dtype=torch.bfloat16, device=q.device)
    s = torch.cuda.current_stream().cuda_stream
    sm = 576 ** -0.5
    if ws is None:
        rc = lib.dsa_sparse_mla_decode_noalloc(q.data_ptr(), pool.data_ptr(), pool.shape[0], idx.data_ptr(),
                                               out.data_ptr(), B, H, topk, nsplit, ctypes.c_float(sm), s)
    else:
        rc = lib.dsa_sparse_mla_decode(q.data_ptr(), pool.data_ptr(), pool.shape[0], idx.data_ptr(),
                                       ws.data_ptr(), out.data_ptr(), B, H, topk, nsplit, ctypes.c_float(sm), s)
    L.check(rc)
    torch.cuda.synchronize()
    return out


def _case(dev, seed, n_rows, B, H, topk):
    c = C.latent_case(seed, n_rows, B, H, topk, valid_frac=0.97)
    pool = torch.from_numpy(c["rows"]).to(dev)
    q = C.q_bf16_dev(c["q"], dev)
    idx = torch.from_numpy(c["idx"]).to(dev)
    return q, pool, idx


@pytest.mark.parametrize("nsplit", [0, 16])
def test_noalloc_equals_workspace_entry(dev, nsplit):
    L = _lib()
    lib = L.load()
    print(f"[no-alloc] nsplit={nsplit}", flush=True)
    L.sync_timeouts(reset=True)
    shapes = [(21, 6000, 4, 32, 2048), (22, 3000, 1, 16, 1000), (23, 6000, 4, 32, 2048)]
    for seed, n_rows, B, H, topk in shapes:
        q, pool, idx = _case(dev, seed, n_rows, B, H, topk)
        ws = torch.zeros(lib.dsa_sparse_mla_workspace_bytes(B, H, nsplit), dtype=torch.uint8, device=dev)
        ref = _run("ws", q, pool, idx, B, H, topk, nsplit, ws=ws)
        for rep in range(2):
            got = _run("noalloc", q, pool, idx, B, H, topk, nsplit)
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"{(B, H, topk)} rep {rep}"
    assert L.sync_timeouts() == 0


def test_noalloc_rejects_oversize(dev):
    L = _lib()
    lib = L.load()
    print("[no-alloc] oversize", flush=True)
    q, pool, idx = _case(dev, 24, 3000, 2, 16, 1024)
    big_B = 600  # 600 (row, head group) barriers: above the static 512
    s = torch.cuda.current_stream().cuda_stream
    out = torch.empty(1, dtype=torch.bfloat16, device=dev)
    rc = lib.dsa_sparse_mla_decode_noalloc(q.data_ptr(), pool.data_ptr(), pool.shape[0], idx.data_ptr(),
                                           out.data_ptr(), big_B, 16, 1024, 1, ctypes.c_float(0.04), s)
    assert rc == L.DSA_ERR_UNSUPPORTED
    # partials above 16 MiB: 4 rows x 8 head groups x 128 splits
    rc = lib.dsa_sparse_mla_decode_noalloc(q.data_ptr(), pool.data_ptr(), pool.shape[0], idx.data_ptr(),
                                           out.data_ptr(), 4, 128, 1024, 128, ctypes.c_float(0.04), s)
    assert rc == L.DSA_ERR_UNSUPPORTED
    torch.cuda.synchronize()
