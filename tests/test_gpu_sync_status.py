"""GPU: expired in-launch waits are reported per buffer (dsa_sync_status).

The fused layer launch hands data between its workgroups through bounded
waits (the select's list barrier and radix barriers, the attention's split
merge).  A wait that expires leaves wrong results, so every expiry is
counted in a status word of the group's own buffers -- the top-k scratch
row and the sparse-MLA workspace -- which dsa_sync_status sums without a
host synchronisation.  The test forces expiry from the host (the internal
spin limit set to 0: a wait gives up after its first unsatisfied poll, every
kernel still runs to its end), checks that the status flags the launch, then
restores the limit and checks that the same buffers give oracle-exact
results again with a zero status (the barriers re-arm after an expiry).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _lib():
    from lagged_indexer_dsa_amd import _lib
    return _lib.load()


@pytest.mark.parametrize("pattern", ["uniform", "window"])
def test_expired_waits_flag_the_buffers(dev, pattern):
    from lagged_indexer_dsa_amd import _lib as LL
    from lagged_indexer_dsa_amd import synthetic as S

    print(f"[sync-status] pattern={pattern}", flush=True)
    lib = _lib()
    lens = [40000]
    pt, npg = S.make_page_table(lens, seed=31, device=dev)
    L = S.make_decode_layer(lens, seed=32, device=dev, page_table=pt, num_pages=npg)
    if pattern == "window":  # the radix select's barriers too
        sc = L.index_k.view(npg, -1)[:, 8192:].view(torch.float32)
        ptc = pt.cpu()
        pos = torch.arange(10000, 13000)
        sc[ptc[0, pos // 64].long().to(dev), (pos % 64).to(dev)] *= 50.0
    att = S.random_selection(lens, 2048, pt, seed=33, device=dev)
    LL.sync_timeouts(reset=True)
    L.run(attend_idx=att)
    assert L.sync_status() == 0
    try:
        lib.dsa_internal_set_spin_limit(0)
        L.run(attend_idx=att)
        torch.cuda.synchronize()
    finally:
        lib.dsa_internal_set_spin_limit(-1)
    n = L.sync_status(clear=False)
    assert n > 0, "forced expiries were not reported in the layer's buffers"
    with pytest.raises(LL.DsaError):
        L.check_sync()  # raises, and clears the words
    assert L.sync_status() == 0
    assert LL.sync_timeouts(reset=True) >= n
    # the same buffers after the expiry: exact again, status 0
    for _ in range(2):
        L.next_idx.fill_(-7)
        L.run(attend_idx=att)
    L.check_sync()
    assert LL.sync_timeouts(reset=True) == 0
    sc = L.scores.cpu().numpy()
    ref = O.topk_select(sc, np.array(lens), 2048, page_table=pt.cpu().numpy())
    assert np.array_equal(L.next_idx.cpu().numpy(), ref)
    ref_out = O.sparse_mla_decode(L.q_bf16.float().cpu().numpy(), L.kv_pool.cpu().numpy(),
                                  att.cpu().numpy(), L.sm_scale)
    out = L.out.float().cpu().numpy()
    assert np.abs(out - ref_out).max() / np.abs(ref_out).max() < 2e-2
