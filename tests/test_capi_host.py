"""CPU-side checks of the C ABI library: it loads, exports every symbol the
public header declares, and rejects contract violations with the documented
codes before touching the device (no compute calls, no GPU needed).

The contract cases mirror the reference launcher's TORCH_CHECKs
(kernels/cuda_fused_sparse_splitk.py K:2399-2611).
"""

from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import REPO

HEADER = REPO / "include" / "dsa_mli.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(dsa_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    from lagged_indexer_dsa_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_the_hot_path():
    names = _declared_functions()
    for n in ["dsa_indexer_scan", "dsa_topk", "dsa_sparse_mla_decode", "dsa_decode_layer",
              "dsa_mli_graph_create", "dsa_mli_graph_launch", "dsa_mli_graph_destroy",
              "dsa_mli_run_eager", "dsa_mli_run_eager_depth", "dsa_mli_graph_create_depth",
              "dsa_sparse_mla_workspace_bytes", "dsa_last_error"]:
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    from lagged_indexer_dsa_amd import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for name in _declared_functions():
        assert name in exported, name
        assert hasattr(lib, name)
    assert set(_lib.SIGNATURES) == set(_declared_functions())


def test_version(lib):
    assert b"gfx950" in lib.dsa_version()


def _scan(lib, **kw):
    a = dict(q=16, w=16, k=16, pages=4, pt=16, seq=16, sc=16, B=1, H=64, pts=4, slab=256)
    a.update(kw)
    return lib.dsa_indexer_scan(a["q"], a["w"], a["k"], a["pages"], a["pt"], a["seq"], a["sc"],
                                a["B"], a["H"], a["pts"], a["slab"], None)


def test_scan_contract(lib):
    from lagged_indexer_dsa_amd._lib import DSA_ERR_INVALID_ARG, DSA_ERR_UNSUPPORTED

    assert _scan(lib, q=None) == DSA_ERR_INVALID_ARG
    assert b"null" in lib.dsa_last_error()
    assert _scan(lib, H=40) == DSA_ERR_UNSUPPORTED
    assert _scan(lib, H=128) == DSA_ERR_UNSUPPORTED
    assert _scan(lib, B=0) == DSA_ERR_INVALID_ARG
    assert _scan(lib, pages=0) == DSA_ERR_INVALID_ARG
    assert _scan(lib, q=17) == DSA_ERR_INVALID_ARG   # misaligned


def test_topk_contract(lib):
    from lagged_indexer_dsa_amd._lib import DSA_ERR_INVALID_ARG, DSA_ERR_UNSUPPORTED

    f = lib.dsa_topk
    assert f(16, 16, None, 0, 16, 16, 1, 1000, 0, 0, -1, None) == DSA_ERR_INVALID_ARG
    assert f(16, 16, None, 0, 16, 16, 1, 1000, 9000, 0, -1, None) == DSA_ERR_UNSUPPORTED
    assert f(16, 16, None, 0, 16, 16, 1, 1000, 4097, 1, -1, None) == DSA_ERR_UNSUPPORTED
    assert f(16, 16, None, 0, 16, 16, 1, 300000, 2048, 0, -1, None) == DSA_ERR_UNSUPPORTED
    assert f(16, 16, 16, 2, 16, 16, 1, 1000, 2048, 0, -1, None) == DSA_ERR_INVALID_ARG  # pt too short
    assert f(16, 16, 16, 16, 16, 16, 1, 1000, 2048, 1, -1, None) == DSA_ERR_INVALID_ARG  # slots + sorted
    assert f(16, 16, None, 0, 16, 16, 1, 1000, 16, 3, -1, None) == DSA_ERR_INVALID_ARG
    assert f(16, 16, None, 0, None, 16, 1, 1000, 16, 0, -1, None) == DSA_ERR_INVALID_ARG  # no scratch
    sb = lib.dsa_topk_scratch_bytes
    assert sb(1, 131072) >= 4 * (4096 + 131072 // 32 + 2 * 4096)
    assert sb(2, 1000) == 2 * sb(1, 1000)
    assert sb(1, 300000) == 0


def test_mla_contract_and_workspace(lib):
    from lagged_indexer_dsa_amd._lib import DSA_ERR_INVALID_ARG, DSA_ERR_UNSUPPORTED

    f = lib.dsa_sparse_mla_decode
    assert f(16, 16, 10, 16, 16, 16, 1, 24, 2048, 0, 0.04, None) == DSA_ERR_UNSUPPORTED
    assert f(16, 16, 10, 16, 16, 16, 1, 16, 2048, 129, 0.04, None) == DSA_ERR_UNSUPPORTED
    assert f(16, 16, 0, 16, 16, 16, 1, 16, 2048, 0, 0.04, None) == DSA_ERR_INVALID_ARG
    assert f(None, 16, 10, 16, 16, 16, 1, 16, 2048, 0, 0.04, None) == DSA_ERR_INVALID_ARG
    ws = lib.dsa_sparse_mla_workspace_bytes
    sync = (16 + 1 + 8) * 64                                     # one group barrier, words
    assert ws(1, 16, 32) == (sync + 32 * 16 * 514) * 4           # barrier + partials
    assert ws(2, 32, 8) == (4 * sync + 2 * 2 * 8 * 16 * 514) * 4
    assert ws(1, 16, 0) == ws(1, 16, 128)
    assert ws(1, 15, 8) == 0


def test_mli_contract(lib):
    from lagged_indexer_dsa_amd._lib import DSA_ERR_INVALID_ARG, LayerArgs

    arr = (LayerArgs * 1)()
    h = ctypes.c_void_p()
    # attention without any selection to attend
    arr[0].q_bf16 = 16
    arr[0].kv_pool = 16
    arr[0].kv_rows = 10
    arr[0].workspace = 16
    arr[0].out_bf16 = 16
    arr[0].B, arr[0].H, arr[0].topk = 1, 16, 2048
    assert lib.dsa_mli_graph_create(arr, 1, None, ctypes.byref(h)) == DSA_ERR_INVALID_ARG
    assert lib.dsa_mli_run_eager(arr, 1, 16) == DSA_ERR_INVALID_ARG
    assert lib.dsa_mli_graph_create(arr, 0, None, ctypes.byref(h)) == DSA_ERR_INVALID_ARG
    assert lib.dsa_mli_graph_destroy(None) == 0
    # lag depth outside [1, 64]
    arr[0].attend_idx = 16
    for k in (0, -1, 65):
        assert lib.dsa_mli_run_eager_depth(arr, 1, k, 16) == DSA_ERR_INVALID_ARG
        assert b"lag depth" in lib.dsa_last_error()
        assert lib.dsa_mli_graph_create_depth(arr, 1, k, 16, ctypes.byref(h)) == DSA_ERR_INVALID_ARG
    assert not h.value


def test_operand_prep_contract(lib):
    """The decode-step quantizers reject bad arguments before any launch."""
    from lagged_indexer_dsa_amd._lib import DSA_ERR_INVALID_ARG, DSA_OK

    assert lib.dsa_quantize_index_query(None, 16, 16, 16, 1, 64, None) == DSA_ERR_INVALID_ARG
    assert lib.dsa_quantize_index_query(16, 16, 16, 16, 0, 64, None) == DSA_ERR_INVALID_ARG
    assert lib.dsa_append_index_keys(16, 16, 16, -1, 16, 4, 16, 4, None) == DSA_ERR_INVALID_ARG
    assert lib.dsa_append_index_keys(None, None, None, 0, None, 0, None, 0, None) == DSA_OK  # nothing to do
    assert lib.dsa_append_index_keys(16, None, 16, 2, 16, 4, 16, 4, None) == DSA_ERR_INVALID_ARG
    assert lib.dsa_append_index_keys(16, 16, 16, 2, 16, 0, 16, 4, None) == DSA_ERR_INVALID_ARG
    assert lib.dsa_append_latent_rows(16, None, 2, 16, 8, None) == DSA_ERR_INVALID_ARG
    assert lib.dsa_append_latent_rows(16, 16, 2, 16, 0, None) == DSA_ERR_INVALID_ARG
    assert lib.dsa_append_latent_rows(None, None, 0, None, 0, None) == DSA_OK


def test_sync_status_contract(lib):
    from lagged_indexer_dsa_amd._lib import DSA_ERR_INVALID_ARG

    f = lib.dsa_sync_status
    assert f(16, 1, 1000, 16, 1, 16, None, 1, None) == DSA_ERR_INVALID_ARG   # no status word
    assert f(16, 0, 1000, None, 0, 0, 16, 1, None) == DSA_ERR_INVALID_ARG    # B_scan < 1
    assert f(16, 1, 300000, None, 0, 0, 16, 1, None) == DSA_ERR_INVALID_ARG  # slab too long
    assert f(None, 0, 0, 16, 1, 24, 16, 1, None) == DSA_ERR_INVALID_ARG      # H not a multiple of 16
    assert b"dsa_sync_status" in lib.dsa_last_error()


def test_dense_layer_key_count_guard(lib):
    """A dense layer's key capacity pt_stride*64 must stay <= 2^30 (the same
    guard as dsa_dense_mla_decode), checked before any launch."""
    from lagged_indexer_dsa_amd._lib import DSA_ERR_UNSUPPORTED, LayerArgs

    a = LayerArgs()
    a.q_bf16 = a.kv_pool = a.workspace = a.out_bf16 = a.page_table = a.seq_lens = 16
    a.kv_rows = 10
    a.B, a.H, a.topk = 1, 16, 2048
    a.dense = 1
    a.pt_stride = (1 << 24) + 1
    assert lib.dsa_decode_layer(ctypes.byref(a), None) == DSA_ERR_UNSUPPORTED
    assert b"2^30" in lib.dsa_last_error()


def test_layer_args_size_matches_binding(lib):
    from lagged_indexer_dsa_amd._lib import LayerArgs

    assert lib.dsa_layer_args_bytes() == ctypes.sizeof(LayerArgs)
