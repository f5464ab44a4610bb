"""ctypes binding of libdsa_mli.so (declarations in include/dsa_mli.h).

The library is the only compute path of this package: if it is missing or
cannot be loaded, every op raises -- there is no CPU fallback.  torch is
imported first so that the library binds to the HIP runtime torch already
loaded (one runtime per process).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before ours)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libdsa_mli.so"

DSA_OK = 0
DSA_ERR_INVALID_ARG = -1
DSA_ERR_UNSUPPORTED = -2
DSA_ERR_HIP = -3
DSA_TOPK_POSITION_ORDER = 0
DSA_TOPK_SORTED = 1

PAGE_TOKENS = 64
INDEX_DIM = 128
INDEX_PAGE_BYTES = 8448
LATENT_DIM = 512
ROPE_DIM = 64
QK_DIM = 576
LATENT_ROW_BYTES = 656
TOPK_MAX_CTX = 262144

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class DsaError(RuntimeError):
    """A C-ABI call returned a negative status (mirrors TORCH_CHECK -> RuntimeError)."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(f"[dsa {code}] {message}")
        self.code = code


class LayerArgs(ctypes.Structure):
    """Mirror of ``dsa_layer_args``."""

    _fields_ = [
        ("q_fp8", _vp), ("w", _vp), ("index_k", _vp), ("num_idx_pages", _i64),
        ("scores", _vp), ("topk_scratch", _vp), ("next_idx", _vp),
        ("q_bf16", _vp), ("kv_pool", _vp), ("kv_rows", _i64), ("attend_idx", _vp),
        ("workspace", _vp), ("out_bf16", _vp),
        ("page_table", _vp), ("seq_lens", _vp),
        ("B", _i32), ("Hidx", _i32), ("H", _i32), ("topk", _i32), ("nsplit", _i32),
        ("pt_stride", _i32), ("slab_stride", _i32),
        ("sm_scale", _f32),
        ("dense", _i32),
    ]


_LIB: ctypes.CDLL | None = None

# (name, restype, argtypes) for every symbol of include/dsa_mli.h
SIGNATURES = {
    "dsa_last_error": (ctypes.c_char_p, []),
    "dsa_version": (ctypes.c_char_p, []),
    "dsa_layer_args_bytes": (ctypes.c_size_t, []),
    "dsa_sync_timeouts": (_i32, [_i32]),
    "dsa_sync_status": (_i32, [_vp, _i32, _i32, _vp, _i32, _i32, _vp, _i32, _vp]),
    "dsa_indexer_scan": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "dsa_topk_scratch_bytes": (ctypes.c_size_t, [_i32, _i32]),
    "dsa_topk": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "dsa_sparse_mla_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32]),
    "dsa_sparse_mla_decode": (_i32, [_vp, _vp, _i64, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _vp]),
    "dsa_dense_mla_decode": (_i32, [_vp, _vp, _i64, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _f32, _vp]),
    "dsa_sparse_mla_decode_noalloc": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _vp]),
    "dsa_decode_layer": (_i32, [ctypes.POINTER(LayerArgs), _vp]),
    "dsa_mli_graph_create": (_i32, [ctypes.POINTER(LayerArgs), _i32, _vp, ctypes.POINTER(_vp)]),
    "dsa_mli_graph_launch": (_i32, [_vp, _vp]),
    "dsa_mli_graph_destroy": (_i32, [_vp]),
    "dsa_mli_run_eager": (_i32, [ctypes.POINTER(LayerArgs), _i32, _vp]),
    "dsa_mli_graph_create_depth": (_i32, [ctypes.POINTER(LayerArgs), _i32, _i32, _vp, ctypes.POINTER(_vp)]),
    "dsa_mli_run_eager_depth": (_i32, [ctypes.POINTER(LayerArgs), _i32, _i32, _vp]),
    "dsa_quantize_index_query": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "dsa_append_index_keys": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _i64, _vp]),
    "dsa_append_latent_rows": (_i32, [_vp, _vp, _i32, _vp, _i64, _vp]),
}


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = Path(path) if path else Path(os.environ.get("DSA_MLI_LIB") or LIB_PATH)
    if not p.exists():
        raise RuntimeError(
            f"HIP library {p} is not built: run `python -m lagged_indexer_dsa_amd._build` "
            "(or __graft_entry__.build()); this package has no CPU fallback")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.dsa_layer_args_bytes() != ctypes.sizeof(LayerArgs):
        raise RuntimeError(f"{p}: dsa_layer_args is {lib.dsa_layer_args_bytes()} bytes in the library, "
                           f"{ctypes.sizeof(LayerArgs)} in this binding (header mismatch)")
    lib.dsa_internal_set_scan_variant.restype = _i32
    lib.dsa_internal_set_scan_variant.argtypes = [_i32]
    lib.dsa_internal_set_coop_select.restype = _i32
    lib.dsa_internal_set_coop_select.argtypes = [_i32]
    lib.dsa_internal_set_flat_scan.restype = _i32
    lib.dsa_internal_set_flat_scan.argtypes = [_i32]
    lib.dsa_internal_group_wait_timeouts.restype = _i32
    lib.dsa_internal_group_wait_timeouts.argtypes = [_i32]
    lib.dsa_internal_set_spin_limit.restype = _i32
    lib.dsa_internal_set_spin_limit.argtypes = [_i32]
    _LIB = lib
    return lib


def check(rc: int) -> None:
    if rc != DSA_OK:
        msg = load().dsa_last_error().decode(errors="replace")
        raise DsaError(rc, msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def sync_timeouts(reset: bool = False) -> int:
    """In-launch group waits that expired since load or the last reset
    (dsa_sync_timeouts); nonzero means some launch's results are wrong."""
    n = load().dsa_sync_timeouts(1 if reset else 0)
    if n < 0:
        raise DsaError(DSA_ERR_HIP, "dsa_sync_timeouts: counter unreadable")
    return n
