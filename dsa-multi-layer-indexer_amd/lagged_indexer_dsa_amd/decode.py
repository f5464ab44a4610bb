"""Paged decode layers and the MLI lag schedule on the GPU.

:class:`DecodeLayer` owns the device buffers of one DSA decode layer for a
batch of B requests (one decode row each): the indexer query/weights, the
paged fp8 index-K cache, the fp8 latent KV pool, the attention query, the
score slab, the selection and the attention output.  :class:`MLISchedule`
runs a stack of layers under the Multi-layer Indexer lag -- layer i attends
the selection of the last earlier indexing layer while layer i's own
indexer scan runs in the same launch (role-decoupled workgroups) -- eagerly
or as one captured hipGraph (C ABI ``dsa_mli_graph_*``).

Reference: DSAModel.forward LAGGED_FUSED (model.py:109-136),
DSALayer.fused_attention_and_indices (dsa_layer.py:173-192), the serving
side-stream fork/join (sglang overlay patch P:1774-1833, P:2942-2997) and
IndexCache reuse (P:1835-1904).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import LayerArgs
from .config import AttentionType, ColdStartPolicy, DSAConfig
from .ops import sparse_mla_workspace, topk_scratch


@dataclass
class DecodeLayer:
    """Device buffers of one decode layer (all contiguous, on one GPU)."""

    q_fp8: torch.Tensor | None       # [B, Hidx, 128] uint8 (None: no indexer)
    w: torch.Tensor | None           # [B, Hidx] f32, q-scale folded
    index_k: torch.Tensor | None     # [P, 8448] uint8
    q_bf16: torch.Tensor             # [B, H, 576] bf16
    kv_pool: torch.Tensor            # [P*64, 656] uint8
    page_table: torch.Tensor         # [B, pt_stride] int32
    seq_lens: torch.Tensor           # [B] int32
    slab_stride: int
    topk: int = 2048
    nsplit: int = 0
    sm_scale: float = 576 ** -0.5
    dense: bool = False               # attention over the whole prefix (full layer / DENSE cold start)

    def __post_init__(self) -> None:
        B = self.q_bf16.shape[0]
        dev = self.q_bf16.device
        self.scores = torch.empty(B, self.slab_stride, dtype=torch.float32, device=dev)
        self.topk_scratch = topk_scratch(B, self.slab_stride, dev)
        self.next_idx = torch.full((B, self.topk), -1, dtype=torch.int32, device=dev)
        self.workspace = sparse_mla_workspace(B, self.q_bf16.shape[1], self.nsplit, dev)
        self.out = torch.zeros(B, self.q_bf16.shape[1], 512, dtype=torch.bfloat16, device=dev)

    @property
    def has_indexer(self) -> bool:
        return self.q_fp8 is not None

    def args(self, attend_idx: torch.Tensor | None = None, indexer: bool = True,
             attention: bool = True) -> LayerArgs:
        """C-ABI argument block.  attend_idx=None: the schedule decides."""
        a = LayerArgs()
        B, H, _ = self.q_bf16.shape
        if indexer and self.has_indexer:
            a.q_fp8 = self.q_fp8.data_ptr()
            a.w = self.w.data_ptr()
            a.index_k = self.index_k.data_ptr()
            a.num_idx_pages = self.index_k.shape[0]
            a.Hidx = self.q_fp8.shape[1]
        a.scores = self.scores.data_ptr()
        a.topk_scratch = self.topk_scratch.data_ptr()
        a.next_idx = self.next_idx.data_ptr()
        if attention:
            a.q_bf16 = self.q_bf16.data_ptr()
            a.kv_pool = self.kv_pool.data_ptr()
            a.kv_rows = self.kv_pool.shape[0]
            a.workspace = self.workspace.data_ptr()
            a.out_bf16 = self.out.data_ptr()
        a.attend_idx = None if attend_idx is None else attend_idx.data_ptr()
        a.page_table = self.page_table.data_ptr()
        a.seq_lens = self.seq_lens.data_ptr()
        a.B = B
        a.H = H
        a.topk = self.topk
        a.nsplit = self.nsplit
        a.pt_stride = self.page_table.shape[1]
        a.slab_stride = self.slab_stride
        a.sm_scale = self.sm_scale
        a.dense = 1 if (self.dense and attention) else 0
        return a

    def sync_status(self, clear: bool = True) -> int:
        """Expired in-launch waits recorded in this layer's buffers (its
        rows' selects and its attention's split merges) since the last
        clear (dsa_sync_status); synchronises.  Nonzero means a launch of
        this layer broke the co-residency assumption and its results are
        wrong."""
        if not hasattr(self, "_status"):
            self._status = torch.zeros(1, dtype=torch.int32, device=self.q_bf16.device)
        B, H, _ = self.q_bf16.shape
        _lib.call("dsa_sync_status", self.topk_scratch.data_ptr(), B, self.slab_stride,
                  self.workspace.data_ptr(), B, H, self._status.data_ptr(), 1 if clear else 0,
                  torch.cuda.current_stream().cuda_stream)
        return int(self._status.item())

    def check_sync(self) -> None:
        """Raise if any in-launch wait of this layer's launches expired."""
        n = self.sync_status(clear=True)
        if n:
            raise _lib.DsaError(_lib.DSA_ERR_HIP, f"{n} in-launch waits expired: this layer's results are invalid")

    def run(self, attend_idx: torch.Tensor | None = None) -> None:
        """One layer on the current stream: indexer -> next_idx, attention
        over attend_idx (lagged) or over next_idx (same-layer, baseline DSA),
        or over the whole prefix when the layer is dense."""
        a = self.args(attend_idx)
        _lib.call("dsa_decode_layer", ctypes.byref(a), torch.cuda.current_stream().cuda_stream)


@dataclass(frozen=True)
class LayerPlan:
    """What one layer does in a decode step under the MLI lag (DSAModel.forward
    LAGGED_FUSED, model.py:51-71, 104-136): ``dense`` -- it attends its whole
    prefix (a FULL layer, or layer 0 as a DSA layer under the DENSE cold
    start); ``indexer`` -- it runs an indexer (iff the next layer is DSA: the
    lag moves production one layer earlier, so a dense prefix's last FULL
    layer gains the boundary indexer and the final layer runs none; plus
    layer 0 under the EAGER cold start, for its own attention);
    ``attends_own`` -- layer 0 under EAGER attends its own fresh selection."""

    dense: bool
    indexer: bool
    attends_own: bool = False


def lagged_layer_plan(config: DSAConfig | tuple[AttentionType, ...] | list[AttentionType],
                      cold_start: ColdStartPolicy = ColdStartPolicy.DENSE) -> list[LayerPlan]:
    """The per-layer plan of ``config.resolved_attention_types`` (or the
    types given directly) under the lag and the cold-start policy."""
    types = config.resolved_attention_types if isinstance(config, DSAConfig) else tuple(config)
    cold_start = ColdStartPolicy(cold_start)
    is_dsa = [AttentionType(t) is AttentionType.DSA for t in types]
    n = len(is_dsa)
    plan = []
    for i in range(n):
        produce = i + 1 < n and is_dsa[i + 1]
        if not is_dsa[i]:
            plan.append(LayerPlan(dense=True, indexer=produce))
        elif i == 0 and cold_start is ColdStartPolicy.DENSE:
            plan.append(LayerPlan(dense=True, indexer=produce))
        elif i == 0:  # EAGER: the layer's own indexer feeds its own attention
            plan.append(LayerPlan(dense=False, indexer=True, attends_own=True))
        else:
            plan.append(LayerPlan(dense=False, indexer=produce))
    return plan


def _arg_array(args: list[LayerArgs]):
    arr = (LayerArgs * len(args))()
    for i, a in enumerate(args):
        arr[i] = a
    return arr


class MLISchedule:
    """A stack of decode layers under the MLI lag.

    ``first_attend`` is the selection layer 0 attends (the previous step's or
    a cold-start set).  Layers whose indexer is disabled (IndexCache reuse)
    attend the most recent earlier selection.
    """

    def __init__(self, layers: list[DecodeLayer], first_attend: torch.Tensor,
                 indexer: bool = True, attention: bool = True,
                 attend_all_first: bool = False, lag_depth: int = 1) -> None:
        """indexer/attention=False drop that half of every layer (timing of
        the other half alone); attend_all_first makes every layer attend
        ``first_attend`` (attention-only timing with the same gather volume).
        lag_depth k (index_reuse_lag_depth, P:4388-4431): indexer layer R_n
        attends R_{n-k}'s selection once n >= k, else the carried set; pass
        layers[0].next_idx as first_attend for the reference's cold start."""
        if not 1 <= int(lag_depth) <= 64:
            raise ValueError(f"lag_depth must be in [1, 64], got {lag_depth}")
        self.lag_depth = int(lag_depth)
        self.layers = layers
        self.first_attend = first_attend
        self._args = []
        for i, layer in enumerate(layers):
            att = first_attend if (i == 0 or attend_all_first) else None
            self._args.append(layer.args(att, indexer=indexer, attention=attention))
        self._arr = _arg_array(self._args)
        self._graph = None

    @classmethod
    def for_config(cls, config: DSAConfig | tuple[AttentionType, ...], make_layer, first_attend=None,
                   cold_start: ColdStartPolicy = ColdStartPolicy.DENSE, lag_depth: int = 1) -> "MLISchedule":
        """Build a step for a DSA stack: ``make_layer(i, indexer)`` returns
        layer i's :class:`DecodeLayer` (with indexer operands iff
        ``indexer``); its dense flag and layer 0's attend set follow
        :func:`lagged_layer_plan`.  ``first_attend`` is what layer 0 attends
        when it is a DSA layer without a cold start of its own (not used
        when layer 0 is dense or attends its own selection)."""
        plan = lagged_layer_plan(config, cold_start)
        layers = []
        for i, p in enumerate(plan):
            layer = make_layer(i, p.indexer)
            layer.dense = p.dense
            layers.append(layer)
        if plan and (plan[0].dense or plan[0].attends_own):
            first_attend = layers[0].next_idx  # dense: not read; EAGER: its own fresh selection
        if first_attend is None:
            raise ValueError("layer 0 attends first_attend, which is required here")
        return cls(layers, first_attend, lag_depth=lag_depth)

    def run_eager(self) -> None:
        # every buffer the launches touch is owned by the layers, which this
        # schedule keeps alive (the allocator-safety rule of P:2986-2990)
        _lib.call("dsa_mli_run_eager_depth", self._arr, len(self._args), self.lag_depth,
                  torch.cuda.current_stream().cuda_stream)

    def capture(self) -> None:
        """Capture the whole step into one hipGraph: one stream, one launch
        per layer (three from 8 rows); the indexer and the attention overlap
        inside each launch, not across streams."""
        if self._graph is not None:
            return
        h = ctypes.c_void_p()
        cap = torch.cuda.Stream()
        _lib.call("dsa_mli_graph_create_depth", self._arr, len(self._args), self.lag_depth,
                  cap.cuda_stream, ctypes.byref(h))
        self._graph = h

    def replay(self) -> None:
        if self._graph is None:
            self.capture()
        _lib.call("dsa_mli_graph_launch", self._graph, torch.cuda.current_stream().cuda_stream)

    def sync_status(self, clear: bool = True) -> int:
        """Expired in-launch waits over every layer's buffers (see
        DecodeLayer.sync_status); synchronises."""
        return sum(layer.sync_status(clear) for layer in self.layers)

    def close(self) -> None:
        if self._graph is not None:
            _lib.load().dsa_mli_graph_destroy(self._graph)
            self._graph = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def indexcache_pattern(num_layers: int, freq: int | None = 1, pattern: str | None = None,
                       refresh_layers=None) -> str:
    """IndexCache retention as an "F"/"S" string (F: the layer runs its
    indexer; S: it reuses), resolved in the precedence of SGLang's
    dsa_layer_skips_topk as the overlay extends it (P:191-201):
      * ``pattern`` (index_topk_pattern): one F/S per layer, layers past its
        end run their indexer;
      * ``refresh_layers`` (index_refresh_layers, list or comma string): those
        layers and layer 0 are F;
      * ``freq`` (index_topk_freq): 1 in every ``freq`` layers, from layer 0.
    Layers marked S get no indexer operands in the schedule."""
    if num_layers < 0:
        raise ValueError("num_layers must be >= 0")
    if pattern is not None:
        bad = set(pattern) - {"F", "S"}
        if bad:
            raise ValueError(f"pattern may hold only F and S, got {sorted(bad)}")
        return "".join("S" if i < len(pattern) and pattern[i] == "S" else "F" for i in range(num_layers))
    if refresh_layers is not None:
        if isinstance(refresh_layers, str):
            refresh_layers = [int(x) for x in refresh_layers.split(",") if x.strip()]
        full = {int(x) for x in refresh_layers} | {0}
        return "".join("F" if i in full else "S" for i in range(num_layers))
    f = 1 if freq is None else int(freq)
    if f < 1:
        raise ValueError(f"freq must be >= 1, got {freq}")
    return "".join("F" if i % f == 0 else "S" for i in range(num_layers))
