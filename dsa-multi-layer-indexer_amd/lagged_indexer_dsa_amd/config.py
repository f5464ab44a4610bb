"""Shapes and schedule enums of a DSA attention stack.

Same names, fields, defaults and validation as the reference's
``lagged_indexer_dsa.config`` (config.py:14-210) so configurations carry
over unchanged: V3.2 defaults (128 heads, kv_lora 512, rope 64, 64x128
indexer, top-2048), the GLM-5 and small presets, and the three enums.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum


class AttentionType(str, Enum):
    """FULL: dense causal attention, no indexer of its own.  DSA: sparse
    attention over an indexer's top-k set (config.py:14-25)."""

    FULL = "full"
    DSA = "dsa"


def dense_prefix_attention_types(num_hidden_layers: int, num_dense: int) -> tuple[AttentionType, ...]:
    """``num_dense`` leading FULL layers, DSA for the rest (config.py:28-40)."""
    if not 0 <= num_dense <= num_hidden_layers:
        raise ValueError(f"num_dense must be in [0, {num_hidden_layers}], got {num_dense}")
    return tuple(AttentionType.FULL if i < num_dense else AttentionType.DSA
                 for i in range(num_hidden_layers))


class ColdStartPolicy(str, Enum):
    """Layer-0 DSA behaviour without a predecessor (config.py:43-56):
    DENSE attends densely, EAGER runs its own indexer same-layer."""

    DENSE = "dense"
    EAGER = "eager"


class ScheduleMode(str, Enum):
    """BASELINE: same-layer indexer.  LAGGED_REFERENCE / LAGGED_FUSED: layer
    L attends layer L-1's set, unfused / fused (config.py:59-74)."""

    BASELINE = "baseline"
    LAGGED_REFERENCE = "lagged_reference"
    LAGGED_FUSED = "lagged_fused"


@dataclass(frozen=True)
class DSAConfig:
    """Dimensions of a DSA stack (config.py:77-154)."""

    hidden_size: int = 7168
    num_hidden_layers: int = 61
    num_attention_heads: int = 128
    q_lora_rank: int = 1536
    kv_lora_rank: int = 512
    qk_nope_head_dim: int = 128
    qk_rope_head_dim: int = 64
    v_head_dim: int = 128
    index_n_heads: int = 64
    index_head_dim: int = 128
    index_topk: int = 2048
    intermediate_size: int = 18432
    first_k_dense_replace: int = 3
    attention_layer_types: tuple[AttentionType, ...] | None = field(default=None)
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    indexer_rope_interleave: bool = False

    @property
    def qk_head_dim(self) -> int:
        return self.kv_lora_rank + self.qk_rope_head_dim

    @property
    def resolved_attention_types(self) -> tuple[AttentionType, ...]:
        if self.attention_layer_types is None:
            return tuple(AttentionType.DSA for _ in range(self.num_hidden_layers))
        return tuple(AttentionType(t) for t in self.attention_layer_types)

    def __post_init__(self) -> None:
        if not 0 <= self.first_k_dense_replace <= self.num_hidden_layers:
            raise ValueError(f"first_k_dense_replace must be in [0, {self.num_hidden_layers}], "
                             f"got {self.first_k_dense_replace}")
        if self.index_topk <= 0:
            raise ValueError("index_topk must be positive")
        if self.num_attention_heads <= 0:
            raise ValueError("num_attention_heads must be positive")
        if self.qk_rope_head_dim % 2 != 0:
            raise ValueError("qk_rope_head_dim must be even for rotary embeddings")
        if self.index_head_dim % 2 != 0:
            raise ValueError("index_head_dim must be even for rotary embeddings")
        if self.attention_layer_types is not None:
            resolved = self.resolved_attention_types
            if len(resolved) != self.num_hidden_layers:
                raise ValueError(f"attention_layer_types has length {len(resolved)}, "
                                 f"expected num_hidden_layers={self.num_hidden_layers}")


GLM5_CONFIG = DSAConfig(
    hidden_size=6144, num_hidden_layers=78, num_attention_heads=64, q_lora_rank=2048,
    kv_lora_rank=512, qk_nope_head_dim=192, qk_rope_head_dim=64, v_head_dim=256,
    index_n_heads=32, index_head_dim=128, index_topk=2048, intermediate_size=12288,
    first_k_dense_replace=3, rope_theta=1_000_000.0, indexer_rope_interleave=True,
)
GLM5_1_CONFIG = GLM5_CONFIG
SMALL_CONFIG = DSAConfig(
    hidden_size=256, num_hidden_layers=6, num_attention_heads=8, q_lora_rank=96,
    kv_lora_rank=64, qk_nope_head_dim=32, qk_rope_head_dim=16, v_head_dim=32,
    index_n_heads=8, index_head_dim=16, index_topk=16, intermediate_size=512,
)


def named_config(name: str) -> DSAConfig:
    presets = {"deepseek": DSAConfig(), "glm5": GLM5_CONFIG, "glm5.1": GLM5_1_CONFIG,
               "small": SMALL_CONFIG}
    if name not in presets:
        raise ValueError(f"unknown config '{name}'; choose from {sorted(presets)}")
    return presets[name]
