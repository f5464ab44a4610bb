"""MI355X-native DeepSeek Sparse Attention decode path with the Multi-layer Indexer.

Hot path (HIP kernels for gfx950 behind the C ABI of include/dsa_mli.h):
lightning-indexer scan over a paged fp8 index-K cache -> exact top-k ->
split-K sparse MLA over the fp8 656-byte latent pool, and the MLI lag
schedule (layer i attends layer i-1's selection while layer i's indexer runs
in the same launch, on workgroups of their own) captured as one hipGraph.

Python surface mirrors the reference package ``lagged_indexer_dsa``
(attention_core / dsa_layer / model / config); every compute call goes to
the HIP library and there is no CPU path.
"""

from ._lib import DsaError
from .config import (
    GLM5_CONFIG,
    SMALL_CONFIG,
    AttentionType,
    ColdStartPolicy,
    DSAConfig,
    ScheduleMode,
    dense_prefix_attention_types,
    named_config,
)

__all__ = [
    "AttentionType",
    "ColdStartPolicy",
    "DSAConfig",
    "DsaError",
    "GLM5_CONFIG",
    "SMALL_CONFIG",
    "ScheduleMode",
    "dense_prefix_attention_types",
    "named_config",
]
