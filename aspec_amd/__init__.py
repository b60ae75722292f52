"""aspec_amd: MI355X-native (gfx950 HIP) DSpark draft hot path.

Drop-in replacements for the reference operators of aspec/models/ops (direct CP / THD attention,
THD sparse metadata, tiled L1, the selective-head losses) backed by hand-written HIP kernels in
libaspec_amd.so, reached through the C ABI of include/aspec_amd.h.
"""

from aspec_amd.direct_cp import (  # noqa: F401
    MASK_VALUE,
    DirectCPMetadata,
    build_context_positions,
    direct_cp_attention,
    direct_cp_attention_from_kv,
    direct_cp_attention_observation,
)
from aspec_amd.thd_attention import thd_fa4_attention  # noqa: F401
from aspec_amd.thd_sparse_metadata import build_thd_sparse_pair  # noqa: F401
from aspec_amd.tiled_l1 import tiled_l1_from_logits  # noqa: F401

__all__ = [
    "MASK_VALUE",
    "DirectCPMetadata",
    "build_context_positions",
    "build_thd_sparse_pair",
    "direct_cp_attention",
    "direct_cp_attention_from_kv",
    "direct_cp_attention_observation",
    "thd_fa4_attention",
    "tiled_l1_from_logits",
]
