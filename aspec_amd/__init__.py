"""aspec_amd: MI355X-native (gfx950 HIP) DSpark draft hot path.

Drop-in replacements for the reference operators of aspec/models/ops (direct CP / THD attention,
the cuDNN FlexAttention surface with its DSpark interval masks, THD sparse metadata, tiled L1, the selective-head losses, the fused Q/K RMSNorm + RoPE, the DSpark
head terms with the Markov bias and confidence head), the work-aware row packing policy
(aspec/controller/packing.py), the packing collator (aspec/data/utils.py), the anchor layout (anchors.py), output-block compaction (output_blocks.py)
and the DSpark targets (dspark.py), backed by hand-written HIP kernels in libaspec_amd.so,
reached through the C ABI of include/aspec_amd.h.
"""

from aspec_amd.anchors import (  # noqa: F401
    document_anchor_slots,
    sample_anchor_positions,
    sample_document_anchor_positions,
    validate_injected_anchors,
)
from aspec_amd.collate import DFlashPackingCollator  # noqa: F401
from aspec_amd.cudnn_flex_attention import (  # noqa: F401
    CudnnFlexMask,
    build_dspark_mla_mask,
    cudnn_flex_attention,
    resolve_cudnn_gqa_mode,
)
from aspec_amd.direct_cp import (  # noqa: F401
    MASK_VALUE,
    DirectCPMetadata,
    build_context_positions,
    direct_cp_attention,
    direct_cp_attention_from_kv,
    direct_cp_attention_observation,
    direct_cp_partial_attention,
    merge_attention_partials,
)
from aspec_amd.dspark_head import (  # noqa: F401
    AcceptRatePredictor,
    VanillaMarkov,
    acceptance_statistics,
    build_markov_head,
    dspark_prediction_terms,
    markov_head_logits,
)
from aspec_amd.dspark_qk_norm_rope import (  # noqa: F401
    dspark_qk_norm_rope,
    dspark_qk_norm_rope_available,
)
from aspec_amd.packing import (  # noqa: F401
    PackingResult,
    count_eligible_anchor_starts,
    count_eligible_anchor_starts_batch,
    pack_work_aware_rows,
)
from aspec_amd.targets import decay_weights, dspark_targets  # noqa: F401
from aspec_amd.output_blocks import (  # noqa: F401
    output_block_counts,
    output_block_indices,
    owner_block_indices,
    prepare_block_layout,
    restore_blocks,
    select_blocks,
)
from aspec_amd.head_loss import selective_head_objective  # noqa: F401
from aspec_amd.loss import ce_l1_fused_grad  # noqa: F401
from aspec_amd.thd_attention import thd_fa4_attention  # noqa: F401
from aspec_amd.thd_sparse_metadata import build_thd_sparse_pair  # noqa: F401
from aspec_amd.tiled_l1 import tiled_l1_from_logits  # noqa: F401

__all__ = [
    "AcceptRatePredictor",
    "CudnnFlexMask",
    "build_dspark_mla_mask",
    "cudnn_flex_attention",
    "resolve_cudnn_gqa_mode",
    "DFlashPackingCollator",
    "PackingResult",
    "count_eligible_anchor_starts",
    "count_eligible_anchor_starts_batch",
    "pack_work_aware_rows",
    "VanillaMarkov",
    "acceptance_statistics",
    "build_markov_head",
    "dspark_prediction_terms",
    "markov_head_logits",
    "decay_weights",
    "document_anchor_slots",
    "dspark_qk_norm_rope",
    "dspark_qk_norm_rope_available",
    "dspark_targets",
    "output_block_counts",
    "output_block_indices",
    "owner_block_indices",
    "prepare_block_layout",
    "restore_blocks",
    "sample_anchor_positions",
    "sample_document_anchor_positions",
    "select_blocks",
    "validate_injected_anchors",
    "MASK_VALUE",
    "DirectCPMetadata",
    "build_context_positions",
    "build_thd_sparse_pair",
    "direct_cp_attention",
    "direct_cp_attention_from_kv",
    "direct_cp_attention_observation",
    "direct_cp_partial_attention",
    "merge_attention_partials",
    "thd_fa4_attention",
    "tiled_l1_from_logits",
]
