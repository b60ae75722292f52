"""`CudnnFlexMask`'s derived-mask and plan caches on the CPU, as the reference's
tests/test_cudnn_flex_attention.py:160-200 pin them: the physical-GQA mask of a THD mask repeats each
query row `ratio` times, scales the query lengths, keeps the key side, is reused while the mask is
unchanged and rebuilt (with a new plan key) after an in-place change of the query lengths."""

import pytest
import torch

from aspec_amd.cudnn_flex_attention import CudnnFlexMask


def test_thd_physical_gqa_reuses_metadata_and_invalidates_changed_lengths():
    mask = CudnnFlexMask(mask_func=torch.zeros(1, 5, 5, dtype=torch.int32),
                         cu_seqlens_q=torch.tensor([0, 2, 5], dtype=torch.int32),
                         cu_seqlens_k=torch.tensor([0, 7, 16], dtype=torch.int32),
                         max_seqlen_q=3, max_seqlen_k=9)
    physical = mask.for_physical_gqa(3)
    assert physical is mask.for_physical_gqa(3)
    assert physical.cu_seqlens_q.tolist() == [0, 6, 15]
    assert physical.max_seqlen_q == 9
    assert physical.cu_seqlens_k is mask.cu_seqlens_k
    assert physical.max_seqlen_k == 9
    query, key = torch.empty(5, 6, 128), torch.empty(16, 2, 128)
    plan_key = mask._plan_key(query, key, key, None)
    mask.cu_seqlens_q[1] = 3
    changed = mask.for_physical_gqa(3)
    assert changed is not physical
    assert changed.cu_seqlens_q.tolist() == [0, 9, 15]
    assert mask._plan_key(query, key, key, None) != plan_key


def test_physical_gqa_mask_repeats_queries_and_reuses_derived_mask():
    # the interval-union mask of two DSpark blocks (block 2, anchors 1 and 4, 8 context tokens),
    # as build_dspark_mla_mask writes it: [0, e0) U [e1, e2) per query row
    mask_func = torch.tensor([[[1, 1, 4, 4], [8, 8, 8, 8], [8, 8, 10, 10]]], dtype=torch.int32)
    mask = CudnnFlexMask(mask_func)
    physical = mask.for_physical_gqa(4)
    assert physical is mask.for_physical_gqa(4)
    assert physical.pack_gqa is False
    torch.testing.assert_close(physical.mask_func, mask.mask_func.repeat_interleave(4, dim=-1))
    assert mask.for_physical_gqa(1) is mask
    mask.mask_func[0, 0, 0] = 2  # an in-place change invalidates the derived mask
    assert mask.for_physical_gqa(4) is not physical
    with pytest.raises(ValueError, match="positive"):
        mask.for_physical_gqa(0)
