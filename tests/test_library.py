"""CPU checks of the drop-in boundary: the C-ABI library loads, exports exactly what
include/aspec_amd.h declares, and the Python surface fails closed like the reference."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from aspec_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "aspec_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(aspec_\w+)\(", text, re.M)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.aspec_abi_version() == _lib.ABI_VERSION


def test_size_queries_and_error_codes_without_gpu():
    lib = _lib.load()
    size = ctypes.c_size_t()
    assert lib.aspec_dspark_plan_bytes(8192, 12288, ctypes.byref(size)) == 0
    assert size.value > 0 and size.value % 256 == 0
    assert lib.aspec_dspark_attn_bwd_workspace_bytes(8192, 12288, 32, 8, ctypes.byref(size)) == 0
    assert size.value == (2 * 8192 * 32 + 2 * 4 * 12288 * 8 * 128) * 4  # delta, lse2; 4 dK/dV partial slots
    assert lib.aspec_loss_stats_floats() == 8
    # invalid geometry is rejected before any launch, with the reference's message
    with pytest.raises(ValueError, match="Invalid THD fixed sparse geometry"):
        _lib.check(lib.aspec_thd_tile_metadata(None, 0, 10, 256, 128, 1, *([None] * 10)))
    with pytest.raises(NotImplementedError, match="head_dim 128"):
        _lib.check(lib.aspec_dspark_attn_fwd(None, 0, 0, None, 0, 0, None, 0, 0, None, None,
                                             16, 48, 4, 2, 64, 0.1, None, 0, 0, None, 4, None))
    with pytest.raises(ValueError, match="divisible"):
        _lib.check(lib.aspec_dspark_attn_fwd(None, 0, 0, None, 0, 0, None, 0, 0, None, None,
                                             16, 48, 5, 2, 128, 0.1, None, 0, 0, None, 4, None))
    with pytest.raises(NotImplementedError, match="bf16 or fp16"):
        _lib.check(lib.aspec_dspark_attn_fwd(None, 0, 0, None, 0, 0, None, 0, 0, None, None,
                                             16, 48, 4, 2, 128, 0.1, None, 0, 0, None, 0, None))
    # the segmented AdamW validates its host table before any launch
    assert lib.aspec_adamw_state_bytes() == 40 + 16 * 64  # step, coef, skip, norm + per-segment counts

    def adamw_segments(grads, numel):
        fake = ctypes.c_void_p(4096)  # never dereferenced: every case below fails validation
        ptrs = (ctypes.c_void_p * len(grads))(*grads)
        sizes = (ctypes.c_int64 * len(numel))(*numel)
        return lib.aspec_adamw_step_segments(fake, fake, fake, fake, ptrs, sizes, len(numel),
                                             1e-3, 0.0, 0.9, 0.999, 1e-8, 1.0, fake, fake, None)

    with pytest.raises(ValueError, match="multiple of 8"):
        _lib.check(adamw_segments([4096, 8192], [12, 8]))
    with pytest.raises(ValueError, match="16-byte aligned"):
        _lib.check(adamw_segments([4096, 8200], [16, 8]))
    with pytest.raises(ValueError, match="no elements"):
        _lib.check(adamw_segments([4096, 0], [16, 0]))
    with pytest.raises(NotImplementedError, match="segment count"):
        _lib.check(adamw_segments([4096] * 65, [8] * 65))


def test_python_surface_fails_closed_on_cpu():
    from aspec_amd import DirectCPMetadata, direct_cp_attention_from_kv, tiled_l1_from_logits

    meta = DirectCPMetadata(torch.tensor([[0, 4]]), torch.tensor([[True, True]]),
                            torch.arange(8)[None], 2, 0, 1, None,
                            context_doc_ids=torch.zeros(1, 8, dtype=torch.long),
                            anchor_doc_ids=torch.zeros(1, 2, dtype=torch.long), sequence_length=8)
    q = torch.randn(1, 4, 4, 128, dtype=torch.bfloat16)
    k = torch.randn(1, 2, 12, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="Combined KV"):
        direct_cp_attention_from_kv(q, k[:, :, :5], k[:, :, :5], meta)
    with pytest.raises(ValueError, match="GPU"):
        direct_cp_attention_from_kv(q, k, k, meta)
    meta.backend = "math"
    with pytest.raises(NotImplementedError, match="HIP kernels only"):
        direct_cp_attention_from_kv(q, k, k, meta)
    with pytest.raises(ValueError, match="unsupported direct CP backend"):
        DirectCPMetadata(torch.tensor([[0]]), torch.tensor([[True]]), torch.arange(4)[None], 2, 0, 1,
                         None, backend="flex")
    values = torch.randn(3, 31, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA logits"):
        tiled_l1_from_logits(values, values)
