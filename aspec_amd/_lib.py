"""ctypes binding of libaspec_amd.so, the HIP C ABI declared in include/aspec_amd.h.

There is no fallback: if the library is missing or a call fails, an exception is raised.
Status codes map to the reference's exception types (ValueError for layout violations,
NotImplementedError for unsupported combinations, RuntimeError for HIP failures).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libaspec_amd.so"

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_size_p = ctypes.POINTER(ctypes.c_size_t)

# name -> (restype, argtypes); the exact export list of include/aspec_amd.h.
SIGNATURES = {
    "aspec_abi_version": (_int, []),
    "aspec_last_error": (ctypes.c_char_p, []),
    "aspec_thd_row_metadata": (_int, [_c_void_p] * 5 + [_i64] * 6 + [_int] + [_c_void_p] * 5),
    "aspec_thd_batch_row_metadata": (_int, [_c_void_p] * 5 + [_i64] * 7 + [_int] + [_c_void_p] * 5),
    "aspec_thd_cp_shard_endpoints": (_int, [_c_void_p] * 5 + [_i64] * 4 + [_c_void_p, _i64, _c_void_p, _i64]
                                     + [_i64] * 3 + [_int] + [_c_void_p] * 3),
    "aspec_dspark_mla_mask_workspace_bytes": (_int, [_i64, _i64, _size_p]),
    "aspec_dspark_mla_mask": (_int, [_c_void_p] * 3 + [_i64] * 4 + [_int] + [_i64] * 2 + [_c_void_p] * 4),
    "aspec_flex_mask_intervals": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64]
                                  + [_c_void_p] * 3),
    "aspec_thd_aux_endpoints": (_int, [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _int,
                                        _c_void_p, _c_void_p, _c_void_p]),
    "aspec_thd_tile_metadata": (_int, [_c_void_p, _i64, _i64, _i64, _i64, _int] + [_c_void_p] * 10),
    "aspec_dspark_plan_bytes": (_int, [_i64, _i64, _size_p]),
    "aspec_dspark_plan_build": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "aspec_dspark_attn_fwd": (
        _int,
        [_c_void_p, _i64, _i64] * 3
        + [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _f32, _c_void_p, _i64, _i64,
           _c_void_p, _int, _c_void_p],
    ),
    "aspec_dspark_attn_bwd_workspace_bytes": (_int, [_i64, _i64, _i64, _i64, _size_p]),
    "aspec_dspark_attn_bwd": (
        _int,
        [_c_void_p, _i64, _i64] * 5
        + [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _f32]
        + [_c_void_p, _i64, _i64] * 3
        + [_c_void_p, _int, _c_void_p],
    ),
    "aspec_dspark_attn_bwd_stages": (
        _int,
        [_int]
        + [_c_void_p, _i64, _i64] * 5
        + [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _f32]
        + [_c_void_p, _i64, _i64] * 3
        + [_c_void_p, _int, _c_void_p],
    ),
    "aspec_loss_stats_floats": (_int, []),
    "aspec_ce_l1_fwd": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64] + [_c_void_p] * 5
    ),
    "aspec_ce_l1_argmax_fwd": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64] + [_c_void_p] * 6
    ),
    "aspec_ce_l1_bwd": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64] + [_c_void_p] * 5
    ),
    "aspec_ce_l1_fused_fwd_bwd": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64] + [_c_void_p] * 9
    ),
    "aspec_scale_bf16_by_device_scalar": (_int, [_c_void_p, _i64, _c_void_p, _c_void_p]),
    "aspec_sampling_stats_floats": (_int, []),
    "aspec_sampling_logits_fwd": (_int, [_c_void_p, _i64, _i64, _f64, _f64, _i64] + [_c_void_p] * 3),
    "aspec_sampling_logits_bwd": (_int, [_c_void_p] * 3 + [_i64, _i64] + [_c_void_p] * 2),
    "aspec_sampled_l1_stats_floats": (_int, []),
    "aspec_sampled_l1_fwd": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _f64, _f64, _i64, _f64, _f64, _i64]
        + [_c_void_p] * 4
    ),
    "aspec_sampled_l1_bwd": (_int, [_c_void_p] * 3 + [_i64, _i64, _i64] + [_c_void_p] * 4),
    "aspec_pack_copy": (_int, [_c_void_p, _i64, _c_void_p]),
    "aspec_pack_row_metadata": (_int, [_c_void_p, _i64, _i64] + [_c_void_p] * 4),
    "aspec_sample_document_anchors": (
        _int, [_c_void_p, _int, _c_void_p, _i64, _c_void_p] + [_i64] * 5 + [_c_void_p] * 5
    ),
    "aspec_sample_anchors": (
        _int, [_c_void_p, _int, _c_void_p, _int] + [_i64] * 5 + [_c_void_p] * 5
    ),
    "aspec_validate_injected_anchors": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _int, _c_void_p] + [_i64] * 4
        + [_int, _c_void_p, _c_void_p, _c_void_p]
    ),
    "aspec_output_block_layout": (_int, [_c_void_p] + [_i64] * 6 + [_c_void_p] * 3),
    "aspec_qk_norm_rope_fwd": (
        _int, [_c_void_p] * 7 + [_i64, _i64] + [_c_void_p] * 3 + [_i64] * 6 + [_f32, _int]
        + [_c_void_p] * 6
    ),
    "aspec_qk_norm_rope_bwd_workspace_bytes": (_int, [_i64] * 5 + [_size_p]),
    "aspec_qk_norm_rope_bwd": (
        _int, [_c_void_p] * 11 + [_i64, _i64] + [_c_void_p] * 3 + [_i64] * 6 + [_f32, _int]
        + [_c_void_p] * 8
    ),
    "aspec_qk_norm_rope_bwd_noalloc": (
        _int, [_c_void_p] * 11 + [_i64, _i64] + [_c_void_p] * 3 + [_i64] * 6 + [_f32, _int]
        + [_c_void_p] * 7
    ),
    "aspec_rmsnorm_fwd": (_int, [_c_void_p] * 3 + [_i64, _i64, _f32] + [_c_void_p] * 4),
    "aspec_rmsnorm_bwd_workspace_bytes": (_int, [_i64, _c_void_p]),
    "aspec_rmsnorm_bwd": (_int, [_c_void_p] * 5 + [_i64, _i64] + [_c_void_p] * 4),
    "aspec_swiglu_fwd": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "aspec_swiglu_bwd": (_int, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "aspec_adamw_state_bytes": (_int, []),
    "aspec_adamw_workspace_bytes": (_int, [_c_void_p]),
    "aspec_adamw_step": (
        _int, [_c_void_p] * 5 + [_i64] + [_f32] * 6 + [_c_void_p] * 3
    ),
    "aspec_adamw_step_segments": (
        _int, [_c_void_p] * 6 + [_int] + [_f32] * 6 + [_c_void_p] * 3
    ),
    "aspec_dspark_targets": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _c_void_p] + [_i64] * 5
        + [_c_void_p] * 8
    ),
    "aspec_count_eligible_anchor_starts": (_int, [_c_void_p] * 3 + [_i64, _i64, _c_void_p]),
    "aspec_pack_work_aware_rows": (_int, [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64] + [_c_void_p] * 3),
}

ABI_VERSION = 15

_lock = threading.Lock()
_lib = None


class AspecError(RuntimeError):
    pass


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and type the HIP library. Raises RuntimeError when it is absent."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path is not None else LIBRARY_PATH
        if not target.exists():
            raise RuntimeError(
                f"aspec_amd HIP library not built: {target} is missing "
                "(run `python -m aspec_amd.build` or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(target))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if lib.aspec_abi_version() != ABI_VERSION:
            raise RuntimeError("aspec_amd library ABI version mismatch; rebuild it")
        if path is None:
            _lib = lib
        return lib


def check(status: int) -> None:
    if status == 0:
        return
    message = (_lib.aspec_last_error() or b"").decode(errors="replace") if _lib else ""
    if status == 1:
        raise ValueError(message)
    if status == 2:
        raise NotImplementedError(message)
    raise RuntimeError(message or f"aspec_amd call failed with status {status}")


def call(name: str, *args) -> None:
    lib = load()
    check(getattr(lib, name)(*args))


# ASPEC_MASK_* dtype codes of include/aspec_amd.h
def mask_dtype_code(tensor) -> int:
    import torch

    codes = {torch.float32: 0, torch.int64: 1, torch.int32: 2, torch.bool: 3, torch.uint8: 3,
             torch.bfloat16: 4, torch.float16: 5}
    if tensor.dtype not in codes:
        raise ValueError(f"unsupported mask dtype {tensor.dtype}")
    return codes[tensor.dtype]


def ptr(tensor) -> int | None:
    """Raw device pointer of a torch tensor (None for None)."""
    return None if tensor is None else tensor.data_ptr()


def stream_handle(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream
