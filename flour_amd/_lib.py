"""ctypes binding of libflour_hip.so (the C-ABI declared in include/flour_hip.h).

The library is built in-tree by ``flour_amd.build``. Loading fails loudly when it is missing:
there is no CPU or pure-PyTorch fallback for any operation of this package.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libflour_hip.so"

F32, BF16, F16 = 0, 1, 2
OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_UNSUPPORTED = -2
ERR_WORKSPACE = -3
ERR_HIP = -4
ERR_OUT_OF_BLOCKS = -5
ERR_CAPACITY = -6

_c_int, _c_i64, _c_f, _vp, _c_sz = (ctypes.c_int, ctypes.c_int64, ctypes.c_float,
                                    ctypes.c_void_p, ctypes.c_size_t)
_i32p = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES: dict[str, tuple] = {
    "flour_hip_last_error": (ctypes.c_char_p, []),
    "flour_hip_version": (ctypes.c_char_p, []),
    "flour_hip_kv_write": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _c_int,
                                    _c_int, _c_i64, _c_int, _vp]),
    "flour_hip_rope_kv_write": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_int, _vp, _vp, _c_i64,
                                         _c_i64, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int,
                                         _c_int, _c_int, _c_i64, _c_int, _vp]),
    "flour_hip_paged_decode_workspace_size": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int,
                                                       ctypes.POINTER(ctypes.c_size_t)]),
    "flour_hip_paged_decode": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _c_int, _vp, _c_int,
                                        _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_f,
                                        _c_int, _vp, _c_sz, _vp]),
    "flour_hip_paged_decode_noalloc_max_workspace": (_c_sz, []),
    "flour_hip_paged_decode_noalloc": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _c_int, _vp,
                                                _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64,
                                                _c_int, _c_f, _c_int, _vp]),
    "flour_hip_varlen_prefill": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp,
                                          _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                          _c_int, _c_int, _c_int, _c_int, _c_i64, _c_f, _c_int,
                                          _vp]),
    "flour_hip_varlen_prefill_workspace_size": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int,
                                                         _c_int, ctypes.POINTER(ctypes.c_size_t)]),
    "flour_hip_varlen_prefill_ws": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _c_i64, _c_i64,
                                             _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_f,
                                             _c_int, _vp, _c_sz, _vp]),
    # include/flour_cache.h
    "flour_block_allocator_create": (_c_int, [_c_int, _vp]),
    "flour_block_allocator_destroy": (None, [_vp]),
    "flour_block_allocator_allocate": (_c_int, [_vp]),
    "flour_block_allocator_incref": (_c_int, [_vp, _c_int]),
    "flour_block_allocator_decref": (_c_int, [_vp, _c_int]),
    "flour_block_allocator_ref_count": (_c_int, [_vp, _c_int]),
    "flour_block_allocator_num_free": (_c_int, [_vp]),
    "flour_block_table_create": (_c_int, [_c_int, _vp]),
    "flour_block_table_destroy": (None, [_vp]),
    "flour_block_table_push_block": (_c_int, [_vp, _c_int]),
    "flour_block_table_advance": (_c_int, [_vp, _c_int]),
    "flour_block_table_clear": (_c_int, [_vp]),
    "flour_block_table_len": (_c_int, [_vp]),
    "flour_block_table_capacity": (_c_int, [_vp]),
    "flour_block_table_block_size": (_c_int, [_vp]),
    "flour_block_table_blocks": (_c_int, [_vp, _vp, _c_int, _vp]),
    "flour_block_table_slot": (_c_i64, [_vp, _c_int]),
    "flour_block_table_slots": (_c_int, [_vp, _c_int, _c_int, _vp]),
    "flour_kv_cache_create": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _vp]),
    "flour_kv_cache_destroy": (None, [_vp]),
    "flour_kv_cache_allocate_kv": (_c_int, [_vp, _c_int]),
    "flour_kv_cache_len": (_c_int, [_vp]),
    "flour_kv_cache_capacity": (_c_int, [_vp]),
    "flour_kv_cache_free_blocks": (_c_int, [_vp]),
    "flour_kv_cache_ref_count": (_c_int, [_vp, _c_int]),
    "flour_kv_cache_blocks": (_c_int, [_vp, _vp, _c_int, _vp]),
    "flour_kv_cache_slots": (_c_int, [_vp, _c_int, _c_int, _vp]),
    "flour_kv_cache_write_kv": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_i64, _c_i64, _vp]),
    "flour_kv_cache_attention": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_i64, _c_i64, _vp,
                                          _c_int, _c_i64, _c_i64, _c_f, _vp]),
    "flour_kv_cache_reset_sequence": (_c_int, [_vp]),
    "flour_kv_cache_match_prefix": (_c_int, [_vp, _vp, _c_int]),
    "flour_kv_cache_register_prefix": (_c_int, [_vp, _vp, _c_int]),
    "flour_kv_cache_clear_prefix_cache": (_c_int, [_vp]),
    "flour_kv_cache_export_bundle": (_c_int, [_vp, ctypes.c_char_p, _vp, _c_int, _c_int, _vp, _c_sz,
                                              ctypes.POINTER(ctypes.c_size_t), _vp]),
    "flour_kv_cache_import_bundle": (_c_int, [_vp, _vp, _c_sz, _vp, _c_int,
                                              ctypes.POINTER(ctypes.c_int), _vp]),
    "flour_kv_batch_create": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _c_int, _c_int, _c_int, _vp]),
    "flour_kv_batch_destroy": (None, [_vp]),
    "flour_kv_batch_add_sequence": (_c_int, [_vp, ctypes.POINTER(ctypes.c_int)]),
    "flour_kv_batch_remove_sequence": (_c_int, [_vp, _c_int]),
    "flour_kv_batch_reset_sequence": (_c_int, [_vp, _c_int]),
    "flour_kv_batch_allocate_kv": (_c_int, [_vp, _c_int, _c_int]),
    "flour_kv_batch_len": (_c_int, [_vp, _c_int]),
    "flour_kv_batch_free_blocks": (_c_int, [_vp]),
    "flour_kv_batch_ref_count": (_c_int, [_vp, _c_int]),
    "flour_kv_batch_blocks": (_c_int, [_vp, _c_int, _vp, _c_int, ctypes.POINTER(ctypes.c_int)]),
    "flour_kv_batch_match_prefix": (_c_int, [_vp, _c_int, _vp, _c_int]),
    "flour_kv_batch_register_prefix": (_c_int, [_vp, _c_int, _vp, _c_int]),
    "flour_kv_batch_clear_prefix_cache": (_c_int, [_vp]),
    "flour_kv_batch_plan": (_c_int, [_vp, _vp, _vp, _c_int, _vp]),
    "flour_kv_batch_step": (_c_int, [_vp, _vp, _vp, _c_int, _vp]),
    "flour_kv_batch_write_kv": (_c_int, [_vp, _c_int, _vp, _vp, _c_i64, _c_i64, _vp]),
    "flour_kv_batch_rope_write_kv": (_c_int, [_vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_int, _vp,
                                              _vp, _c_i64, _c_i64, _vp, _vp, _c_int, _vp]),
    "flour_kv_batch_attention": (_c_int, [_vp, _c_int, _vp, _c_int, _c_i64, _c_i64, _vp, _c_int,
                                          _c_i64, _c_i64, _c_f, _vp]),
    "flour_kv_batch_write_kv_attention": (_c_int, [_vp, _c_int, _vp, _vp, _c_i64, _c_i64, _vp,
                                                   _c_int, _c_i64, _c_i64, _vp, _c_int, _c_i64,
                                                   _c_i64, _c_f, _vp]),
    "flour_kv_batch_pool": (_c_int, [_vp, _c_int, _vp, _vp, _vp]),
    "flour_kv_cache_pool": (_c_int, [_vp, _c_int, _vp, _vp, _vp]),
}


class FlourError(RuntimeError):
    """An error reported by libflour_hip.so (negative return code)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Load libflour_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("FLOUR_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise FlourError(ERR_HIP, f"{path} is missing: build it with `python -m flour_amd.build` "
                                  "(there is no fallback path)")
    handle = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    for name in EXTRA_SIGNATURES:
        res, args = EXTRA_SIGNATURES[name]
        fn = getattr(handle, name, None)
        if fn is not None:
            fn.restype = res
            fn.argtypes = args
    _lib = handle
    return handle


# Optional, non-header helpers (test / tuning switches).
EXTRA_SIGNATURES: dict[str, tuple] = {
    "flour_hip_set_prefill_precise_p": (_c_int, [_c_int]),
    "flour_hip_set_decode_workgroups": (_c_int, [_c_int]),
    "flour_hip_set_decode_xcd_weight": (_c_int, [_c_int]),
    "flour_hip_set_prefill_persistent": (_c_int, [_c_int]),
    "flour_hip_set_prefill_dma": (_c_int, [_c_int]),
    "flour_hip_set_prefill_f32_mfma": (_c_int, [_c_int]),
    "flour_hip_set_batch_split": (_c_int, [_c_int]),
    "flour_hip_set_batch_fuse": (_c_int, [_c_int]),
    "flour_hip_empty_launch": (_c_int, [_vp]),
}


def check(code: int) -> None:
    if code != OK:
        msg = lib().flour_hip_last_error().decode(errors="replace")
        raise FlourError(code, msg)


def last_error() -> str:
    return lib().flour_hip_last_error().decode(errors="replace")
