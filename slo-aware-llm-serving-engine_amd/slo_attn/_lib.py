"""ctypes binding of libslo_attn.so, the C-ABI declared in include/slo_attn.h.

The library is built in-tree by ``build.py`` (``hipcc --offload-arch=gfx950``)
next to this file.  There is deliberately no fallback: if the library is
missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libslo_attn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

SLO_OK = 0
KV_BF16 = 0
KV_FP8_E4M3FN = 1
PHASE_DECODE = 1
PHASE_PREFILL = 2
PHASE_ALL = 3
FP8_SCALE_FLOOR = 2.0 ** -64
NOALLOC_SCRATCH_BYTES = 64 << 20
FP8_MAX = 448.0

_c_int32 = ctypes.c_int32
_c_int64 = ctypes.c_int64
_c_void_p = ctypes.c_void_p


class PagedAttentionArgs(ctypes.Structure):
    """Mirror of ``slo_paged_attention_args`` (include/slo_attn.h)."""

    _fields_ = [
        ("q", _c_void_p), ("q_row_stride", _c_int64),
        ("out", _c_void_p), ("out_row_stride", _c_int64),
        ("num_q_rows", _c_int32),
        ("k_cache", _c_void_p), ("v_cache", _c_void_p),
        ("k_scale", _c_void_p), ("v_scale", _c_void_p),
        ("kv_dtype", _c_int32), ("num_blocks", _c_int32), ("block_size", _c_int32),
        ("num_decode", _c_int32),
        ("decode_lens", _c_void_p), ("decode_tables", _c_void_p),
        ("decode_table_stride", _c_int32), ("decode_table_width", _c_int32),
        ("num_prefill", _c_int32),
        ("prefill_cu_q", _c_void_p), ("prefill_cu_k", _c_void_p),
        ("max_q", _c_int32), ("max_k", _c_int32),
        ("prefill_tables", _c_void_p),
        ("prefill_table_stride", _c_int32), ("prefill_table_width", _c_int32),
        ("k", _c_void_p), ("k_row_stride", _c_int64),
        ("v", _c_void_p), ("v_row_stride", _c_int64),
        ("num_kv_rows", _c_int32),
        ("num_heads", _c_int32), ("num_kv_heads", _c_int32), ("head_dim", _c_int32),
        ("softmax_scale", ctypes.c_float),
        ("workspace", _c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("phases", _c_int32),
        ("store_slot_mapping", _c_void_p),
        ("new_k", _c_void_p), ("new_k_row_stride", _c_int64),
        ("new_v", _c_void_p), ("new_v_row_stride", _c_int64),
        ("num_new_rows", _c_int32),
        ("store_scale_floor", ctypes.c_float),
    ]


_lock = threading.Lock()
_lib = None

EXPORTS = (
    "slo_store_kvcache",
    "slo_qk_norm_rope_store",
    "slo_lm_head_argmax",
    "slo_build_mixed_metadata",
    "slo_attention_workspace_bytes",
    "slo_paged_attention",
    "slo_paged_attention_noalloc",
    "slo_attention_workspace_check",
    "slo_last_error",
    "slo_paged_attention_args_size",
)


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it is absent (no CPU fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_NAME} is not built (expected at {LIB_PATH}); run build.py or "
                "__graft_entry__.build() first. There is no CPU fallback.")
        lib = ctypes.CDLL(LIB_PATH)
        lib.slo_store_kvcache.restype = ctypes.c_int
        lib.slo_store_kvcache.argtypes = [
            _c_void_p, _c_int64, _c_void_p, _c_int64, _c_void_p, _c_int32, _c_int32, _c_int32,
            _c_int32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int64, ctypes.c_float, _c_void_p]
        lib.slo_qk_norm_rope_store.restype = ctypes.c_int
        lib.slo_qk_norm_rope_store.argtypes = [
            _c_void_p, _c_int64, _c_void_p, _c_int32, _c_int32, _c_int32, _c_int32, _c_void_p, _c_void_p,
            ctypes.c_float, _c_void_p, _c_int32, _c_void_p, _c_void_p, _c_void_p, _c_int32, _c_void_p, _c_void_p,
            _c_void_p, _c_void_p, _c_int64, ctypes.c_float, _c_void_p]
        lib.slo_lm_head_argmax.restype = ctypes.c_int
        lib.slo_lm_head_argmax.argtypes = [
            _c_void_p, _c_int64, _c_int32, _c_void_p, _c_int64, _c_int32, _c_int32, _c_void_p, _c_int64,
            _c_void_p, _c_void_p, _c_void_p]
        lib.slo_build_mixed_metadata.restype = ctypes.c_int
        lib.slo_build_mixed_metadata.argtypes = [
            _c_void_p, _c_void_p, _c_int32, _c_int32, _c_int32, _c_void_p, _c_int32, _c_int32, _c_int32,
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]
        lib.slo_attention_workspace_bytes.restype = ctypes.c_int
        lib.slo_attention_workspace_bytes.argtypes = [
            _c_int32, _c_int32, _c_int32, _c_int32, _c_int32, ctypes.POINTER(ctypes.c_size_t)]
        lib.slo_paged_attention.restype = ctypes.c_int
        lib.slo_paged_attention.argtypes = [ctypes.POINTER(PagedAttentionArgs), _c_void_p]
        lib.slo_paged_attention_noalloc.restype = ctypes.c_int
        lib.slo_paged_attention_noalloc.argtypes = [ctypes.POINTER(PagedAttentionArgs), _c_void_p]
        lib.slo_attention_workspace_check.restype = ctypes.c_int
        lib.slo_attention_workspace_check.argtypes = [_c_void_p, ctypes.c_size_t, _c_void_p, _c_void_p]
        lib.slo_last_error.restype = ctypes.c_char_p
        lib.slo_last_error.argtypes = []
        lib.slo_paged_attention_args_size.restype = ctypes.c_size_t
        lib.slo_paged_attention_args_size.argtypes = []
        if lib.slo_paged_attention_args_size() != ctypes.sizeof(PagedAttentionArgs):
            raise RuntimeError("slo_paged_attention_args layout mismatch between header and binding")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != SLO_OK:
        msg = load().slo_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def workspace_bytes(max_decode_rows: int, max_decode_len: int, num_heads: int,
                    num_kv_heads: int, head_dim: int) -> int:
    out = ctypes.c_size_t(0)
    check(load().slo_attention_workspace_bytes(max_decode_rows, max_decode_len, num_heads,
                                               num_kv_heads, head_dim, ctypes.byref(out)),
          "slo_attention_workspace_bytes")
    return int(out.value)
