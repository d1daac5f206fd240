"""Slot-mapped KV-cache write -- CPU definition.

Restates store_kvcache_kernel (nanovllm/layers/attention.py:10-30): for every
token i whose slot s = slot_mapping[i] is not -1, the token's
num_kv_heads*head_dim row of key/value replaces row s of the cache viewed as
[num_blocks*block_size, num_kv_heads*head_dim]; every other slot keeps its
bytes.  The quantised variant stores E4M3FN codes and one fp32 scale per
(token, kv head) (docs/project_manual.md:527-537, 583) using ``fp8.quantize_kv``.
Arrays are numpy; bf16 tensors travel as their uint16 bit patterns so the
comparison is bitwise.
"""
from __future__ import annotations

import numpy as np

from . import fp8


def _rows(cache: np.ndarray) -> np.ndarray:
    return cache.reshape(cache.shape[0] * cache.shape[1], -1)


def store_kvcache(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  slot_mapping) -> None:
    """In-place write of ``key``/``value`` [N, H, D] into caches [nblk, bs, H, D]."""
    slots = np.asarray(slot_mapping, dtype=np.int64)
    live = slots != -1
    kr, vr = _rows(k_cache), _rows(v_cache)
    kr[slots[live]] = key.reshape(key.shape[0], -1)[live]
    vr[slots[live]] = value.reshape(value.shape[0], -1)[live]


def store_kvcache_fp8(key_f32: np.ndarray, value_f32: np.ndarray, k_codes: np.ndarray,
                      v_codes: np.ndarray, k_scale: np.ndarray, v_scale: np.ndarray, slot_mapping,
                      scale_floor: float = fp8.SCALE_FLOOR) -> None:
    """Quantised write: codes [nblk, bs, H, D] uint8, scales [nblk, bs, H] fp32."""
    slots = np.asarray(slot_mapping, dtype=np.int64)
    live = slots != -1
    for src, codes, scales in ((key_f32, k_codes, k_scale), (value_f32, v_codes, v_scale)):
        c, s = fp8.quantize_kv(src[live], scale_floor)
        _rows(codes)[slots[live]] = c.reshape(c.shape[0], -1)
        scales.reshape(-1, scales.shape[-1])[slots[live]] = s
