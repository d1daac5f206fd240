"""q/k RMSNorm, rotary embedding and the fused KV write -- CPU definition (numpy).

* ``rms_norm`` restates RMSNorm.rms_forward (nanovllm/layers/layernorm.py:16-26)
  over the last axis: x in fp32, var = mean(x^2), x * rsqrt(var + eps) in fp32,
  rounded to bf16, then multiplied by the bf16 weight (the product of two bf16
  values is exact in fp32) and rounded to bf16 again.  Two points the
  reference leaves to its compiler are fixed here: the mean is the exact mean
  rounded once to fp32 (the sum of squares is taken in float64, where it is
  exact for the magnitudes involved), and rsqrt is correctly rounded (float64
  1/sqrt, rounded once to fp32).
* ``rope`` restates apply_rotary_emb (nanovllm/layers/rotary_embedding.py:6-14):
  halves x1, x2 of the head in fp32, y1 = x1*cos - x2*sin, y2 = x2*cos + x1*sin
  with every product and sum rounded to fp32 (eager evaluation, no fused
  multiply-add), then bf16.  ``cos_sin`` is the reference's cos_sin_cache
  (rotary_embedding.py:27-35): row p holds cos(p*inv_freq) then sin(p*inv_freq).
* ``qkv_step`` is the part of Qwen3Attention.forward between qkv_proj and the
  attention call (nanovllm/models/qwen3.py:80-85) on the fused QKV rows,
  followed by the KV write of ``kvstore`` (attention.py:10-40): k after RoPE,
  v as given.  Positions outside the table are clamped into it, as the HIP
  kernel does.

bf16 tensors travel as uint16 bit patterns so every comparison is bitwise.
"""
from __future__ import annotations

import numpy as np

from . import kvstore


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def rms_norm(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    x = bf16_to_f32(x_bits)
    ss = np.square(x.astype(np.float64)).sum(axis=-1, keepdims=True)
    var = (ss / x.shape[-1]).astype(np.float32)
    r = (1.0 / np.sqrt((var + np.float32(eps)).astype(np.float64))).astype(np.float32)
    n = f32_to_bf16(x * r)
    return f32_to_bf16(bf16_to_f32(n) * bf16_to_f32(w_bits))


def rope(x_bits: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [N, H, D] bf16 bits; cos/sin [N, D/2] fp32 for each token's position."""
    x = bf16_to_f32(x_bits)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c = np.asarray(cos, dtype=np.float32)[:, None, :]
    s = np.asarray(sin, dtype=np.float32)[:, None, :]
    y1 = (x1 * c) - (x2 * s)
    y2 = (x2 * c) + (x1 * s)
    return f32_to_bf16(np.concatenate([y1, y2], axis=-1))


def qkv_step(qkv_bits, positions, q_w_bits, k_w_bits, eps, cos_sin, num_heads, num_kv_heads,
             head_dim=128):
    """Returns (q, k, v) bf16 bits: q/k normalised and rotated, v unchanged."""
    qkv_bits = np.asarray(qkv_bits, dtype=np.uint16)
    n = qkv_bits.shape[0]
    q = qkv_bits[:, :num_heads * head_dim].reshape(n, num_heads, head_dim)
    k = qkv_bits[:, num_heads * head_dim:(num_heads + num_kv_heads) * head_dim].reshape(n, num_kv_heads, head_dim)
    v = qkv_bits[:, (num_heads + num_kv_heads) * head_dim:(num_heads + 2 * num_kv_heads) * head_dim]
    v = v.reshape(n, num_kv_heads, head_dim)
    pos = np.clip(np.asarray(positions, dtype=np.int64), 0, cos_sin.shape[0] - 1)
    cos = cos_sin[pos, :head_dim // 2]
    sin = cos_sin[pos, head_dim // 2:]
    q = rope(rms_norm(q, q_w_bits, eps), cos, sin)
    k = rope(rms_norm(k, k_w_bits, eps), cos, sin)
    return q, k, v.copy()


def qkv_step_store(qkv_bits, positions, q_w_bits, k_w_bits, eps, cos_sin, num_heads, num_kv_heads,
                   slot_mapping, k_cache, v_cache, k_scale=None, v_scale=None, head_dim=128):
    """``qkv_step`` and the KV write into numpy pools (bf16 bits, or E4M3FN codes + scales)."""
    q, k, v = qkv_step(qkv_bits, positions, q_w_bits, k_w_bits, eps, cos_sin, num_heads, num_kv_heads,
                       head_dim)
    if k_scale is None:
        kvstore.store_kvcache(k, v, k_cache, v_cache, slot_mapping)
    else:
        kvstore.store_kvcache_fp8(bf16_to_f32(k), bf16_to_f32(v), k_cache, v_cache, k_scale, v_scale,
                                  slot_mapping)
    return q, k, v
