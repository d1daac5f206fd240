"""Attention -- definition in fp32 (plain torch; CPU by default).

* ``dense_suffix_attention`` restates benchmarks/v1_validation/reference.py:7-23:
  GQA by repeating each kv head over its G query heads, scores scaled by
  ``scale`` (default head_dim**-0.5), causal mask aligned bottom-right (query i
  of nq sits at key position nk - nq + i), softmax in fp32.
* ``gather_pages`` restates reference.py:60-62 / layer_replay.py:40-47.
* ``varlen`` / ``decode`` restate reference.py:64-82 (the paged and contiguous
  flash-attn call shapes of nanovllm/layers/attention.py:68-78).
* ``mixed`` restates forward_mixed (nanovllm/layers/mixed_attention.py:29-57):
  decode rows [:d] through the paged decode, prefill rows [d:] through varlen
  over the pool when any prefill row has history, else over the contiguous new
  K/V, outputs concatenated decode-first.  The caller writes the KV first.

A decode row with zero keys (a padded graph row) yields zeros; the reference
leaves that output unspecified.  The definitions are device-agnostic torch, so a
full-model check can evaluate them on GPU-resident pools.  ``dtype`` (fp32 by
default, the reference's precision) selects the arithmetic type; fp64 serves as
an independent evaluation of the same definition that calibrates how far two
exact evaluations drift apart once their outputs are rounded to bf16.
"""
from __future__ import annotations

import math

import torch


def dense_suffix_attention(q, k, v, scale=None, dtype=torch.float32):
    if q.ndim != 3 or k.ndim != 3 or v.shape != k.shape:
        raise ValueError("expected [tokens, heads, dim] Q/K/V")
    nq, heads, dim = q.shape
    nk, kv_heads, kdim = k.shape
    if not 0 < nq <= nk or dim != kdim or heads % kv_heads:
        raise ValueError("invalid causal suffix / GQA shape")
    for x in (q, k, v):
        if not torch.isfinite(x).all():
            raise ValueError("nonfinite Q/K/V")
    group = heads // kv_heads
    qf = q.to(dtype).permute(1, 0, 2)                                  # [H, nq, D]
    kf = k.to(dtype).repeat_interleave(group, dim=1).permute(1, 2, 0)  # [H, D, nk]
    vf = v.to(dtype).repeat_interleave(group, dim=1).permute(1, 0, 2)  # [H, nk, D]
    s = torch.bmm(qf, kf.contiguous()) * (dim ** -0.5 if scale is None else scale)
    qpos = torch.arange(nk - nq, nk, device=q.device).view(nq, 1)
    kpos = torch.arange(nk, device=q.device).view(1, nk)
    s = s.masked_fill(kpos > qpos, -math.inf)
    out = torch.bmm(torch.softmax(s, dim=-1), vf.contiguous())     # [H, nq, D]
    return out.permute(1, 0, 2).contiguous()


def gather_pages(cache, table, length):
    if cache.ndim != 4 or length <= 0:
        raise ValueError("expected paged [pages, block, heads, dim] cache")
    block = cache.shape[1]
    pages = (length + block - 1) // block
    table = [int(x) for x in table[:pages]]
    if len(table) < pages or any(not 0 <= p < cache.shape[0] for p in table):
        raise ValueError("missing/out-of-range physical page")
    return cache[torch.tensor(table, dtype=torch.long, device=cache.device)].flatten(0, 1)[:length]


def decode(q, k_cache, v_cache, lens, tables, scale, dtype=torch.float32):
    """q [d, H, D]; returns [d, H, D] in ``dtype``."""
    outs = []
    for i, n in enumerate(int(x) for x in lens):
        if n == 0:
            outs.append(torch.zeros(q.shape[1:], dtype=dtype, device=q.device))
            continue
        outs.append(dense_suffix_attention(q[i:i + 1], gather_pages(k_cache, tables[i], n),
                                           gather_pages(v_cache, tables[i], n), scale, dtype)[0])
    return torch.stack(outs) if outs else torch.zeros((0,) + tuple(q.shape[1:]), dtype=dtype)


def varlen(q, k, v, cu_q, cu_k, scale, tables=None, dtype=torch.float32):
    """q [Tq, H, D]; k/v contiguous [Tk, Hkv, D] or paged pools when ``tables``."""
    cu_q = [int(x) for x in cu_q]
    cu_k = [int(x) for x in cu_k]
    outs = []
    for r in range(len(cu_q) - 1):
        a, b = cu_q[r], cu_q[r + 1]
        n = cu_k[r + 1] - cu_k[r]
        if tables is None:
            pk, pv = k[cu_k[r]:cu_k[r + 1]], v[cu_k[r]:cu_k[r + 1]]
        else:
            pk, pv = gather_pages(k, tables[r], n), gather_pages(v, tables[r], n)
        outs.append(dense_suffix_attention(q[a:b], pk, pv, scale, dtype))
    return torch.cat(outs)


def mixed(q, k, v, k_cache, v_cache, meta, scale, dtype=torch.float32):
    """Oracle of one mixed step after the KV write; ``meta`` holds host lists."""
    d = meta["num_decode"]
    parts = []
    if d:
        parts.append(decode(q[:d], k_cache, v_cache, meta["decode_lens"], meta["decode_tables"], scale, dtype))
    if meta["num_prefill_tokens"]:
        if meta["prefill_has_history"]:
            parts.append(varlen(q[d:], k_cache, v_cache, meta["prefill_cu_q"], meta["prefill_cu_k"],
                                scale, meta["prefill_tables"], dtype))
        else:
            parts.append(varlen(q[d:], k[d:], v[d:], meta["prefill_cu_q"], meta["prefill_cu_k"], scale,
                                dtype=dtype))
    return parts[0] if len(parts) == 1 else torch.cat(parts)
