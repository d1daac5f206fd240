"""Drop-in ``Attention`` module and ``store_kvcache`` for the nano-vLLM engine.

Mirrors nanovllm/layers/attention.py:33-79: same constructor, attributes
(``num_heads``, ``head_dim``, ``scale``, ``num_kv_heads``, ``k_cache``,
``v_cache``) and ``forward(q, k, v)`` dispatch on the global ``Context``:

* ``context.mixed`` set -> ``forward_mixed`` (one KV write + one ragged launch);
* V0 prefill -> KV write, then causal varlen attention over the cache when
  ``block_tables`` is given (prefix cache), else over the contiguous new K/V;
* V0 decode -> KV write, then paged decode; returns ``[B, 1, Hq, D]`` like
  flash_attn_with_kvcache on ``q.unsqueeze(1)``.

Optional ``k_scale`` / ``v_scale`` attributes (fp32
``[num_blocks, block_size, num_kv_heads]``) select the E4M3FN pool when the
runner assigns uint8 / float8_e4m3fn ``k_cache`` / ``v_cache`` views.
``forward(q, k, v, kv_stored=True)`` skips the KV write, for callers whose
``qk_norm_rope_store`` already wrote this step's K/V into the pool.
"""
from __future__ import annotations

import torch
from torch import nn

from .context import get_context
from .mixed_attention import forward_mixed
from .ops import check_store, foldable, paged_attention, store_kvcache

__all__ = ["Attention", "store_kvcache"]


def _stored(*args):
    """store_fn for a step whose K/V are already in the pool."""


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.k_scale = self.v_scale = None

    def _scales(self):
        return () if self.k_scale is None else (self.k_scale, self.v_scale)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_stored: bool = False):
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        if context.mixed is not None:
            return forward_mixed(q, k, v, k_cache, v_cache, context, self.scale,
                                 _stored if kv_stored else store_kvcache, self.k_scale, self.v_scale)
        have_cache = bool(k_cache.numel() and v_cache.numel())
        # A bf16 pool is written inside the attention launch when the new rows
        # are contiguous (same result, one launch less); otherwise, and for an
        # E4M3FN pool, the store kernel runs first.
        fold = have_cache and not kv_stored and self.k_scale is None and foldable(k, v)
        if fold:
            check_store(k, v, k_cache, v_cache, context.slot_mapping)
        elif have_cache and not kv_stored:
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping, *self._scales())
        store = dict(store_slot_mapping=context.slot_mapping, new_k=k, new_v=v) if fold else {}
        if context.is_prefill:
            rows = context.cu_seqlens_q.numel() - 1
            paged = context.block_tables is not None
            pool = paged or fold
            return paged_attention(
                q, k_cache if pool else None, v_cache if pool else None, self.scale,
                num_kv_heads=self.num_kv_heads, k_scale=self.k_scale if paged else None,
                v_scale=self.v_scale if paged else None, num_prefill=rows,
                prefill_cu_q=context.cu_seqlens_q, prefill_cu_k=context.cu_seqlens_k,
                max_q=context.max_seqlen_q, max_k=context.max_seqlen_k,
                prefill_tables=context.block_tables, k=None if paged else k, v=None if paged else v, **store)
        o = paged_attention(
            q, k_cache, v_cache, self.scale, num_kv_heads=self.num_kv_heads,
            k_scale=self.k_scale, v_scale=self.v_scale, num_decode=q.shape[0],
            decode_lens=context.context_lens, decode_tables=context.block_tables, **store)
        return o.unsqueeze(1)
