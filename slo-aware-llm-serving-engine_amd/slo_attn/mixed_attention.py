"""V1 mixed step: one KV write and ONE ragged attention launch.

Mirrors nanovllm/layers/mixed_attention.py:15-57.  ``MixedAttentionContext``
keeps the reference's fields, order and defaults, so ``prepare_mixed``
(nanovllm/engine/mixed_model_runner.py:66-92) fills it unchanged.  Where the
reference issues flash_attn_with_kvcache on the decode rows ``[:d]``, then
flash_attn_varlen_func on the prefill rows ``[d:]`` and a ``torch.cat``, this
module issues a single HIP launch that writes both phases into one output.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .ops import check_store, foldable, paged_attention, store_kvcache


@dataclass
class MixedAttentionContext:
    num_decode: int
    num_prefill_tokens: int
    decode_lens: torch.Tensor | None
    decode_tables: torch.Tensor | None
    prefill_cu_q: torch.Tensor | None
    prefill_cu_k: torch.Tensor | None
    prefill_tables: torch.Tensor | None
    max_q: int
    max_k: int
    prefill_has_history: bool = True


def forward_mixed(q, k, v, k_cache, v_cache, context, scale, store_fn,
                  k_scale=None, v_scale=None, phases=_lib.PHASE_ALL):
    """Write all new K/V first, then attend: decode rows first, prefill after.

    Same arguments as the reference (mixed_attention.py:29).  ``k_scale`` /
    ``v_scale`` are the fp32 scale pools of an E4M3FN cache.  ``phases``
    restricts the launch to decode or prefill rows (the split mode that mirrors
    the reference's per-phase calls); rows of the other phase are left
    untouched in the returned tensor.
    """
    meta = context.mixed
    if not k_cache.numel() or not v_cache.numel():
        raise RuntimeError("mixed forward requires an allocated KV pool")
    # The library's own store runs inside the attention launch when the new
    # rows are contiguous and the step has decode rows (same result, one
    # launch less; a step without decode rows gets the store kernel first from
    # the same call, so that its long rows can split their keys over
    # 32-position blocks); any other store_fn runs first.  An E4M3FN pool folds it into pure decode steps only (with at
    # most 8 query heads per kv head): the launch then quantises each decode
    # row's newest token itself (16 rows of 64-1,024 tokens: 25.3 us, against
    # the store kernel and a 24.1 us launch).  With prefill rows the folded
    # E4M3FN launch measured slower than the store kernel and the launch: rows
    # reading the pool re-quantise their new tokens' tiles in every item (24
    # decode rows and two chunks, one after a 1,024-token prefix: 108 against
    # 72 us), and cold rows run in the E4M3FN instantiation, which spills
    # registers (4 cold rows: 134 against 107 us).
    fold = (store_fn is store_kvcache and phases == _lib.PHASE_ALL and foldable(k, v)
            and (k_scale is None or (q.shape[1] <= 8 * k.shape[1] and not meta.num_prefill_tokens)))
    if fold:
        check_store(k, v, k_cache, v_cache, context.slot_mapping, k_scale, v_scale)
    elif k_scale is None:
        store_fn(k, v, k_cache, v_cache, context.slot_mapping)
    else:
        store_fn(k, v, k_cache, v_cache, context.slot_mapping, k_scale, v_scale)
    d = meta.num_decode
    num_prefill = 0
    if meta.num_prefill_tokens:
        num_prefill = meta.prefill_cu_q.numel() - 1
    history = bool(meta.prefill_has_history)
    return paged_attention(
        q, k_cache, v_cache, scale, num_kv_heads=k.shape[1], k_scale=k_scale, v_scale=v_scale,
        num_decode=d, decode_lens=meta.decode_lens, decode_tables=meta.decode_tables,
        num_prefill=num_prefill, prefill_cu_q=meta.prefill_cu_q, prefill_cu_k=meta.prefill_cu_k,
        max_q=meta.max_q, max_k=meta.max_k,
        prefill_tables=meta.prefill_tables if history else None,
        k=None if history else k[d:], v=None if history else v[d:], phases=phases,
        store_slot_mapping=context.slot_mapping if fold else None, new_k=k if fold else None,
        new_v=v if fold else None)
