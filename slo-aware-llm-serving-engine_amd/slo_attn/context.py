"""Per-process attention metadata side channel.

Same contract as nanovllm/utils/context.py:5-28: the model runner publishes one
``Context`` per step with ``set_context`` and every ``Attention`` layer reads it
with ``get_context``.  Field names, order and meaning are kept so that runners
written for the reference set it unchanged:

* ``is_prefill``: V0 prefill step (else V0 decode) when ``mixed`` is None.
* ``cu_seqlens_q`` / ``cu_seqlens_k``: int32 device prefix sums of query / key
  lengths per sequence (V0 prefill).
* ``max_seqlen_q`` / ``max_seqlen_k``: host ints.
* ``slot_mapping``: int32 device, one slot per new token, -1 for padding.
* ``context_lens``: int32 device, keys per sequence (V0 decode).
* ``block_tables``: int32 device ``[rows, width]``, -1 padded.
* ``mixed``: a ``MixedAttentionContext`` for the V1 mixed step.

Like the reference, the global is not thread-safe; one Python thread per rank.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    mixed: object | None = None


_CURRENT = Context()


def get_context() -> Context:
    return _CURRENT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None, mixed=None) -> None:
    global _CURRENT
    _CURRENT = Context(is_prefill=is_prefill, cu_seqlens_q=cu_seqlens_q,
                       cu_seqlens_k=cu_seqlens_k, max_seqlen_q=max_seqlen_q,
                       max_seqlen_k=max_seqlen_k, slot_mapping=slot_mapping,
                       context_lens=context_lens, block_tables=block_tables, mixed=mixed)


def reset_context() -> None:
    global _CURRENT
    _CURRENT = Context()
