"""Slot and per-row metadata -- CPU definition.

* ``slot_of`` is the slot formula of build_batch
  (nanovllm/engine/batch_metadata.py:105): table[pos // bs] * bs + pos % bs.
* ``expected_slots`` restates benchmarks/v1_diagnostics/layer_replay.py:32-37.
* ``mixed_metadata`` restates what prepare_mixed
  (nanovllm/engine/mixed_model_runner.py:66-92) hands to the attention layer:
  decode lengths (= end_pos), -1 padded tables (:62-64), cu_q over scheduled
  tokens, cu_k over end_pos, max_q, max_k and prefill_has_history (:88).
"""
from __future__ import annotations


def slot_of(table, pos: int, block_size: int) -> int:
    return table[pos // block_size] * block_size + pos % block_size


def expected_slots(table, start: int, end: int, block_size: int) -> list[int]:
    if not 0 <= start < end or block_size <= 0 or len(table) * block_size < end:
        raise ValueError("invalid logical span/table")
    if any(p < 0 for p in table):
        raise ValueError("negative page")
    return [slot_of(table, p, block_size) for p in range(start, end)]


def pad_tables(rows):
    width = max(len(r) for r in rows)
    return [list(r) + [-1] * (width - len(r)) for r in rows]


def mixed_metadata(decode_end_pos, decode_tables, prefill_start, prefill_count, prefill_tables):
    """Host lists of the mixed step's attention metadata."""
    cu_q, cu_k = [0], [0]
    for s, n in zip(prefill_start, prefill_count):
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + s + n)
    return {
        "num_decode": len(decode_end_pos),
        "num_prefill_tokens": sum(prefill_count),
        "decode_lens": list(decode_end_pos),
        "decode_tables": pad_tables(decode_tables) if decode_tables else None,
        "prefill_cu_q": cu_q,
        "prefill_cu_k": cu_k,
        "prefill_tables": pad_tables(prefill_tables) if prefill_tables else None,
        "max_q": max(prefill_count) if prefill_count else 0,
        "max_k": max(s + n for s, n in zip(prefill_start, prefill_count)) if prefill_count else 0,
        "prefill_has_history": any(s > 0 for s in prefill_start),
    }
