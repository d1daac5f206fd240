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


def padded_step(row_start, row_tokens, decode_capacity, prefill_capacity, token_capacity, tables, block_size):
    """Capacity-padded metadata of one mixed step (host lists).

    Rows [0, Dc) are decode rows (1 token, 0 for an unused row), rows
    [Dc, Dc + Pc) prefill rows; token b is decode row b, token Dc + cu_q[r] + i
    is token i of prefill row r, at position start + i, with the slot formula
    of build_batch (batch_metadata.py:105); decode_lens holds end_pos
    (mixed_model_runner.py:83); cu_q / cu_k accumulate num_tokens / end_pos
    over prefill rows (:75-78), with 0 for a row without tokens; every other
    token has slot -1 and position 0.
    """
    dc, pc = decode_capacity, prefill_capacity

    def slot(row, pos):
        t = tables[row]
        idx = pos // block_size
        if pos < 0 or idx >= len(t) or t[idx] < 0:
            return -1
        return t[idx] * block_size + pos % block_size

    positions = [0] * token_capacity
    slots = [-1] * token_capacity
    decode_lens = [0] * dc
    last = [-1] * (dc + pc)
    for b in range(dc):
        if row_tokens[b] > 0:
            positions[b] = row_start[b]
            slots[b] = slot(b, row_start[b])
            decode_lens[b] = row_start[b] + 1
            last[b] = b
    cu_q, cu_k = [0], [0]
    for r in range(pc):
        n = max(row_tokens[dc + r], 0)
        for i in range(n):
            t = dc + cu_q[-1] + i
            if t < token_capacity:
                positions[t] = row_start[dc + r] + i
                slots[t] = slot(dc + r, row_start[dc + r] + i)
        if n:
            last[dc + r] = dc + cu_q[-1] + n - 1
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + (row_start[dc + r] + n if n else 0))
    return {"positions": positions, "slot_mapping": slots, "decode_lens": decode_lens,
            "cu_seqlens_q": cu_q, "cu_seqlens_k": cu_k, "last_token": last}
