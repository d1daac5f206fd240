"""Mixed steps in HIP graphs: capacity-padded buffers and on-GPU metadata.

The reference captures only pure-decode steps (nanovllm/engine/model_runner.py:
223-257, replayed by run_model :196-212) and runs every mixed step eagerly
(mixed_model_runner.py:112-114) with metadata built by Python loops and
copied to the device tensor by tensor (mixed_model_runner.py:58-92).  Here a
bucket of capacities (decode rows, prefill rows, tokens) owns static device
buffers; ``load`` sends the step's rows in one host-to-device copy (per row:
start position, new tokens and block table; plus the token ids), and the
captured step begins with ``slo_build_mixed_metadata``, which derives
positions, slots, decode lengths and cu_seqlens on the GPU.  Rows and tokens
beyond the step's are inert (slot -1, zero-length rows), so one graph serves
every batch that fits its bucket.  By default the prefill rows read their keys
from the pool (``prefill_has_history=True``): a bf16 pool holds exactly the
K/V a cold prefill would read from the new rows.  An E4M3FN pool holds their
quantised codes instead, so the reference's rule (the new rows unless some
prefill row has a cached prefix, mixed_model_runner.py:88 and
mixed_attention.py:45-54) needs a second captured graph for steps whose
prefill rows all start at position 0 (``MixedStepGraph(...,
exact_history=True)``).
"""
from __future__ import annotations

import torch

from . import _lib
from .context import reset_context, set_context
from .mixed_attention import MixedAttentionContext
from .ops import _ptr, _stream


class MixedStepBuffers:
    """Static buffers of one capacity bucket and its metadata launch."""

    def __init__(self, decode_capacity: int, prefill_capacity: int, token_capacity: int, table_width: int,
                 block_size: int, max_model_len: int, device):
        if token_capacity < decode_capacity:
            raise ValueError("token capacity must hold one token per decode row")
        self.dc, self.pc, self.tc = decode_capacity, prefill_capacity, token_capacity
        self.width, self.block_size, self.max_model_len = table_width, block_size, max_model_len
        self.device = torch.device(device)
        rows = decode_capacity + prefill_capacity
        # one host-to-device copy per step: [row_start | row_tokens | tables | input ids]
        self._host = torch.zeros(2 * rows + rows * table_width + token_capacity, dtype=torch.int64,
                                 pin_memory=True)
        self._packed = torch.zeros_like(self._host, device=self.device)
        p = self._packed
        self.row_start32 = torch.zeros(rows, dtype=torch.int32, device=self.device)
        self.row_tokens32 = torch.zeros(rows, dtype=torch.int32, device=self.device)
        self.tables = torch.full((rows, table_width), -1, dtype=torch.int32, device=self.device)
        self.input_ids = p[2 * rows + rows * table_width:]
        self.positions = torch.zeros(token_capacity, dtype=torch.int64, device=self.device)
        self.slot_mapping = torch.full((token_capacity,), -1, dtype=torch.int32, device=self.device)
        self.decode_lens = torch.zeros(max(decode_capacity, 1), dtype=torch.int32, device=self.device)
        self.cu_q = torch.zeros(prefill_capacity + 1, dtype=torch.int32, device=self.device)
        self.cu_k = torch.zeros(prefill_capacity + 1, dtype=torch.int32, device=self.device)
        self.last_token = torch.full((rows,), -1, dtype=torch.int32, device=self.device)
        self._copied = torch.cuda.Event()

    def load(self, decode_start: list[int], prefill_rows: list[tuple[int, int]], tables: list[list[int]],
             input_ids: list[int]) -> None:
        """Host rows of one step: decode rows' positions, prefill rows' (start, tokens),
        block tables (decode rows first) and the new tokens' ids in token order."""
        d, r = len(decode_start), len(prefill_rows)
        if d > self.dc or r > self.pc or d + sum(n for _, n in prefill_rows) > self.tc - (self.dc - d):
            raise ValueError("step does not fit this bucket")
        if len(tables) != d + r or any(len(t) > self.width for t in tables):
            raise ValueError("one block table per row, at most table_width entries")
        rows = self.dc + self.pc
        h = self._host
        self._copied.synchronize()  # the previous step's copy has left the pinned buffer
        h.zero_()
        start, tok = h[:rows], h[rows:2 * rows]
        tab = h[2 * rows:2 * rows + rows * self.width].view(rows, self.width)
        tab.fill_(-1)
        ids = h[2 * rows + rows * self.width:]
        for b, s in enumerate(decode_start):
            start[b], tok[b] = s, 1
            tab[b, :len(tables[b])] = torch.tensor(tables[b], dtype=torch.int64)
            ids[b] = input_ids[b]
        at = d
        for i, (s, n) in enumerate(prefill_rows):
            start[self.dc + i], tok[self.dc + i] = s, n
            tab[self.dc + i, :len(tables[d + i])] = torch.tensor(tables[d + i], dtype=torch.int64)
        ids[self.dc:self.dc + len(input_ids) - d] = torch.tensor(input_ids[d:], dtype=torch.int64)
        self._packed.copy_(h, non_blocking=True)
        self._copied.record()
        p = self._packed
        self.row_start32.copy_(p[:rows])
        self.row_tokens32.copy_(p[rows:2 * rows])
        self.tables.copy_(p[2 * rows:2 * rows + rows * self.width].view(rows, self.width))

    def build(self) -> None:
        """Derives the step's metadata on the GPU (capturable)."""
        _lib.check(_lib.load().slo_build_mixed_metadata(
            _ptr(self.row_start32), _ptr(self.row_tokens32), self.dc, self.pc, self.tc, _ptr(self.tables),
            self.width, self.width, self.block_size, _ptr(self.positions), _ptr(self.slot_mapping),
            _ptr(self.decode_lens) if self.dc else None, _ptr(self.cu_q), _ptr(self.cu_k), _ptr(self.last_token),
            _stream(self.device)), "slo_build_mixed_metadata")

    def set_context(self, history: bool = True) -> None:
        """Publishes the bucket's Context for the attention layers (context.py:21-28).

        ``history`` is ``prefill_has_history``: prefill rows read their keys
        from the pool (True) or from the step's new K/V rows (False, valid when
        every prefill row starts at position 0)."""
        meta = MixedAttentionContext(
            self.dc, self.tc - self.dc, self.decode_lens[:self.dc] if self.dc else None,
            self.tables[:self.dc] if self.dc else None, self.cu_q, self.cu_k, self.tables[self.dc:],
            self.tc - self.dc, self.max_model_len, history)
        set_context(False, slot_mapping=self.slot_mapping, mixed=meta)


class MixedStepGraph:
    """``fn(input_ids, positions)`` (one model forward over the bucket's tokens)
    captured together with the metadata launch; ``run`` loads a step and replays.

    With ``exact_history`` (required for E4M3FN pools) a second graph is
    captured for steps whose prefill rows all start at position 0, which then
    attend to their new K/V rows as the reference's ``prefill_has_history``
    rule says; ``run`` picks the graph from the host-known start positions.
    The two graphs share the bucket's buffers (and cost two graph memory
    pools)."""

    def __init__(self, buffers: MixedStepBuffers, fn, warmup: int = 1, exact_history: bool = False):
        self.buffers, self.fn = buffers, fn
        self.graphs, self.outputs = {}, {}
        for history in ((False, True) if exact_history else (True,)):
            s = torch.cuda.Stream(device=buffers.device)
            s.wait_stream(torch.cuda.current_stream(buffers.device))
            with torch.cuda.stream(s):
                for _ in range(warmup):
                    self._body(history)
            torch.cuda.current_stream(buffers.device).wait_stream(s)
            torch.cuda.synchronize(buffers.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self.outputs[history] = self._body(history)
            self.graphs[history] = graph
            reset_context()
        self.graph, self.output = self.graphs[True], self.outputs[True]

    def _body(self, history: bool = True):
        b = self.buffers
        b.build()
        b.set_context(history)
        try:
            return self.fn(b.input_ids, b.positions)
        finally:
            reset_context()

    def run(self, decode_start, prefill_rows, tables, input_ids) -> torch.Tensor:
        """Loads the step and replays its graph; returns the (static) output."""
        history = any(s > 0 for s, n in prefill_rows if n) if False in self.graphs else True
        self.buffers.load(decode_start, prefill_rows, tables, input_ids)
        self.graphs[history].replay()
        return self.outputs[history]
