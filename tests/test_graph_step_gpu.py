"""Mixed steps in HIP graphs with on-GPU metadata (slo_attn.graph).

* slo_build_mixed_metadata equals oracle.metadata.padded_step (build_batch's
  slot formula, prepare_mixed's decode_lens / cu_seqlens, padding inert) on
  buckets with unused decode rows, zero-token prefill rows, rows that fill the
  bucket exactly, and prefixes that cross block boundaries.
* A two-layer Qwen3-shaped model (8 query / 2 kv heads of 128, fused q/k
  norm + RoPE + KV write, one ragged attention launch per layer) is captured
  once per bucket, metadata launch included, and replayed for three different
  steps; every replay equals the same padded step run eagerly, bit for bit
  (hidden states and pool bytes), and its real tokens agree with an unpadded
  eager run of the step within bf16 GEMM noise (the GEMMs see more rows).
"""
import numpy as np
import pytest
import torch

from oracle import metadata
from qwen3_step import Geometry, Qwen3
from slo_attn import Attention, KVPool, MixedStepBuffers, MixedStepGraph, MixedAttentionContext, reset_context, \
    set_context

pytestmark = pytest.mark.gpu


def _rand_step(g, dc, pc, tc, width, bs, nblk):
    d = int(torch.randint(0, dc + 1, (1,), generator=g))
    r = int(torch.randint(0, pc + 1, (1,), generator=g))
    budget = tc - dc
    perm = torch.randperm(nblk, generator=g).tolist()
    tables, rows, at = [], [], 0
    dstart = []
    for _ in range(d):
        s = int(torch.randint(0, width * bs - 1, (1,), generator=g))
        n = s // bs + 1
        tables.append(perm[at:at + n]); at += n
        dstart.append(s)
    for i in range(r):
        n = int(torch.randint(0, max(1, budget // max(r, 1)) + 1, (1,), generator=g))
        budget -= n
        s = int(torch.randint(0, width * bs - n - 1, (1,), generator=g)) if n else 0
        k = (s + n + bs - 1) // bs if n else 1
        tables.append(perm[at:at + k]); at += k
        rows.append((s, n))
    return dstart, rows, tables


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_metadata_kernel_matches_oracle(device, seed):
    g = torch.Generator().manual_seed(seed)
    dc, pc, tc, width, bs = [(5, 3, 300, 6, 64), (0, 4, 128, 4, 256), (8, 0, 8, 5, 64), (3, 2, 40, 3, 16)][seed]
    buf = MixedStepBuffers(dc, pc, tc, width, bs, width * bs, device)
    for trial in range(3):
        dstart, rows, tables = _rand_step(g, dc, pc, tc, width, bs, 4096)
        ids = list(range(len(dstart) + sum(n for _, n in rows)))
        buf.load(dstart, rows, tables, ids)
        buf.build()
        torch.cuda.synchronize()
        starts = dstart + [0] * (dc - len(dstart)) + [s for s, _ in rows] + [0] * (pc - len(rows))
        toks = [1] * len(dstart) + [0] * (dc - len(dstart)) + [n for _, n in rows] + [0] * (pc - len(rows))
        tabs = tables[:len(dstart)] + [[]] * (dc - len(dstart)) + tables[len(dstart):] + [[]] * (pc - len(rows))
        want = metadata.padded_step(starts, toks, dc, pc, tc, tabs, bs)
        assert buf.positions.cpu().tolist() == want["positions"]
        assert buf.slot_mapping.cpu().tolist() == want["slot_mapping"]
        if dc:
            assert buf.decode_lens[:dc].cpu().tolist() == want["decode_lens"]
        assert buf.cu_q.cpu().tolist() == want["cu_seqlens_q"]
        assert buf.cu_k.cpu().tolist() == want["cu_seqlens_k"]
        assert buf.last_token.cpu().tolist() == want["last_token"]
        # the real rows agree with prepare_mixed's metadata (mixed_model_runner.py:66-92)
        m = metadata.mixed_metadata([s + 1 for s in dstart], tables[:len(dstart)], [s for s, _ in rows],
                                    [n for _, n in rows], tables[len(dstart):])
        assert want["decode_lens"][:len(dstart)] == m["decode_lens"]
        assert want["cu_seqlens_q"][:len(rows) + 1] == m["prefill_cu_q"]


def test_graph_replays_equal_eager(device):
    geom = Geometry(num_layers=2, hidden=256, num_heads=8, num_kv_heads=2, intermediate=512, vocab=1000,
                    max_position=4096)
    model = Qwen3(geom, device, seed=7)
    model.fused = True
    dc, pc, tc, width, bs, nblk = 6, 3, 256, 8, 64, 160
    g = torch.Generator().manual_seed(11)

    def fresh_pool():
        pool = KVPool(geom.num_layers, nblk, bs, geom.num_kv_heads, geom.head_dim, "bf16", device)
        pool.kv.copy_(torch.randn(pool.kv.shape, generator=g).to(torch.bfloat16))
        return pool

    base = fresh_pool()
    mods = [Attention(geom.num_heads, geom.head_dim, model.scale, geom.num_kv_heads) for _ in range(2)]
    model.attn = mods
    graph_pool = KVPool(geom.num_layers, nblk, bs, geom.num_kv_heads, geom.head_dim, "bf16", device)
    graph_pool.kv.copy_(base.kv)
    graph_pool.attach(mods)
    buf = MixedStepBuffers(dc, pc, tc, width, bs, width * bs, device)
    buf.load([5], [(0, 3)], [[0], [1]], [1, 2, 3, 4])  # any step fits for the capture warmup
    step = MixedStepGraph(buf, lambda ids, pos: model.forward(ids, pos))
    graph_pool.kv.copy_(base.kv)  # the warmup and capture wrote KV; start the replays from the base pool

    eager_buf = MixedStepBuffers(dc, pc, tc, width, bs, width * bs, device)
    eager_pool = KVPool(geom.num_layers, nblk, bs, geom.num_kv_heads, geom.head_dim, "bf16", device)
    eager_pool.kv.copy_(base.kv)
    for trial in range(3):
        dstart, rows, tables = _rand_step(g, dc, pc, tc, width, bs, nblk)
        d = len(dstart)
        n_tok = d + sum(n for _, n in rows)
        ids = torch.randint(0, geom.vocab, (n_tok,), generator=g).tolist()
        out = step.run(dstart, rows, tables, ids).clone()
        # the same padded step, eagerly, on a pool in the same state
        before = eager_pool.kv.clone()
        eager_pool.attach(mods)
        eager_buf.load(dstart, rows, tables, ids)
        eager_buf.build()
        eager_buf.set_context()
        try:
            want = model.forward(eager_buf.input_ids, eager_buf.positions)
        finally:
            reset_context()
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all(), "padding rows must stay finite"
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {trial} differs from eager"
        assert torch.equal(graph_pool.kv.view(torch.int16), eager_pool.kv.view(torch.int16))
        # the real tokens against the unpadded step (prepare_mixed metadata, eager)
        if n_tok:
            ref_pool = KVPool(geom.num_layers, nblk, bs, geom.num_kv_heads, geom.head_dim, "bf16", device)
            ref_pool.kv.copy_(before)
            ref_pool.attach(mods)
            m = metadata.mixed_metadata([s0 + 1 for s0 in dstart], tables[:d], [s0 for s0, _ in rows],
                                        [n for _, n in rows], tables[d:])
            pos = dstart + [s0 + i for s0, n in rows for i in range(n)]
            slots = [metadata.slot_of(t, p_, bs) for t, p_ in zip(tables[:d], dstart)]
            slots += [metadata.slot_of(tables[d + r], s0 + i, bs) for r, (s0, n) in enumerate(rows) for i in range(n)]
            i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=device)  # noqa: E731
            nr = len(rows)
            ctx = MixedAttentionContext(
                d, n_tok - d, i32(m["decode_lens"]) if d else None, i32(m["decode_tables"]) if d else None,
                i32(m["prefill_cu_q"]) if nr else None, i32(m["prefill_cu_k"]) if nr else None,
                i32(m["prefill_tables"]) if nr else None, m["max_q"], m["max_k"], m["prefill_has_history"])
            set_context(False, slot_mapping=i32(slots), mixed=ctx)
            try:
                ref = model.forward(torch.tensor(ids, device=device), torch.tensor(pos, device=device))
            finally:
                reset_context()
            real = list(range(d)) + list(range(dc, dc + n_tok - d))
            a, b_ = out[real].float(), ref.float()
            rel = ((a - b_).norm() / b_.norm()).item()
            assert rel < 2e-2, f"step {trial}: padded graph step and unpadded eager step differ by {rel:.3e}"
        graph_pool.attach(mods)
