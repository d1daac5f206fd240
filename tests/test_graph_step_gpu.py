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
  With an E4M3FN pool the step graph is captured twice (``exact_history``):
  a step whose prefill rows all start at position 0 replays the graph in which
  they attend to their new bf16 K/V, as the eager path and the reference's
  ``prefill_has_history`` rule do (mixed_model_runner.py:88); the first step of
  each run is such a step.
"""
import numpy as np
import pytest
import torch

from oracle import metadata
from qwen3_step import Geometry, Qwen3
from slo_attn import Attention, KVPool, MixedStepBuffers, MixedStepGraph, MixedAttentionContext, reset_context, \
    set_context

pytestmark = pytest.mark.gpu


def _rand_step(g, dc, pc, tc, width, bs, nblk, cold=False):
    d = int(torch.randint(0, dc + 1, (1,), generator=g))
    r = int(torch.randint(0, pc + 1, (1,), generator=g))
    if cold:  # a step whose prefill rows all start at position 0: at least two of them, with tokens
        r = max(r, min(pc, 2))
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
        n = int(torch.randint(1 if cold else 0, max(1, budget // max(r, 1)) + 1, (1,), generator=g))
        budget -= n
        s = int(torch.randint(0, width * bs - n - 1, (1,), generator=g)) if n and not cold else 0
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


def test_metadata_kernel_flat_offsets_kat(device):
    # tests/test_v1_state.py:88-101 through the metadata kernel: one decode row
    # at position 256 and the first 256-token chunk of a 513-token prompt.
    bs = 256
    tables = [[0, 1], [2, 3, 4]]
    buf = MixedStepBuffers(1, 1, 257, 3, bs, 3 * bs, device)
    buf.load([256], [(0, 256)], tables, list(range(257)))
    buf.build()
    torch.cuda.synchronize()
    pos = buf.positions.cpu().tolist()
    assert tuple(pos[:3]) == (256, 0, 1)
    cu = buf.cu_q.cpu().tolist()
    assert (0, 1) + tuple(1 + c for c in cu[1:]) == (0, 1, 257)
    assert buf.slot_mapping.cpu().tolist() == [256] + metadata.expected_slots(tables[1], 0, 256, bs)
    assert buf.decode_lens.cpu().tolist() == [257]


@pytest.mark.parametrize("kv", ["bf16", "fp8_e4m3fn"])
def test_graph_replays_equal_eager(device, kv):
    geom = Geometry(num_layers=2, hidden=256, num_heads=8, num_kv_heads=2, intermediate=512, vocab=1000,
                    max_position=4096)
    model = Qwen3(geom, device, seed=7)
    model.fused = True
    dc, pc, tc, width, bs, nblk = 6, 3, 256, 8, 64, 160
    g = torch.Generator().manual_seed(11)
    fp8 = kv != "bf16"

    def new_pool(src=None):
        pool = KVPool(geom.num_layers, nblk, bs, geom.num_kv_heads, geom.head_dim, kv, device)
        if src is not None:
            copy_pool(pool, src)
        return pool

    def copy_pool(dst, src):
        dst.kv.copy_(src.kv)
        if fp8:
            dst.scale.copy_(src.scale)

    def pools_equal(a, b):
        bits = torch.uint8 if fp8 else torch.int16
        return torch.equal(a.kv.view(bits), b.kv.view(bits)) and (
            not fp8 or torch.equal(a.scale.view(torch.int32), b.scale.view(torch.int32)))

    base = new_pool()
    x = torch.randn(base.kv.shape, generator=g)
    if fp8:  # E4M3FN codes of N(0, 1) values with unit scales
        base.kv.copy_(x.to(torch.float8_e4m3fn).view(torch.uint8))
    else:
        base.kv.copy_(x.to(torch.bfloat16))
    mods = [Attention(geom.num_heads, geom.head_dim, model.scale, geom.num_kv_heads) for _ in range(2)]
    model.attn = mods
    graph_pool = new_pool(base)
    graph_pool.attach(mods)
    buf = MixedStepBuffers(dc, pc, tc, width, bs, width * bs, device)
    buf.load([5], [(0, 3)], [[0], [1]], [1, 2, 3, 4])  # any step fits for the capture warmup
    step = MixedStepGraph(buf, lambda ids, pos: model.forward(ids, pos), exact_history=fp8)
    copy_pool(graph_pool, base)  # the warmup and capture wrote KV; start the replays from the base pool

    eager_buf = MixedStepBuffers(dc, pc, tc, width, bs, width * bs, device)
    eager_pool = new_pool(base)
    for trial in range(3):
        dstart, rows, tables = _rand_step(g, dc, pc, tc, width, bs, nblk, cold=trial == 0)
        d = len(dstart)
        n_tok = d + sum(n for _, n in rows)
        history = any(s0 > 0 for s0, n in rows if n) or not fp8
        ids = torch.randint(0, geom.vocab, (n_tok,), generator=g).tolist()
        out = step.run(dstart, rows, tables, ids).clone()
        # the same padded step, eagerly, on a pool in the same state
        before = new_pool(eager_pool)
        eager_pool.attach(mods)
        eager_buf.load(dstart, rows, tables, ids)
        eager_buf.build()
        eager_buf.set_context(history)
        try:
            want = model.forward(eager_buf.input_ids, eager_buf.positions)
        finally:
            reset_context()
        torch.cuda.synchronize()
        print(f"{kv} step {trial}: {d} decode rows, prefill rows {rows}, prefill_has_history={history}")
        assert torch.isfinite(out.float()).all(), "padding rows must stay finite"
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {trial} differs from eager"
        assert pools_equal(graph_pool, eager_pool)
        # the real tokens against the unpadded step (prepare_mixed metadata, eager)
        if n_tok:
            ref_pool = new_pool(before)
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
