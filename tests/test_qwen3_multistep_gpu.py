"""Consecutive Qwen3-4B mixed steps through the captured step graph, tokens fed back.

Step 0 holds D decode rows (end positions uniform in [512, hi], seed 7) and
one cold C-token prefill chunk; in steps 1-3 every row, the chunk's included,
decodes its next token.  Two sizes, each on bf16 and E4M3FN pools: D = 16,
C = 256, hi = 2048, and the config-4 size (64 decode rows, end positions in
[512, 4096], a 1,024-token chunk).  So from step 1 on, each decode row reads as history
the K/V that the earlier steps of the same path wrote into the pool, and the
chunk's row reads the 256 keys that its prefill wrote.

* HIP path: ``slo_attn.MixedStepGraph`` over the full model (36 layers of
  ``slo_attn.Attention``, metadata built by ``slo_build_mixed_metadata``),
  captured once per pool and replayed every step.  An E4M3FN pool captures
  the second graph of ``exact_history`` for the cold chunk of step 0.
* Reference: the same model with the oracle's attention in fp32
  (``qwen3_step.ReferenceAttention``) run eagerly on its own copy of the pool.

Both paths take the reference's sampled tokens as the next step's inputs
(teacher forcing, as benchmarks/v1/check_v1.py:200-236 compares generated
rows), so every step compares the two on the same inputs.  Every step: each
sampled row's greedy token equals the reference's, and each row passes the
reference's numerics policy (benchmarks/v1/numerics.py:5-18).
"""
from __future__ import annotations

import pytest
import torch

from oracle import metadata
from qwen3_step import CONDITIONED, Batch, Geometry, Pool, Qwen3, ReferenceAttention, numerics_policy, run_step
from slo_attn import Attention, MixedStepBuffers, MixedStepGraph

pytestmark = pytest.mark.gpu

STEPS, BS = 4, 256


@pytest.fixture(scope="module")
def model(device):
    m = Qwen3(Geometry(**CONDITIONED), device, seed=4)
    yield m
    del m
    torch.cuda.empty_cache()


def _plan(vocab: int, D: int, C: int, hi: int):
    g = torch.Generator().manual_seed(7)
    lens0 = torch.randint(512, hi + 1, (D,), generator=g).tolist()
    first = [L - 1 for L in lens0] + [None]          # decode rows' step-0 positions; the chunk row
    need = [L - 1 + STEPS for L in lens0] + [C + STEPS]
    pages = [(n + BS - 1) // BS for n in need]
    num_blocks = sum(pages) + 4
    perm = torch.randperm(num_blocks, generator=g).tolist()
    tables, at = [], 0
    for n in pages:
        tables.append(perm[at:at + n])
        at += n
    ids0 = torch.randint(0, vocab, (D + C,), generator=g).tolist()
    return first, tables, ids0, num_blocks


@pytest.mark.parametrize("fp8,D,C,hi", [(False, 16, 256, 2048), (True, 16, 256, 2048), (False, 64, 1024, 4096),
                                        (True, 64, 1024, 4096)],
                         ids=["bf16", "e4m3fn", "bf16-config4-size", "e4m3fn-config4-size"])
def test_multistep_graph_matches_reference(device, model, fp8, D, C, hi):
    geom = model.geom
    hq, hkv, d, layers = geom.num_heads, geom.num_kv_heads, geom.head_dim, geom.num_layers
    first, tables, ids0, num_blocks = _plan(geom.vocab, D, C, hi)
    pool = Pool(geom, num_blocks, BS, device, fp8)
    ref_pool = pool.clone()
    width = max(len(t) for t in tables)

    mods = [Attention(hq, d, model.scale, hkv) for _ in range(layers)]
    pool.attach(mods)
    model.attn = mods
    buffers = MixedStepBuffers(D + 1, 1, D + 1 + C, width, BS, width * BS, device)
    graph = MixedStepGraph(buffers, lambda ids, pos: model.forward(ids, pos), exact_history=fp8)
    refs = [ReferenceAttention(hq, d, model.scale, hkv) for _ in range(layers)]

    ids = list(ids0)
    for step in range(STEPS):
        if step == 0:
            dstart = first[:D]
            prefill = [(0, C)]
            positions = dstart + list(range(C))
            sample = list(range(D)) + [buffers.dc + C - 1]
        else:
            dstart = [p + step for p in first[:D]] + [C - 1 + step]
            prefill = []
            positions = dstart
            sample = list(range(D + 1))
        slots = [metadata.slot_of(tables[b], p, BS) for b, p in enumerate(dstart)]
        if prefill:
            slots += [metadata.slot_of(tables[D], p, BS) for p in range(C)]
        batch = Batch([p + 1 for p in dstart], [n for _, n in prefill], [s for s, _ in prefill], tables, ids,
                      positions, slots, num_blocks, BS)
        with torch.inference_mode():
            model.attn = mods
            hidden = graph.run(dstart, prefill, tables, ids)
            logits = model.logits(hidden, torch.tensor(sample, dtype=torch.int64, device=device)).float()
        ref_logits, ref_tokens = run_step(model, batch, refs, ref_pool)
        torch.cuda.synchronize()
        ok, top1, rel, cos, max_abs = numerics_policy(logits, ref_logits)
        rows = ref_tokens.numel()
        print(f"{'e4m3fn' if fp8 else 'bf16'} step {step}: {len(dstart)} decode rows{' + chunk' if prefill else ''}, "
              f"greedy = reference in {int(top1.sum())}/{rows}, policy passed by {int(ok.sum())}/{rows} "
              f"(worst rel-L2 {rel.max().item():.4f}, cosine {cos.min().item():.6f})", flush=True)
        bad = (~top1).nonzero().flatten().tolist()
        assert not bad, f"step {step} rows {bad}: greedy tokens differ from the reference"
        bad = (~ok).nonzero().flatten().tolist()
        assert not bad, f"step {step} rows {bad} fail the reference's numerics policy"
        ids = ref_tokens.tolist()  # teacher forcing: the reference's tokens feed both paths
    del graph, buffers, pool, ref_pool, mods, refs
    torch.cuda.empty_cache()
