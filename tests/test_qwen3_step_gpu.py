"""Full Qwen3-4B mixed forward step with the HIP attention path as a drop-in.

Random-init bf16 weights (seed 4), 36 layers, hidden 2560, 32 query / 8 kv
heads of 128, SwiGLU 9728, vocab 151936, RoPE theta 1e6, tied LM head, with
the residual-branch conditioning of ``qwen3_step.CONDITIONED`` (o_proj and
down_proj scaled down so that every row's greedy token is decided by a clear
margin; see there).  Batch: 64 decode rows with end_pos uniform in [512, 4096]
and one 1024-token prefill chunk without a cached prefix, all in one mixed step
over a pool of 681 blocks of 256 tokens whose cached prefixes are N(0, 1).  The
same model runs three times: with ``slo_attn.Attention`` in every layer, with
the oracle's attention in fp32 (the reference: store, decode and varlen of
nanovllm/layers/mixed_attention.py:29-57), and with the oracle in fp64 (a
control).  For the bf16 pool, the E4M3FN pool with per-(token, kv head) fp32
scales, and the E4M3FN pool with the fused q/k norm + RoPE + KV write:

* greedy tokens: every sampled row (the 64 decode rows and the chunk's last
  token, mixed_model_runner.py:115-126) picks the reference's token (100%), and
  the fp64 control picks it too; the smallest top-2 margin of the reference and
  the fp32-vs-fp64 noise floor ``tau`` are printed, and the margin must exceed
  ``tau``.
* the reference's acceptance rule on every row's fp32 logits
  (benchmarks/v1/numerics.py:5-18 as check_v1.py:216-236 applies it): top-1
  match, relative L2 <= 0.02, cosine >= 0.999, max-abs <= 0.5.
* every layer's KV write is bit-exact: the bytes at the step's slots are the
  oracle's store of the K/V that layer was given (E4M3FN codes and fp32 scales
  by ``oracle.fp8.quantize_kv``, evaluated over token slices in threads), and
  every other byte of the pool is unchanged.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from qwen3_step import (CONDITIONED, Geometry, Pool, Qwen3, Recorder, ReferenceAttention, config4_batch,
                        numerics_policy, quantize_kv, run_step, top2_gaps)
from slo_attn import Attention

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(device):
    m = Qwen3(Geometry(**CONDITIONED), device, seed=4)
    yield m
    del m
    torch.cuda.empty_cache()


def _rows(t: torch.Tensor, width: int, slots: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1, width)[slots]


@pytest.mark.parametrize("fp8,fused", [(False, False), (True, False), (True, True)],
                         ids=["bf16", "e4m3fn", "e4m3fn-fused-qk-norm-rope-store"])
def test_qwen3_4b_mixed_step_greedy_and_kv_bytes(device, model, fp8, fused):
    geom = model.geom
    hq, hkv, d, layers = geom.num_heads, geom.num_kv_heads, geom.head_dim, geom.num_layers
    batch = config4_batch(geom.vocab)
    print(f"qwen3-4b step: {batch.num_decode} decode rows (sum end_pos {sum(batch.decode_lens)}), "
          f"chunk {batch.prefill_count[0]}, pool {'e4m3fn' if fp8 else 'bf16'}", flush=True)
    pool = Pool(geom, batch.num_blocks, batch.block_size, device, fp8)
    ref_pool, ctl_pool = pool.clone(), pool.clone()

    ours = [Recorder(Attention(hq, d, model.scale, hkv)) for _ in range(layers)]
    model.fused = fused
    try:
        logits, tokens = run_step(model, batch, ours, pool)
    finally:
        model.fused = False
    torch.cuda.synchronize()
    print("HIP-path step done", flush=True)
    ref = [ReferenceAttention(hq, d, model.scale, hkv) for _ in range(layers)]
    ref_logits, ref_tokens = run_step(model, batch, ref, ref_pool)
    ctl = [ReferenceAttention(hq, d, model.scale, hkv, torch.float64) for _ in range(layers)]
    ctl_logits, ctl_tokens = run_step(model, batch, ctl, ctl_pool)
    torch.cuda.synchronize()
    print("reference (fp32) and control (fp64) steps done", flush=True)
    del ctl_pool, ctl

    tau = (ref_logits - ctl_logits).abs().max().item()
    gaps = top2_gaps(ref_logits)
    rows = tokens.numel()
    # the reference's acceptance rule, row by row (numerics.py:5-18, check_v1.py:216-236)
    ok, top1, rel, cos, max_abs = numerics_policy(logits, ref_logits)
    print(f"sampled rows {rows}: greedy = reference in {int(top1.sum())}/{rows}, control (fp64) = reference in "
          f"{int((ctl_tokens == ref_tokens).sum())}/{rows}; smallest reference top-2 margin {gaps.min().item():.3f}, "
          f"noise floor tau {tau:.4f}; reference policy passed by {int(ok.sum())}/{rows} rows "
          f"(worst rel-L2 {rel.max().item():.4f}, cosine {cos.min().item():.6f}, max-abs {max_abs.max().item():.4f})",
          flush=True)
    assert torch.equal(ctl_tokens, ref_tokens), "the fp64 control disagrees with the fp32 reference (conditioning)"
    assert gaps.min().item() > tau, f"top-2 margin {gaps.min().item()} within the noise floor {tau}"
    bad = (~top1).nonzero().flatten().tolist()
    assert not bad, f"rows {bad}: greedy tokens {tokens[bad].tolist()} differ from the reference's {ref_tokens[bad].tolist()}"
    bad = (~ok).nonzero().flatten().tolist()
    assert not bad, (f"rows {bad} fail the reference's numerics policy: rel-L2 {rel[bad].tolist()}, cosine "
                     f"{cos[bad].tolist()}, max-abs {max_abs[bad].tolist()}")

    slots = torch.tensor(batch.slots, dtype=torch.long, device=device)
    n = slots.numel()
    for l in range(layers):
        k, v = ours[l].seen[0]
        for i, x in ((0, k), (1, v)):
            got = _rows(pool.kv[i, l], hkv * d, slots)
            if not fp8:
                assert torch.equal(got.view(torch.int16), x.reshape(n, -1).view(torch.int16)), \
                    f"layer {l} {'kv'[i]}: bf16 rows differ from the new K/V"
                continue
            codes, scales = quantize_kv(x.float().cpu().numpy())
            np.testing.assert_array_equal(got.cpu().numpy(), codes.reshape(n, -1),
                                          err_msg=f"layer {l} {'kv'[i]}: E4M3FN codes")
            got_s = _rows(pool.scale[i, l], hkv, slots).cpu().numpy()
            np.testing.assert_array_equal(got_s.view(np.uint32), scales.view(np.uint32),
                                          err_msg=f"layer {l} {'kv'[i]}: fp32 scales")

    # Every byte outside the step's slots is unchanged: give the reference pool
    # (same initial bytes, written at the same slots) our rows and compare whole pools.
    for i in range(2):
        for l in range(layers):
            ref_pool.kv[i, l].view(-1, hkv * d)[slots] = pool.kv[i, l].view(-1, hkv * d)[slots]
            if fp8:
                ref_pool.scale[i, l].view(-1, hkv)[slots] = pool.scale[i, l].view(-1, hkv)[slots]
    bits = torch.uint8 if fp8 else torch.int16
    assert torch.equal(pool.kv.view(bits), ref_pool.kv.view(bits))
    if fp8:
        assert torch.equal(pool.scale.view(torch.int32), ref_pool.scale.view(torch.int32))
    del pool, ref_pool, ours, ref
    torch.cuda.empty_cache()
