"""Full Qwen3-4B mixed forward step with the HIP attention path as a drop-in.

Random-init bf16 weights (seed 4, N(0, 0.02), unit norm weights), 36 layers,
hidden 2560, 32 query / 8 kv heads of 128, SwiGLU 9728, vocab 151936, RoPE
theta 1e6.  Batch: 64 decode rows with end_pos uniform in [512, 4096] and one
1024-token prefill chunk without a cached prefix, all in one mixed step over a
pool of 681 blocks of 256 tokens whose cached prefixes are N(0, 1).  The same
model runs three times: with ``slo_attn.Attention`` in every layer, with the
oracle's attention in fp32 (the reference: store, decode and varlen of
nanovllm/layers/mixed_attention.py:29-57), and with the oracle evaluated in
fp64 (a control).  For the bf16 pool and for the E4M3FN pool with
per-(token, kv head) fp32 scales:

* greedy tokens.  With random weights the 151936 logits of a row are close to
  Gaussian, so the top two are often within one bf16 ulp of each other (the LM
  head's output is bf16); any change of rounding anywhere in the 36 layers then
  picks the other one.  The fp32 and fp64 evaluations of the same exact
  attention are such a change, so their logit difference is the noise floor
  ``tau`` of the check.  Every sampled row (the 64 decode rows and the chunk's
  last token, mixed_model_runner.py:115-126) must pick a token whose
  reference logit is within ``tau`` of the reference's maximum, which means
  the same greedy token wherever the reference's top-2 gap exceeds ``tau``,
  and our logits must stay within 2 tau of the reference's.
* every layer's KV write is bit-exact: the bytes at the step's slots are the
  oracle's store of the K/V that layer was given (E4M3FN codes and fp32 scales
  by ``oracle.fp8.quantize_kv``, evaluated over token slices in threads), and
  every other byte of the pool is unchanged.

The third case runs the HIP side with q/k RMSNorm, RoPE and the KV write fused
into one launch per layer (slo_attn.qk_norm_rope_store, Attention.forward with
kv_stored=True); the reference side keeps the reference's separate layers.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from qwen3_step import (Geometry, Pool, Qwen3, Recorder, ReferenceAttention, config4_batch,
                        quantize_kv, run_step, top2_gaps)
from slo_attn import Attention

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(device):
    m = Qwen3(Geometry(), device, seed=4)
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
    short = ref_logits.amax(dim=-1) - ref_logits.gather(1, tokens[:, None])[:, 0]
    dlog = (logits - ref_logits).abs().amax(dim=-1)
    rows = tokens.numel()
    print(f"sampled rows {rows}: greedy = reference in {(tokens == ref_tokens).sum().item()}, "
          f"= control in {(tokens == ctl_tokens).sum().item()}; control = reference in "
          f"{(ctl_tokens == ref_tokens).sum().item()}; noise floor tau {tau:.4f}; "
          f"rows with reference top-2 gap > tau {(gaps > tau).sum().item()}; "
          f"largest reference-logit shortfall of our token {short.max().item():.4f}; "
          f"logits max |ours - reference| {dlog.max().item():.4f}", flush=True)
    bad = (short > tau).nonzero().flatten().tolist()
    assert not bad, (f"rows {bad}: our greedy token's reference logit is {short[bad].tolist()} below the "
                     f"reference maximum, beyond the noise floor {tau}")
    assert dlog.max().item() <= 2 * tau, f"logits differ by {dlog.max().item()} (> 2 tau = {2 * tau})"

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
