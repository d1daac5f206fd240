"""KV pool sizing and block lifecycle (host logic, CPU tensors).

* kv_block_bytes: the bf16 case is the reference's block_bytes
  (nanovllm/engine/model_runner.py:112, mixed_model_runner.py:27-29); the
  E4M3FN case adds two fp32 scales per (token, kv head), which at head_dim 128
  is the 512 -> 264 bytes per token and kv head of docs/project_manual.md:548-556.
* num_kv_blocks: the reference formula (mixed_model_runner.py:30-33) on known
  numbers, with and without the block cap.
* attach: per-layer views in module order (mixed_model_runner.py:43-47), with
  scale views for E4M3FN pools; views alias the pool.
* copy_blocks / reset_blocks / snapshot / restore move codes and scales together.
"""
import pytest
import torch

from slo_attn import Attention, KVPool, kv_block_bytes, num_kv_blocks


def test_block_bytes():
    assert kv_block_bytes(36, 256, 8, 128, "bf16") == 2 * 36 * 256 * 8 * 128 * torch.bfloat16.itemsize
    per_token_head_bf16 = kv_block_bytes(1, 1, 1, 128, "bf16")
    per_token_head_fp8 = kv_block_bytes(1, 1, 1, 128, "fp8_e4m3fn")
    assert (per_token_head_bf16, per_token_head_fp8) == (512, 264)
    with pytest.raises(ValueError):
        kv_block_bytes(1, 1, 1, 128, "int4")


def test_num_blocks_formula():
    gib = 1 << 30
    bb = kv_block_bytes(36, 256, 8, 128, "bf16")
    n = num_kv_blocks(288 * gib, 20 * gib, 9 * gib, 8 * gib, 0.9, bb)
    assert n == int(288 * gib * 0.9 - 20 * gib - 9 * gib + 8 * gib) // bb
    assert num_kv_blocks(288 * gib, 20 * gib, 9 * gib, 8 * gib, 0.9, bb, cap=100) == 100
    fp8 = num_kv_blocks(288 * gib, 20 * gib, 9 * gib, 8 * gib, 0.9, kv_block_bytes(36, 256, 8, 128, "fp8_e4m3fn"))
    assert 1.9 < fp8 / n < 1.95


@pytest.mark.parametrize("fmt", ["bf16", "fp8_e4m3fn"])
def test_attach_and_lifecycle(fmt):
    pool = KVPool(3, 5, 16, 2, 128, fmt, device="cpu")
    layers = torch.nn.ModuleList([Attention(8, 128, 0.1, 2) for _ in range(3)])
    assert pool.attach(layers) == 3
    for l, m in enumerate(layers):
        assert m.k_cache.data_ptr() == pool.kv[0, l].data_ptr() and m.v_cache.data_ptr() == pool.kv[1, l].data_ptr()
        if fmt == "bf16":
            assert m.k_scale is None
        else:
            assert m.k_scale.data_ptr() == pool.scale[0, l].data_ptr()
    g = torch.Generator().manual_seed(0)
    if fmt == "bf16":
        pool.kv.copy_(torch.randn(pool.kv.shape, generator=g).to(torch.bfloat16))
    else:
        pool.kv.copy_(torch.randint(0, 126, pool.kv.shape, generator=g, dtype=torch.uint8))
        pool.scale.copy_(torch.rand(pool.scale.shape, generator=g))
    before = pool.snapshot([1, 3])
    pool.copy_blocks([1, 3], [4, 0])
    assert torch.equal(pool.kv[:, :, 4], pool.kv[:, :, 1]) and torch.equal(pool.kv[:, :, 0], pool.kv[:, :, 3])
    if pool.fp8:
        assert torch.equal(pool.scale[:, :, 4], pool.scale[:, :, 1])
    pool.reset_blocks([1, 3])
    assert (pool.kv[:, :, 1].float() == 0).all()
    if pool.fp8:
        assert (pool.scale[:, :, 3] == 1).all()
    pool.restore(before)
    assert torch.equal(pool.kv[:, :, 1], before["kv"][:, :, 0]) and torch.equal(pool.kv[:, :, 3], before["kv"][:, :, 1])
    with pytest.raises(ValueError):
        pool.copy_blocks([1], [1])
    with pytest.raises(ValueError):
        KVPool(1, 1, 16, 1, 128, "bf16", device="cpu").restore(before)
