"""Fused q/k RMSNorm + RoPE + KV write on the GPU against oracle/qknorm.py.

Bitwise: q and k outputs, the pool bytes at the step's slots (bf16, or
E4M3FN codes and fp32 scales), and every other pool byte unchanged.  Shapes:
Qwen3-4B heads (32 q / 8 kv of 128) with the 1088-token step of the full-model
check, a few tokens, QKV rows that are a strided view, slot -1 padding,
positions at both ends of the table (and beyond it: clamped), GQA 8:2.  Then
the mixed attention step with the fused write (kv_stored=True) equals the
step that writes the same K/V with store_kvcache.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import qknorm
from slo_attn import (Attention, MixedAttentionContext, forward_mixed, qk_norm_rope_store, rope_cos_sin,
                      store_kvcache)

pytestmark = pytest.mark.gpu
HD = 128
EPS = 1e-6


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _case(n, hq, hkv, nblk, fp8, seed, strided=False, max_pos=40960):
    g = torch.Generator().manual_seed(seed)
    width = (hq + 2 * hkv) * HD
    pad = 256 if strided else 0
    qkv_full = (torch.randn(n, width + pad, generator=g) * 3).to(torch.bfloat16)
    qkv = qkv_full[:, :width]
    pos = torch.randint(0, max_pos, (n,), generator=g)
    if n >= 4:
        pos[0], pos[1], pos[2], pos[3] = 0, max_pos - 1, max_pos + 5, -3
    slots = torch.randperm(nblk * 256, generator=g)[:n].to(torch.int32)
    if n >= 6:
        slots[4] = slots[5] = -1
    qw = (1 + 0.2 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    if fp8:
        kc = torch.randint(0, 256, (nblk, 256, hkv, HD), generator=g, dtype=torch.uint8)
        kc[(kc & 0x7F) == 0x7F] = 0
        vc = kc.flip(0).clone()
        ks = torch.rand(nblk, 256, hkv, generator=g) + 0.5
        vs = ks.flip(0).clone()
    else:
        kc = torch.randn(nblk, 256, hkv, HD, generator=g).to(torch.bfloat16)
        vc = torch.randn(nblk, 256, hkv, HD, generator=g).to(torch.bfloat16)
        ks = vs = None
    return qkv_full, qkv, pos, slots, qw, kw, kc, vc, ks, vs


def _run(device, n, hq, hkv, nblk, fp8, seed, strided=False):
    qkv_full, qkv, pos, slots, qw, kw, kc, vc, ks, vs = _case(n, hq, hkv, nblk, fp8, seed, strided)
    table = rope_cos_sin(HD, 40960, 1e6, "cpu")
    dev = lambda t: None if t is None else t.to(device)  # noqa: E731
    qkv_d = qkv_full.to(device)[:, :qkv.shape[1]]
    kc_d, vc_d, ks_d, vs_d = dev(kc), dev(vc), dev(ks), dev(vs)
    q, k, v = qk_norm_rope_store(qkv_d, dev(pos), dev(qw), dev(kw), EPS, dev(table), hq, hkv, kc_d, vc_d,
                                 dev(slots), ks_d, vs_d)
    torch.cuda.synchronize()
    # oracle, on copies of the same pools
    kc_o, vc_o = (kc.numpy().copy(), vc.numpy().copy()) if fp8 else (_bits(kc).copy(), _bits(vc).copy())
    ks_o, vs_o = (ks.numpy().copy(), vs.numpy().copy()) if fp8 else (None, None)
    qo, ko, vo = qknorm.qkv_step_store(_bits(qkv), pos.numpy(), _bits(qw), _bits(kw), EPS, table.numpy(), hq, hkv,
                                       slots.numpy(), kc_o, vc_o, ks_o, vs_o)
    assert np.array_equal(_bits(q), qo), "q differs from the oracle"
    assert np.array_equal(_bits(k), ko), "k differs from the oracle"
    assert np.array_equal(_bits(v), vo)
    if fp8:
        assert np.array_equal(kc_d.cpu().numpy(), kc_o) and np.array_equal(vc_d.cpu().numpy(), vc_o), "E4M3FN codes"
        assert np.array_equal(ks_d.cpu().numpy().view(np.uint32), ks_o.view(np.uint32)), "k scales"
        assert np.array_equal(vs_d.cpu().numpy().view(np.uint32), vs_o.view(np.uint32)), "v scales"
    else:
        assert np.array_equal(_bits(kc_d), kc_o) and np.array_equal(_bits(vc_d), vc_o), "bf16 pool bytes"
    return q, k, v


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "e4m3fn"])
def test_qwen3_step_shape_bit_exact(device, fp8):
    _run(device, 1088, 32, 8, 8, fp8, seed=10)


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "e4m3fn"])
def test_small_strided_padded_gqa(device, fp8):
    _run(device, 7, 8, 2, 2, fp8, seed=11, strided=True)
    _run(device, 1, 32, 8, 1, fp8, seed=12)


def test_rejects_bad_arguments(device):
    qkv = torch.zeros(4, 48 * HD, dtype=torch.bfloat16, device=device)
    pos = torch.zeros(4, dtype=torch.int64, device=device)
    w = torch.ones(HD, dtype=torch.bfloat16, device=device)
    table = rope_cos_sin(HD, 16, 1e6, device)
    kc = torch.zeros(1, 256, 8, HD, dtype=torch.bfloat16, device=device)
    slots = torch.zeros(4, dtype=torch.int32, device=device)
    with pytest.raises(ValueError):
        qk_norm_rope_store(qkv, pos.to(torch.int32), w, w, EPS, table, 32, 8, kc, kc.clone(), slots)
    with pytest.raises(ValueError):
        qk_norm_rope_store(qkv[:, :-8], pos, w, w, EPS, table, 32, 8, kc, kc.clone(), slots)
    with pytest.raises(ValueError):
        qk_norm_rope_store(qkv, pos, w, w, EPS, table, 32, 8, kc.to(torch.uint8), kc.to(torch.uint8), slots)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        qk_norm_rope_store(qkv.cpu(), pos.cpu(), w.cpu(), w.cpu(), EPS, table.cpu(), 32, 8, kc.cpu(), kc.cpu(),
                           slots.cpu())


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "e4m3fn"])
def test_mixed_step_with_fused_write_equals_separate_write(device, fp8):
    # 3 decode rows (history 300, 17, 700) and one 40-token chunk after a 100-token prefix.
    g = torch.Generator().manual_seed(13)
    hq, hkv, nblk, bs = 32, 8, 12, 256
    hist = [300, 17, 700]
    tables = [[0, 1], [2], [3, 4, 5], [6]]
    n = len(hist) + 40
    slots = [t[h // bs] * bs + h % bs for t, h in zip(tables, hist)]
    slots += [tables[3][p // bs] * bs + p % bs for p in range(100, 140)]
    pos = torch.tensor(hist + list(range(100, 140)), dtype=torch.int64, device=device)
    qkv = (torch.randn(n, (hq + 2 * hkv) * HD, generator=g) * 2).to(torch.bfloat16).to(device)
    qw = (1 + 0.2 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(device)
    kw = (1 + 0.2 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(device)
    table = rope_cos_sin(HD, 4096, 1e6, device)
    if fp8:
        kc = torch.randint(0, 120, (nblk, bs, hkv, HD), generator=g, dtype=torch.uint8).to(device)
        vc = kc.flip(0).contiguous()
        ks = (torch.rand(nblk, bs, hkv, generator=g) * 0.01 + 0.001).to(device)
        vs = ks.flip(0).contiguous()
    else:
        kc = torch.randn(nblk, bs, hkv, HD, generator=g).to(torch.bfloat16).to(device)
        vc = torch.randn(nblk, bs, hkv, HD, generator=g).to(torch.bfloat16).to(device)
        ks = vs = None
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=device)  # noqa: E731
    meta = MixedAttentionContext(3, 40, i32([h + 1 for h in hist]), i32([t + [-1] * (3 - len(t)) for t in tables[:3]]),
                                 i32([0, 40]), i32([0, 140]), i32([tables[3]]), 40, 140, True)
    slot_t = i32(slots)
    pools = [(kc.clone(), vc.clone(), None if ks is None else ks.clone(), None if vs is None else vs.clone())
             for _ in range(2)]
    # fused write, then attention without a store
    q, k, v = qk_norm_rope_store(qkv, pos, qw, kw, EPS, table, hq, hkv, pools[0][0], pools[0][1], slot_t,
                                 pools[0][2], pools[0][3])
    noop = lambda *a: None  # noqa: E731
    out_fused = forward_mixed(q, k, v, pools[0][0], pools[0][1], _ctx(slot_t, meta), HD ** -0.5, noop,
                              pools[0][2], pools[0][3])
    # the same q/k/v written by store_kvcache inside forward_mixed
    out_sep = forward_mixed(q, k, v, pools[1][0], pools[1][1], _ctx(slot_t, meta), HD ** -0.5, store_kvcache,
                            pools[1][2], pools[1][3])
    torch.cuda.synchronize()
    for a, b in zip(pools[0], pools[1]):
        if a is not None:
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    assert torch.equal(out_fused.view(torch.int16), out_sep.view(torch.int16))
    # Attention.forward with kv_stored=True takes the same path
    from slo_attn import reset_context, set_context
    attn = Attention(hq, HD, HD ** -0.5, hkv)
    attn.k_cache, attn.v_cache = pools[0][0], pools[0][1]
    if fp8:
        attn.k_scale, attn.v_scale = pools[0][2], pools[0][3]
    set_context(False, slot_mapping=slot_t, mixed=meta)
    try:
        out_mod = attn(q, k, v, kv_stored=True)
    finally:
        reset_context()
    assert torch.equal(out_mod.view(torch.int16), out_fused.view(torch.int16))


def _ctx(slot_t, meta):
    from slo_attn.context import Context
    return Context(is_prefill=False, slot_mapping=slot_t, mixed=meta)
