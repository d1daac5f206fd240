"""The drop-in ``Attention.forward`` / ``Context`` contract on the GPU.

Covers the V0 branches of nanovllm/layers/attention.py:59-79 (prefill over
contiguous K/V, prefill over the pool with a prefix cache, decode returning
[B, 1, Hq, D]), the CUDA-graph padding contract of model_runner.py:206-210
(slot -1, context_len 0, -1 table padding, stale rows), graph capture and
replay of the mixed step, and the module attributes the runner assigns.
"""
import pytest
import torch

from attn_cases import assert_close_gate
from oracle import attention as oatt
from oracle import metadata
from slo_attn import Attention, MixedAttentionContext, reserve_workspace, reset_context, set_context

pytestmark = pytest.mark.gpu


def _module(device, hq=32, hkv=8, d=128, nblk=16, bs=256, fp8=False):
    attn = Attention(hq, d, d ** -0.5, hkv)
    assert attn.k_cache.numel() == 0 and attn.num_heads == hq and attn.num_kv_heads == hkv
    if fp8:
        attn.k_cache = torch.zeros(nblk, bs, hkv, d, dtype=torch.uint8, device=device)
        attn.v_cache = torch.zeros_like(attn.k_cache)
        attn.k_scale = torch.ones(nblk, bs, hkv, device=device)
        attn.v_scale = torch.ones(nblk, bs, hkv, device=device)
    else:
        attn.k_cache = torch.zeros(nblk, bs, hkv, d, dtype=torch.bfloat16, device=device)
        attn.v_cache = torch.zeros_like(attn.k_cache)
    return attn


def i32(x, device):
    return torch.tensor(x, dtype=torch.int32, device=device)


def test_v0_prefill_then_decode_roundtrip(device):
    # A cold prefill of two prompts (contiguous K/V), then a decode step that
    # reads the cached prompt through the pool.
    g = torch.Generator().manual_seed(5)
    lens, bs = [300, 77], 256
    tables = [[3, 7], [1]]
    attn = _module(device)
    T = sum(lens)
    q = torch.randn(T, 32, 128, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(T, 8, 128, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(T, 8, 128, generator=g).to(torch.bfloat16).to(device)
    slots = sum((metadata.expected_slots(t, 0, n, bs) for t, n in zip(tables, lens)), [])
    cu = i32([0, lens[0], T], device)
    set_context(True, cu, cu, max(lens), max(lens), i32(slots, device))
    out = attn(q, k, v)
    reset_context()
    want = oatt.varlen(q.float().cpu(), k.float().cpu(), v.float().cpu(), [0, lens[0], T], [0, lens[0], T],
                       128 ** -0.5)
    assert out.shape == (T, 32, 128)
    assert_close_gate(out, want)
    # decode one more token per sequence
    qd = torch.randn(2, 32, 128, generator=g).to(torch.bfloat16).to(device)
    kd = torch.randn(2, 8, 128, generator=g).to(torch.bfloat16).to(device)
    vd = torch.randn(2, 8, 128, generator=g).to(torch.bfloat16).to(device)
    dslots = [metadata.slot_of(t, n, bs) for t, n in zip(tables, lens)]
    set_context(False, slot_mapping=i32(dslots, device), context_lens=i32([n + 1 for n in lens], device),
                block_tables=i32(metadata.pad_tables(tables), device))
    o = attn(qd, kd, vd)
    reset_context()
    assert o.shape == (2, 1, 32, 128)
    kf, vf = attn.k_cache.float().cpu(), attn.v_cache.float().cpu()
    want = oatt.decode(qd.float().cpu(), kf, vf, [n + 1 for n in lens], metadata.pad_tables(tables), 128 ** -0.5)
    assert_close_gate(o.squeeze(1), want)


def test_v0_prefix_cache_prefill(device):
    # cu_seqlens_k > cu_seqlens_q -> block_tables set -> keys from the pool.
    g = torch.Generator().manual_seed(6)
    bs, tables = 256, [[4, 2, 9], [0]]
    cached, new = [512, 100], [40, 28]
    attn = _module(device)
    old = [torch.randn(c, 8, 128, generator=g).to(torch.bfloat16) for c in cached]
    for t, o_ in zip(tables, old):
        for p in range(o_.shape[0]):
            attn.k_cache[t[p // bs], p % bs] = o_[p].to(device)
            attn.v_cache[t[p // bs], p % bs] = (-o_[p]).to(device)
    T = sum(new)
    q = torch.randn(T, 32, 128, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(T, 8, 128, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(T, 8, 128, generator=g).to(torch.bfloat16).to(device)
    slots = sum((metadata.expected_slots(t, c, c + n, bs) for t, c, n in zip(tables, cached, new)), [])
    cu_q = [0, new[0], T]
    cu_k = [0, cached[0] + new[0], cached[0] + new[0] + cached[1] + new[1]]
    set_context(True, i32(cu_q, device), i32(cu_k, device), max(new), max(c + n for c, n in zip(cached, new)),
                i32(slots, device), None, i32(metadata.pad_tables(tables), device))
    out = attn(q, k, v)
    reset_context()
    want = oatt.varlen(q.float().cpu(), attn.k_cache.float().cpu(), attn.v_cache.float().cpu(), cu_q, cu_k,
                       128 ** -0.5, metadata.pad_tables(tables))
    assert_close_gate(out, want)


def test_graph_padding_rows_are_inert(device):
    # Decode graph buckets pad rows with slot -1, context_len 0 and stale or
    # -1 table rows (model_runner.py:206-210); live rows must be unaffected.
    g = torch.Generator().manual_seed(11)
    attn = _module(device, nblk=8)
    attn.k_cache.copy_(torch.randn(attn.k_cache.shape, generator=g).to(torch.bfloat16))
    attn.v_cache.copy_(torch.randn(attn.v_cache.shape, generator=g).to(torch.bfloat16))
    bs = 256
    live_lens, live_tables = [300, 5], [[6, 2], [5]]
    tables = live_tables + [[-1, -1], [1, 3]]  # a -1 row and a stale row
    lens = live_lens + [0, 0]
    slots = [metadata.slot_of(t, n - 1, bs) for t, n in zip(live_tables, live_lens)] + [-1, -1]
    q = torch.randn(4, 32, 128, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(4, 8, 128, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(4, 8, 128, generator=g).to(torch.bfloat16).to(device)
    before = attn.k_cache.clone()
    set_context(False, slot_mapping=i32(slots, device), context_lens=i32(lens, device),
                block_tables=i32(metadata.pad_tables(tables), device))
    o = attn(q, k, v).squeeze(1)
    reset_context()
    torch.cuda.synchronize()
    changed = (attn.k_cache != before).any(-1).any(-1).nonzero().tolist()
    assert sorted(map(tuple, changed)) == [(2, 43), (5, 4)]
    assert torch.isfinite(o.float()).all()
    assert (o[2:] == 0).all()
    want = oatt.decode(q[:2].float().cpu(), attn.k_cache.float().cpu(), attn.v_cache.float().cpu(), live_lens,
                       live_tables, 128 ** -0.5)
    assert_close_gate(o[:2], want)


@pytest.mark.parametrize("fp8", [False, True])
def test_mixed_step_graph_capture_replays(device, fp8):
    # Record store + attention into a graph with static buffers, replay it
    # several times with eager work in between, compare every replay to eager.
    from slo_attn import forward_mixed, store_kvcache
    from types import SimpleNamespace
    g = torch.Generator().manual_seed(12)
    bs, nblk = 256, 24
    attn = _module(device, nblk=nblk, fp8=fp8)
    dec_lens, dec_tables = [700, 1200, 90], [[3, 8, 1], [0, 9, 12, 4, 5], [7]]
    pre_hist, pre_cnt, pre_tables = [300], [150], [[10, 2]]
    nd, T = 3, 3 + 150
    slots = [metadata.slot_of(t, n - 1, bs) for t, n in zip(dec_tables, dec_lens)]
    slots += metadata.expected_slots(pre_tables[0], 300, 450, bs)
    meta = MixedAttentionContext(nd, 150, i32(dec_lens, device), i32(metadata.pad_tables(dec_tables), device),
                                 i32([0, 150], device), i32([0, 450], device), i32(pre_tables, device), 150, 450,
                                 True)
    ctx = SimpleNamespace(mixed=meta, slot_mapping=i32(slots, device))
    q = torch.randn(T, 32, 128, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(T, 8, 128, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(T, 8, 128, generator=g).to(torch.bfloat16).to(device)
    fill = torch.randn(attn.k_cache.shape, generator=g)
    if fp8:
        attn.k_cache.copy_((fill * 20).to(torch.int32).clamp(0, 120).to(torch.uint8))
        attn.v_cache.copy_((fill * 30).to(torch.int32).clamp(0, 125).to(torch.uint8))
        attn.k_scale.copy_(torch.rand(attn.k_scale.shape, generator=g))
        attn.v_scale.copy_(torch.rand(attn.v_scale.shape, generator=g))
    else:
        attn.k_cache.copy_(fill.to(torch.bfloat16))
        attn.v_cache.copy_((-fill).to(torch.bfloat16))
    reserve_workspace(device, nd, 8 * bs, 32, 8, 128)
    scales = (attn.k_scale, attn.v_scale) if fp8 else (None, None)
    eager = forward_mixed(q, k, v, attn.k_cache, attn.v_cache, ctx, attn.scale, store_kvcache, *scales)
    torch.cuda.synchronize()
    out = torch.empty_like(eager)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # warm-up on the capture stream
        out.copy_(forward_mixed(q, k, v, attn.k_cache, attn.v_cache, ctx, attn.scale, store_kvcache, *scales))
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out.copy_(forward_mixed(q, k, v, attn.k_cache, attn.v_cache, ctx, attn.scale, store_kvcache, *scales))
    for rep in range(4):
        out.zero_()
        junk = torch.randn(1024, 1024, device=device) @ torch.randn(1024, 1024, device=device)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from eager"
        del junk
