"""The KV write folded into the attention launch (bf16 and E4M3FN pools).

``forward_mixed`` and ``Attention.forward`` run the library's own store inside
the attention launch: the launch writes the step's new K/V rows to their slots
and reads the new tokens from those rows instead of the pool.  The reference
order is store first, then attend (nanovllm/layers/mixed_attention.py:33-34,
nanovllm/layers/attention.py:66-67); these tests check that the folded launch
gives the same output and the same pool bytes, bit for bit, as that order run
as two launches (a ``store_fn`` that is not the library's own store takes the
two-launch path), on the benchmark workloads (decode rows, prefill rows with
and without history) and through the V0 branches, including slot -1 padding.
"""
import pytest
import torch

from slo_attn import (Attention, MixedAttentionContext, forward_mixed, reserve_workspace, reset_context,
                      set_context, store_kvcache)
import workloads
from slo_attn.ops import paged_attention
from types import SimpleNamespace

pytestmark = pytest.mark.gpu


def _two_launch_store(*args):
    store_kvcache(*args)


@pytest.mark.parametrize("index", [0, 1, 2, 3])
def test_forward_mixed_folded_store_equals_store_then_attend(device, index):
    w = workloads.config(index)
    d = workloads.to_device(w, device)
    ctx = SimpleNamespace(mixed=d["meta"], slot_mapping=d["slot_mapping"])
    q, k, v = d["q"], d["k"], d["v"]
    kc0, vc0 = w.k_cache.to(device), w.v_cache.to(device)
    if w.num_decode:
        reserve_workspace(device, w.num_decode, max(len(t) for t in w.decode_tables) * w.block_size, 32, 8, 128)
    kc1, vc1 = kc0.clone(), vc0.clone()
    ref = forward_mixed(q, k, v, kc0, vc0, ctx, w.scale, _two_launch_store)
    got = forward_mixed(q, k, v, kc1, vc1, ctx, w.scale, store_kvcache)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(kc1.view(torch.int16), kc0.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc0.view(torch.int16))


def _fp8_pools(w, device):
    """E4M3FN codes and scales of the workload's bf16 pool, written by the store kernel."""
    base_k, base_v = w.k_cache.to(device), w.v_cache.to(device)
    nblk, bs, hkv, dh = base_k.shape
    kc = torch.empty(nblk, bs, hkv, dh, dtype=torch.uint8, device=device)
    vc = torch.empty_like(kc)
    ks = torch.empty(nblk, bs, hkv, dtype=torch.float32, device=device)
    vs = torch.empty_like(ks)
    slots = torch.arange(nblk * bs, dtype=torch.int32, device=device)
    store_kvcache(base_k.view(-1, hkv, dh), base_v.view(-1, hkv, dh), kc, vc, slots, ks, vs)
    return kc, vc, ks, vs


def _fp8_fold_matches_store_then_attend(device, meta, slots, q, k, v, pools, scale, history):
    """The folded E4M3FN launch against the store kernel followed by the same
    launch: outputs, codes and scales bit for bit."""
    d = meta.num_decode
    nr = (meta.prefill_cu_q.numel() - 1) if meta.num_prefill_tokens else 0
    p1 = tuple(t.clone() for t in pools)

    def launch(kc, vc, ks, vs, **store):
        return paged_attention(
            q, kc, vc, scale, num_kv_heads=k.shape[1], k_scale=ks, v_scale=vs, num_decode=d,
            decode_lens=meta.decode_lens, decode_tables=meta.decode_tables, num_prefill=nr,
            prefill_cu_q=meta.prefill_cu_q, prefill_cu_k=meta.prefill_cu_k, max_q=meta.max_q, max_k=meta.max_k,
            prefill_tables=meta.prefill_tables if history else None, k=None if history else k[d:],
            v=None if history else v[d:], **store)
    store_kvcache(k, v, pools[0], pools[1], slots, pools[2], pools[3])
    ref = launch(*pools)
    got = launch(*p1, store_slot_mapping=slots, new_k=k, new_v=v)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    for a_, b_ in zip(p1, pools):
        assert torch.equal(a_.view(torch.uint8), b_.view(torch.uint8))


@pytest.mark.parametrize("index", [0, 1, 2, 3, 4])
def test_folded_fp8_store_equals_store_then_attend(device, index):
    # E4M3FN pool: the launch quantises the new rows as the store kernel does
    # (decode rows' newest tokens, prefill tiles of new tokens, the tile that
    # straddles a prefix, the write at the end) -- same codes, scales and
    # outputs, bit for bit, as the store kernel followed by the launch; with
    # the rows reading the pool (history) and, where the workload allows,
    # without.  forward_mixed folds pure decode steps.
    w = workloads.config(index)
    d = workloads.to_device(w, device)
    if w.num_decode:
        reserve_workspace(device, w.num_decode, max(len(t) for t in w.decode_tables) * w.block_size, 32, 8, 128)
    for history in ((True, False) if not w.has_history else (True,)):
        _fp8_fold_matches_store_then_attend(device, d["meta"], d["slot_mapping"], d["q"], d["k"], d["v"],
                                            _fp8_pools(w, device), w.scale, history)
    if not w.prefill_q:  # a pure decode step: forward_mixed takes the folded launch
        ctx = SimpleNamespace(mixed=d["meta"], slot_mapping=d["slot_mapping"])
        p0, p1 = _fp8_pools(w, device), _fp8_pools(w, device)
        ref = forward_mixed(d["q"], d["k"], d["v"], p0[0], p0[1], ctx, w.scale, _two_launch_store, p0[2], p0[3])
        got = forward_mixed(d["q"], d["k"], d["v"], p1[0], p1[1], ctx, w.scale, store_kvcache, p1[2], p1[3])
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
        for a_, b_ in zip(p1, p0):
            assert torch.equal(a_.view(torch.uint8), b_.view(torch.uint8))


def test_folded_fp8_store_on_small_blocks_and_straddled_prefixes(device):
    # 64-token blocks, prefixes inside a key tile (100, 700: the tile holding
    # the prefix end is written to the pool by each item before it is read)
    # and decode rows whose newest token sits at a 16/32-token step edge.
    from attn_cases import Case
    case = Case([31, 63, 300, 1000], [100, 700, 0], [45, 90, 33], bs=64, seed=21, kv_fp8=True)
    kc, vc = case.cpu_pools()
    codes, scales = case.fp8_pools(kc, vc)
    pools = tuple(torch.from_numpy(x.copy()).to(device) for x in (*codes, *scales))
    slots = torch.tensor(case.slots, dtype=torch.int32, device=device)
    _fp8_fold_matches_store_then_attend(device, case.meta(device), slots, case.q.to(device), case.k.to(device),
                                        case.v.to(device), pools, case.scale, True)


def test_folded_store_skips_padding_slots_and_matches_explicit_launch(device):
    # Decode rows of a captured batch: real rows, then padding rows (slot -1,
    # length 0).  The folded launch must leave every byte but the real slots
    # alone and give the outputs of store + attend.
    g = torch.Generator().manual_seed(9)
    hq, hkv, dh, bs, nblk = 32, 8, 128, 256, 6
    pool_k = torch.randn(nblk, bs, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    pool_v = torch.randn(nblk, bs, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    lens = [300, 1, 257, 0, 0]
    tables = torch.tensor([[0, 1, -1], [2, -1, -1], [3, 4, -1], [-1, -1, -1], [5, 5, 5]],
                          dtype=torch.int32, device=device)
    slots = torch.tensor([bs + 43, 2 * bs, 4 * bs + 0, -1, -1], dtype=torch.int32, device=device)
    B = len(lens)
    q = torch.randn(B, hq, dh, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(B, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(B, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    dl = torch.tensor(lens, dtype=torch.int32, device=device)
    reserve_workspace(device, B, 3 * bs, hq, hkv, dh)
    kc0, vc0 = pool_k.clone(), pool_v.clone()
    store_kvcache(k, v, kc0, vc0, slots)
    ref = paged_attention(q, kc0, vc0, dh ** -0.5, num_kv_heads=hkv, num_decode=B, decode_lens=dl,
                          decode_tables=tables)
    kc1, vc1 = pool_k.clone(), pool_v.clone()
    got = paged_attention(q, kc1, vc1, dh ** -0.5, num_kv_heads=hkv, num_decode=B, decode_lens=dl,
                          decode_tables=tables, store_slot_mapping=slots, new_k=k, new_v=v)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(kc1.view(torch.int16), kc0.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc0.view(torch.int16))


def test_v0_branches_fold_the_store(device):
    # Cold prefill, prefix-cache prefill and decode through Attention.forward
    # (bf16 pool: folded) against the same calls with the store run first and
    # kv_stored=True (two launches).
    g = torch.Generator().manual_seed(11)
    hq, hkv, dh, bs, nblk = 32, 8, 128, 256, 8
    a1 = Attention(hq, dh, dh ** -0.5, hkv)
    a2 = Attention(hq, dh, dh ** -0.5, hkv)
    base_k = torch.randn(nblk, bs, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    base_v = torch.randn(nblk, bs, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    a1.k_cache, a1.v_cache = base_k.clone(), base_v.clone()
    a2.k_cache, a2.v_cache = base_k.clone(), base_v.clone()

    def i32(x):
        return torch.tensor(x, dtype=torch.int32, device=device)

    def both(q, k, v, **ctx):
        set_context(**ctx)
        try:
            got = a1(q, k, v)
            store_kvcache(k, v, a2.k_cache, a2.v_cache, ctx["slot_mapping"])
            ref = a2(q, k, v, kv_stored=True)
        finally:
            reset_context()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
        assert torch.equal(a1.k_cache.view(torch.int16), a2.k_cache.view(torch.int16))
        assert torch.equal(a1.v_cache.view(torch.int16), a2.v_cache.view(torch.int16))

    # cold prefill: two prompts of 100 and 300 tokens in blocks 0 and 1-2
    lq = [100, 300]
    T = sum(lq)
    q = torch.randn(T, hq, dh, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(T, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(T, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    slots = list(range(0, 100)) + list(range(bs, bs + 300))
    both(q, k, v, is_prefill=True, cu_seqlens_q=i32([0, 100, T]), cu_seqlens_k=i32([0, 100, T]),
         max_seqlen_q=300, max_seqlen_k=300, slot_mapping=i32(slots))
    # prefix-cache prefill: row 0 has 256 cached tokens (block 3) + 60 new (block 4)
    q = torch.randn(60, hq, dh, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(60, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(60, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    both(q, k, v, is_prefill=True, cu_seqlens_q=i32([0, 60]), cu_seqlens_k=i32([0, 316]),
         max_seqlen_q=60, max_seqlen_k=316, slot_mapping=i32(list(range(4 * bs, 4 * bs + 60))),
         block_tables=i32([[3, 4]]))
    # decode: the two prompts' next tokens plus a padded row
    q = torch.randn(3, hq, dh, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(3, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(3, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    reserve_workspace(device, 3, 2 * bs, hq, hkv, dh)
    both(q, k, v, is_prefill=False, slot_mapping=i32([100, bs + 300, -1]), context_lens=i32([101, 301, 0]),
         block_tables=i32([[0, -1], [1, 2], [-1, -1]]))


def test_fold_rejects_wide_fp8_groups_and_bad_rows(device):
    # An E4M3FN pool with more than 8 query heads per kv head cannot carry the
    # write (forward_mixed then runs the store kernel first).
    hq, hkv, dh, bs = 16, 1, 128, 256
    q = torch.zeros(2, hq, dh, dtype=torch.bfloat16, device=device)
    k = torch.zeros(2, hkv, dh, dtype=torch.bfloat16, device=device)
    kc = torch.zeros(2, bs, hkv, dh, dtype=torch.uint8, device=device)
    sc = torch.ones(2, bs, hkv, device=device)
    dl = torch.tensor([1, 1], dtype=torch.int32, device=device)
    tb = torch.tensor([[0], [1]], dtype=torch.int32, device=device)
    slots = torch.tensor([0, bs], dtype=torch.int32, device=device)
    with pytest.raises(ValueError):
        paged_attention(q, kc, kc.clone(), 1.0, num_kv_heads=hkv, k_scale=sc, v_scale=sc.clone(), num_decode=2,
                        decode_lens=dl, decode_tables=tb, store_slot_mapping=slots, new_k=k, new_v=k)
    hq, hkv = 8, 2
    q = torch.zeros(2, hq, dh, dtype=torch.bfloat16, device=device)
    k = torch.zeros(2, hkv, dh, dtype=torch.bfloat16, device=device)
    kb = torch.zeros(2, bs, hkv, dh, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        paged_attention(q, kb, kb.clone(), 1.0, num_kv_heads=hkv, num_decode=2, decode_lens=dl, decode_tables=tb,
                        store_slot_mapping=slots[:1].contiguous(), new_k=k[:1], new_v=k[:1])


@pytest.mark.parametrize("prefixes", [(300, 77, 0), (64, 511, 1000)])
def test_folded_store_with_prefixes_inside_a_key_tile(device, prefixes):
    # Prefill rows whose cached prefix ends inside a 64-key tile (a chunked
    # prompt): that tile mixes pool keys and new keys; plus decode rows.  The
    # folded launch must equal the store followed by the attention launch.
    g = torch.Generator().manual_seed(13)
    hq, hkv, dh, bs, nblk = 32, 8, 128, 256, 24
    pool_k = torch.randn(nblk, bs, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    pool_v = torch.randn(nblk, bs, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    perm = torch.randperm(nblk, generator=g).tolist()
    chunks = [130, 45, 200]
    dec_lens = [700, 33]
    rows, tables, slots, nxt = [], [], [], 0

    def take(n_tokens):
        nonlocal nxt
        nb = (n_tokens + bs - 1) // bs
        t = perm[nxt:nxt + nb]
        nxt += nb
        return t

    dec_tables = []
    for L in dec_lens:
        t = take(L)
        dec_tables.append(t)
        slots.append(t[(L - 1) // bs] * bs + (L - 1) % bs)
    pf_tables = []
    for pfx, n in zip(prefixes, chunks):
        t = take(pfx + n)
        pf_tables.append(t)
        slots += [t[j // bs] * bs + j % bs for j in range(pfx, pfx + n)]
    width = max(len(t) for t in dec_tables + pf_tables)

    def pad(ts):
        return torch.tensor([t + [-1] * (width - len(t)) for t in ts], dtype=torch.int32, device=device)

    T = len(dec_lens) + sum(chunks)
    q = torch.randn(T, hq, dh, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(T, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(T, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    cu_q = [0]
    cu_k = [0]
    for pfx, n in zip(prefixes, chunks):
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + pfx + n)
    meta = MixedAttentionContext(len(dec_lens), sum(chunks), torch.tensor(dec_lens, dtype=torch.int32, device=device),
                                 pad(dec_tables), torch.tensor(cu_q, dtype=torch.int32, device=device),
                                 torch.tensor(cu_k, dtype=torch.int32, device=device), pad(pf_tables), max(chunks),
                                 max(p + n for p, n in zip(prefixes, chunks)), True)
    ctx = SimpleNamespace(mixed=meta, slot_mapping=torch.tensor(slots, dtype=torch.int32, device=device))
    reserve_workspace(device, len(dec_lens), width * bs, hq, hkv, dh)
    kc0, vc0 = pool_k.clone(), pool_v.clone()
    kc1, vc1 = pool_k.clone(), pool_v.clone()
    ref = forward_mixed(q, k, v, kc0, vc0, ctx, dh ** -0.5, _two_launch_store)
    got = forward_mixed(q, k, v, kc1, vc1, ctx, dh ** -0.5, store_kvcache)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(kc1.view(torch.int16), kc0.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc0.view(torch.int16))
    # strided new rows (a view of a fused projection) take the two-launch path
    wide = torch.randn(T, 3, hkv, dh, generator=g).to(torch.bfloat16).to(device)
    ks, vs = wide[:, 1], wide[:, 2]
    kc2, vc2 = pool_k.clone(), pool_v.clone()
    kc3, vc3 = pool_k.clone(), pool_v.clone()
    ref2 = forward_mixed(q, ks, vs, kc2, vc2, ctx, dh ** -0.5, _two_launch_store)
    got2 = forward_mixed(q, ks, vs, kc3, vc3, ctx, dh ** -0.5, store_kvcache)
    torch.cuda.synchronize()
    assert torch.equal(got2.view(torch.int16), ref2.view(torch.int16))
    assert torch.equal(kc3.view(torch.int16), kc2.view(torch.int16))
