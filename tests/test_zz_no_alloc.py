"""slo_paged_attention_noalloc (the entry point that allocates nothing) against
slo_paged_attention on the same inputs, through the C-ABI.

The two entry points run the same kernels; only the workspace differs (the
library's static per-GPU scratch instead of the caller's buffer), so outputs
and pool bytes must be identical bit for bit.  Two calls in a row with the
second on a smaller input check that the scratch's state carries nothing from
one call to the next; a launch too large for the scratch is refused with a
clear error before any work is queued.
"""
import ctypes

import pytest
import torch

import workloads
from slo_attn import _lib
from slo_attn.ops import _stream, paged_attention

pytestmark = pytest.mark.gpu


def _launch(w, dev, pools, noalloc, phases=_lib.PHASE_ALL, fold=False, kv_fp8=False):
    d = dev
    meta = d["meta"]
    kc, vc, ks, vs = pools
    out = torch.full_like(d["q"], 7.0)
    history = w.has_history or fold
    store = dict(store_slot_mapping=d["slot_mapping"], new_k=d["k"], new_v=d["v"]) if fold else {}
    paged_attention(
        d["q"], kc, vc, w.scale, num_kv_heads=d["k"].shape[1], k_scale=ks, v_scale=vs,
        num_decode=meta.num_decode, decode_lens=meta.decode_lens, decode_tables=meta.decode_tables,
        num_prefill=(meta.prefill_cu_q.numel() - 1) if meta.prefill_cu_q is not None else 0,
        prefill_cu_q=meta.prefill_cu_q, prefill_cu_k=meta.prefill_cu_k, max_q=meta.max_q, max_k=meta.max_k,
        prefill_tables=meta.prefill_tables if history else None,
        k=None if history else d["k"][w.num_decode:], v=None if history else d["v"][w.num_decode:],
        phases=phases, out=out, noalloc=noalloc, **store)
    return out


def _pools(w, device, kv_fp8):
    kc, vc = w.k_cache.to(device), w.v_cache.to(device)
    if not kv_fp8:
        return kc, vc, None, None
    from slo_attn import store_kvcache
    nblk, bs, hkv, d = kc.shape
    kq = torch.empty(nblk, bs, hkv, d, dtype=torch.uint8, device=device)
    vq = torch.empty_like(kq)
    ks = torch.empty(nblk, bs, hkv, dtype=torch.float32, device=device)
    vs = torch.empty_like(ks)
    slots = torch.arange(nblk * bs, dtype=torch.int32, device=device)
    store_kvcache(kc.view(-1, hkv, d), vc.view(-1, hkv, d), kq, vq, slots, ks, vs)
    return kq, vq, ks, vs


def _check_scratch(device):
    lib = _lib.load()
    _lib.check(lib.slo_attention_workspace_check(None, 0, None, _stream(device)), "slo_attention_workspace_check")


@pytest.mark.parametrize("first,second,kv_fp8,fold", [
    (3, 0, False, True),    # mixed step with the KV write folded in, then a smaller decode-only step
    (4, 3, False, False),   # 64 long decode rows + a 1,024 chunk, then the 24-row mixed step
    (2, 0, True, False),    # prefill-only after cached prefixes (split prefill items), E4M3FN pool
])
def test_noalloc_matches_the_workspace_entry_point(device, first, second, kv_fp8, fold):
    for index in (first, second):
        w = workloads.config(index)
        dev = workloads.to_device(w, device)
        base_pools = _pools(w, device, kv_fp8)
        twin_pools = tuple(None if t is None else t.clone() for t in base_pools)
        want = _launch(w, dev, base_pools, noalloc=False, fold=fold and not kv_fp8)
        got = _launch(w, dev, twin_pools, noalloc=True, fold=fold and not kv_fp8)
        torch.cuda.synchronize()
        print(f"config {index} (fp8={kv_fp8}, fold={fold}): static scratch and workspace launches compared")
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"config {index}: outputs differ"
        for a, b in zip(base_pools, twin_pools):
            if a is not None:
                assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"config {index}: pool bytes differ"
        _check_scratch(device)
        del base_pools, twin_pools, dev, w
        torch.cuda.empty_cache()


def test_noalloc_refuses_a_launch_larger_than_its_scratch(device):
    # 512 decode rows of up to 4,096 tokens: 512 x 32 x 8 records of 4 x 528
    # bytes = 277 MB of split-K partials, beyond the 64 MiB array
    rows, width = 512, 16
    q = torch.zeros(rows, 32, 128, dtype=torch.bfloat16, device=device)
    kc = torch.zeros(64, 256, 8, 128, dtype=torch.bfloat16, device=device)
    lens = torch.full((rows,), 300, dtype=torch.int32, device=device)
    tables = torch.zeros(rows, width, dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError, match="static scratch holds"):
        paged_attention(q, kc, kc, 0.1, num_kv_heads=8, num_decode=rows, decode_lens=lens, decode_tables=tables,
                        out=torch.empty_like(q), noalloc=True)
    # the same launch with a caller workspace runs
    paged_attention(q, kc, kc, 0.1, num_kv_heads=8, num_decode=rows, decode_lens=lens, decode_tables=tables)
    torch.cuda.synchronize()
    _check_scratch(device)


def test_noalloc_refuses_a_workspace_argument(device):
    args = _lib.PagedAttentionArgs()
    args.head_dim, args.num_heads, args.num_kv_heads, args.phases = 128, 32, 8, 3
    args.workspace, args.workspace_bytes = 256, 1 << 20
    rc = _lib.load().slo_paged_attention_noalloc(ctypes.byref(args), None)
    assert rc == 1 and "workspace must be NULL" in _lib.load().slo_last_error().decode()
