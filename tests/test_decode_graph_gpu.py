"""Pure-decode steps captured in HIP graphs exactly as the reference captures them.

ModelRunner.capture_cudagraph (nanovllm/engine/model_runner.py:223-257) captures
one graph per batch bucket bs in [1, 2, 4, 8, 16, 32, ..., 512] over shared
static tensors: input rows, slot_mapping, context_lens and block_tables
[max_bs, max_num_blocks] all zero at capture (so the capture's own KV writes go
to slot 0).  run_model (:196-212) replays the bucket >= bs after filling
slot_mapping with -1 then the live slots, zeroing context_lens then the live
lengths, and overwriting only block_tables[:bs, :width] - rows past bs and
columns past the step's width keep whatever earlier steps left there.

Here the captured module is ``slo_attn.Attention`` (V0 decode branch: the KV
write, then paged decode) for Qwen3-4B heads, max_model_len 4096 (16 blocks of
256).  Each replayed step is checked against the fp32 oracle on its live rows
(gate max-abs 2e-2, mean-abs 2e-3), the new tokens' pool bytes are checked
against the oracle's store, and rows past bs (length 0) must be zeros.
"""
import pytest
import torch

from attn_cases import assert_close_gate
from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import kvstore
from slo_attn import Attention, reserve_workspace, reset_context, set_context

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 32, 8, 128, 256
MAX_LEN = 4096
MAX_BLOCKS = MAX_LEN // BS  # 16
MAX_BS = 512
BUCKETS = [1, 2, 4, 8] + list(range(16, MAX_BS + 1, 16))


def _steps(g, num_blocks):
    """Replayed steps: live rows with lengths (new token included) and tables.
    Each row's last page is its own block; earlier pages are shared at random
    (read-only), so slots are unique per step as build_batch guarantees."""
    out = []
    for bs in (512, 500, 100, 13, 3):
        lens = torch.randint(1, MAX_LEN + 1, (bs,), generator=g).tolist()
        own = torch.randperm(num_blocks - 64, generator=g)[:bs].add(64).tolist()   # blocks 64+ are last pages
        tables = []
        for b, L in enumerate(lens):
            n = (L + BS - 1) // BS
            tables.append(torch.randint(0, 64, (n - 1,), generator=g).tolist() + [own[b]])
        out.append((lens, tables))
    return out


@pytest.mark.parametrize("kv", ["bf16", "fp8_e4m3fn"])
def test_decode_graphs_at_the_reference_buckets(device, kv):
    fp8 = kv != "bf16"
    g = torch.Generator().manual_seed(21)
    num_blocks = 64 + MAX_BS
    gd = torch.Generator(device=device).manual_seed(22)
    attn = Attention(HQ, D, D ** -0.5, HKV)
    shape = (num_blocks, BS, HKV, D)
    if fp8:  # cached values N(0, 1), stored as E4M3FN codes with per-(token, kv head) absmax scales
        pool = []
        for _ in range(2):
            x = torch.empty(shape, device=device).normal_(generator=gd)
            sc = x.abs().amax(-1) / 448
            pool.append((x / sc[..., None]).to(torch.float8_e4m3fn).view(torch.uint8))
            pool.append(sc)
        pool = [pool[0], pool[2], pool[1], pool[3]]
        attn.k_cache, attn.v_cache, attn.k_scale, attn.v_scale = pool
    else:
        pool = [torch.empty(shape, dtype=torch.bfloat16, device=device).normal_(generator=gd) for _ in range(2)]
        attn.k_cache, attn.v_cache = pool
    reserve_workspace(device, MAX_BS, MAX_LEN, HQ, HKV, D)

    # graph_vars of capture_cudagraph, all zero at capture
    q = torch.zeros(MAX_BS, HQ, D, dtype=torch.bfloat16, device=device)
    k = torch.zeros(MAX_BS, HKV, D, dtype=torch.bfloat16, device=device)
    v = torch.zeros(MAX_BS, HKV, D, dtype=torch.bfloat16, device=device)
    slot_mapping = torch.zeros(MAX_BS, dtype=torch.int32, device=device)
    context_lens = torch.zeros(MAX_BS, dtype=torch.int32, device=device)
    block_tables = torch.zeros(MAX_BS, MAX_BLOCKS, dtype=torch.int32, device=device)
    outputs = torch.zeros(MAX_BS, HQ * D, dtype=torch.bfloat16, device=device)
    graphs, mempool = {}, None
    for bs in reversed(BUCKETS):
        graph = torch.cuda.CUDAGraph()
        set_context(False, slot_mapping=slot_mapping[:bs], context_lens=context_lens[:bs],
                    block_tables=block_tables[:bs])
        outputs[:bs] = attn(q[:bs], k[:bs], v[:bs]).view(bs, -1)   # warmup
        with torch.cuda.graph(graph, mempool):
            outputs[:bs] = attn(q[:bs], k[:bs], v[:bs]).view(bs, -1)
        if mempool is None:
            mempool = graph.pool()
        graphs[bs] = graph
        torch.cuda.synchronize()
        reset_context()
    print(f"{kv}: captured {len(graphs)} decode graphs, buckets {BUCKETS[0]}..{BUCKETS[-1]}")
    # the oracle's copy of the pool, taken after the captures (which wrote slot 0, as the reference's do)
    host = [t.cpu() for t in pool]
    if fp8:
        kq, vq, ks, vs = (t.numpy() for t in host)
    else:
        kc, vc = host

    for step, (lens, tables) in enumerate(_steps(g, num_blocks)):
        bs = len(lens)
        bucket = next(x for x in BUCKETS if x >= bs)
        width = max(len(t) for t in tables)
        nq = torch.randn(bs, HQ, D, generator=g)
        nq = (nq / nq.square().mean(-1, keepdim=True).sqrt()).to(torch.bfloat16)
        nk = torch.randn(bs, HKV, D, generator=g).to(torch.bfloat16)
        nv = torch.randn(bs, HKV, D, generator=g).to(torch.bfloat16)
        slots = [t[(L - 1) // BS] * BS + (L - 1) % BS for t, L in zip(tables, lens)]
        padded = torch.full((bs, width), -1, dtype=torch.int32)
        for b, t in enumerate(tables):
            padded[b, :len(t)] = torch.tensor(t, dtype=torch.int32)
        # run_model's replay (model_runner.py:202-211)
        q[:bs], k[:bs], v[:bs] = nq.to(device), nk.to(device), nv.to(device)
        slot_mapping.fill_(-1)
        slot_mapping[:bs] = torch.tensor(slots, dtype=torch.int32, device=device)
        context_lens.zero_()
        context_lens[:bs] = torch.tensor(lens, dtype=torch.int32, device=device)
        block_tables[:bs, :width] = padded.to(device)
        graphs[bucket].replay()
        torch.cuda.synchronize()
        got = outputs[:bs].view(bs, HQ, D).cpu()

        # the oracle's store of the step's new tokens, then decode over the pool
        if fp8:
            kvstore.store_kvcache_fp8(nk.float().numpy(), nv.float().numpy(), kq, vq, ks, vs, slots)
            want_pools = (kq, vq, ks, vs)
            kf = torch.from_numpy(ofp8.dequantize_kv(kq, ks))
            vf = torch.from_numpy(ofp8.dequantize_kv(vq, vs))
        else:
            kvstore.store_kvcache(nk.view(torch.int16).numpy(), nv.view(torch.int16).numpy(),
                                  kc.view(torch.int16).numpy(), vc.view(torch.int16).numpy(), slots)
            want_pools = (kc, vc)
            kf, vf = kc, vc
        want = oatt.decode(nq.float(), kf, vf, lens, padded.tolist(), D ** -0.5)
        mx, mn = assert_close_gate(got, want)
        for a, b in zip(pool, want_pools):
            bb = b if isinstance(b, torch.Tensor) else torch.from_numpy(b)
            assert torch.equal(a.cpu().view(torch.uint8), bb.view(torch.uint8)), f"step {step}: pool bytes differ"
        if bucket > bs:
            assert torch.count_nonzero(outputs[bs:bucket]).item() == 0, "rows past bs must be zeros"
        print(f"{kv} step {step}: bs {bs} on bucket {bucket}, width {width}: max-abs {mx:.3e} mean-abs {mn:.3e}")
