"""Ragged mixed paged attention on the GPU vs the fp32 oracle.

Gate (from the benchmark definition): max-abs <= 2e-2 and mean-abs <= 2e-3
against the fp32 CPU oracle, for bf16 and E4M3FN pools (the oracle attends to
the same quantised bytes, dequantised in fp32).  The KV writes inside each step
are compared byte for byte.

The first cases reproduce the reference's own GPU suites
(tests/test_v1_attention_gpu.py:42-142, tests/test_v1_reference_gpu.py:10-66)
with the oracle in place of flash-attn; the rest cover the benchmark
configurations at full size, page/tile boundaries, padded rows, GQA ratios,
split launches and determinism.
"""
import pytest
import torch

from attn_cases import Case, assert_close_gate, pool_bytes_equal

pytestmark = pytest.mark.gpu


def _check(case, device, phases=3):
    got, gpu_pools = case.run_gpu(device, phases)
    torch.cuda.synchronize()
    want, cpu_pools = case.oracle()
    assert pool_bytes_equal(gpu_pools, cpu_pools), "KV pool bytes differ from the oracle write"
    return assert_close_gate(got, want), got, want


# --------------------------------------------- reference suite shapes
@pytest.mark.parametrize("kv_fp8", [False, True])
def test_gqa_paged_mixed_and_page_reuse(device, kv_fp8):
    # test_v1_attention_gpu.py:42-81: 8:2 GQA, decode history 256+1, prefill
    # cached 255 + 3-token chunk, reversed physical pages, then page reuse.
    for round_id, tables in enumerate(([[3, 1], [2, 0]], [[0, 2], [1, 3]])):
        case = Case([256], [255], [3], hq=8, hkv=2, seed=41 + round_id, kv_fp8=kv_fp8, tables=tables,
                    num_blocks=4)
        _check(case, device)


def test_cold_prefill_uses_contiguous_kv_and_writes_exact_bytes(device):
    # test_v1_attention_gpu.py:83-104: no history, contiguous K/V, cache bytes exact.
    case = Case([], [0], [256], hq=8, hkv=2, seed=42, tables=[[1]], num_blocks=2)
    assert case.meta_host["prefill_has_history"] is False
    _check(case, device)


@pytest.mark.parametrize("kv_fp8", [False, True])
def test_multiple_prefill_rows_with_different_cached_lengths(device, kv_fp8):
    # test_v1_attention_gpu.py:106-142: lengths [1,255,257,513], histories
    # [256,0,256,513], permuted pages; row 0 is the decode row.
    lengths, histories = [1, 255, 257, 513], [256, 0, 256, 513]
    physical = iter([13, 2, 11, 4, 14, 0, 9, 1, 12, 7, 5])
    tables = [[next(physical) for _ in range((h + n + 255) // 256)] for h, n in zip(histories, lengths)]
    case = Case([histories[0]], histories[1:], lengths[1:], hq=8, hkv=2, seed=43, kv_fp8=kv_fp8,
                tables=tables, num_blocks=16)
    _check(case, device)


@pytest.mark.parametrize("kv_fp8", [False, True])
def test_real_gqa_mixed_rows_and_page_reuse(device, kv_fp8):
    # test_v1_reference_gpu.py:10-45: Qwen3-4B geometry, histories [256,249,0],
    # counts [1,8,17], two rounds with page reuse, sentinels 19/-23.
    for round_id, tables in enumerate(([[5, 1], [3, 0], [2]], [[0, 4], [1, 5], [3]])):
        case = Case([256], [249, 0], [8, 17], seed=101 + round_id, kv_fp8=kv_fp8, tables=tables,
                    num_blocks=6, sentinel=(19.0, -23.0))
        _check(case, device)


def test_corrupt_old_values_are_detected(device):
    # test_v1_reference_gpu.py:47-66: a corrupted cached V must fail the gate.
    from types import SimpleNamespace
    from oracle import attention as oatt
    from slo_attn import MixedAttentionContext, forward_mixed, store_kvcache

    def i32(x):
        return torch.tensor(x, device=device, dtype=torch.int32)
    q = torch.zeros(8, 32, 128, device=device, dtype=torch.bfloat16)
    k = torch.zeros(8, 8, 128, device=device, dtype=torch.bfloat16)
    v = torch.full_like(k, 2.0)
    ck = torch.zeros(2, 256, 8, 128, device=device, dtype=torch.bfloat16)
    cv = torch.ones_like(ck)
    meta = MixedAttentionContext(0, 8, None, None, i32([0, 8]), i32([0, 257]), i32([[0, 1]]), 8, 257, True)
    ctx = SimpleNamespace(mixed=meta, slot_mapping=torch.arange(249, 257, device=device, dtype=torch.int32))
    expected = oatt.dense_suffix_attention(q.cpu(), torch.zeros(257, 8, 128),
                                           torch.cat([torch.ones(249, 8, 128), v.float().cpu()]))
    good = forward_mixed(q, k, v, ck, cv, ctx, 128 ** -0.5, store_kvcache)
    assert_close_gate(good, expected)
    cv[0, :249].fill_(7.0)
    bad = forward_mixed(q, k, v, ck, cv, ctx, 128 ** -0.5, store_kvcache)
    with pytest.raises(AssertionError):
        assert_close_gate(bad, expected)


@pytest.mark.parametrize("kv_fp8", [False, True])
@pytest.mark.parametrize("nd,cap,hq,hkv", [(4, 512, 32, 8), (16, 1024, 32, 8), (16, 2048, 32, 8), (24, 4096, 32, 8),
                                           (16, 1024, 32, 2)])
def test_direct_decode_chunk_lengths(device, kv_fp8, nd, cap, hq, hkv):
    # Short decode-only launches run one workgroup per (row, chunk, kv head)
    # with chunks of 2, 4, 8 or 16 workgroup steps (the shortest whose grid
    # fits the GPU).  These shapes take each length on a 256-CU MI355X: rows
    # of 1 token, one chunk plus one token, and the table's full width.
    g = torch.Generator().manual_seed(nd * 31 + cap)
    lens = torch.randint(1, cap + 1, (nd,), generator=g).tolist()
    lens[0], lens[1], lens[2], lens[3] = cap, 1, 129, min(cap, 1025)
    case = Case([L - 1 for L in lens], [], [], hq=hq, hkv=hkv, seed=nd + cap, kv_fp8=kv_fp8)
    (mx, mn), _, _ = _check(case, device)
    print(f"{nd} rows up to {cap} tokens, {hq}/{hkv} heads, fp8={kv_fp8}: max-abs {mx:.3e} mean-abs {mn:.3e}")


# --------------------------------------------- benchmark configurations
def _workload_case(index, kv_fp8=False, hq=32, hkv=8):
    import workloads
    w = workloads.config(index, hq, hkv)
    nd = w.num_decode
    case = Case([L - 1 for L in w.decode_lens], w.prefill_prefix, w.prefill_q, hq=hq, hkv=hkv, seed=1000 + index,
                kv_fp8=kv_fp8, tables=w.decode_tables + w.prefill_tables, num_blocks=w.k_cache.shape[0])
    # use the workload's own values so the test runs the benchmarked inputs
    case.q, case.k, case.v = w.q, w.k, w.v
    kc, vc = w.k_cache, w.v_cache
    case.cpu_pools = lambda: (kc.clone(), vc.clone())
    assert case.slots == w.slot_mapping and len(case.q) == nd + sum(w.prefill_q)
    return case


@pytest.mark.parametrize("index", [0, 1, 2, 3, 4])
def test_benchmark_config_bf16(device, index):
    # config 4 (64 long decode rows) is long enough for the decode work lists
    # to rotate kv heads across chunks
    case = _workload_case(index)
    (mx, mn), _, _ = _check(case, device)
    print(f"config {index}: max-abs {mx:.3e} mean-abs {mn:.3e}")


@pytest.mark.parametrize("index", [0, 1, 2, 3, 4])
def test_benchmark_config_fp8(device, index):
    # config 1 (cold prefill rows only) reads nothing from the E4M3FN pool and
    # runs the bf16 kernel; configs 2 and 3 read prefixes from it; config 4 is
    # one model layer's step (64 decode rows beside a 1,024-token chunk)
    case = _workload_case(index, kv_fp8=True)
    (mx, mn), _, _ = _check(case, device)
    print(f"config {index} fp8: max-abs {mx:.3e} mean-abs {mn:.3e}")


@pytest.mark.parametrize("index,kv_fp8", [(3, False), (3, True), (4, False), (4, True)])
def test_benchmark_config_tp2_rank_shape(device, index, kv_fp8):
    # one tensor-parallel rank at TP=2: 16 query and 4 kv heads (qwen3.py:29-35,
    # README.md:9), same rows, tables and slots as the full-head workload
    case = _workload_case(index, kv_fp8, hq=16, hkv=4)
    (mx, mn), _, _ = _check(case, device)
    print(f"config {index} at 16/4 heads fp8={kv_fp8}: max-abs {mx:.3e} mean-abs {mn:.3e}")


# --------------------------------------------- boundaries and padding
@pytest.mark.parametrize("kv_fp8", [False, True])
def test_decode_length_boundaries(device, kv_fp8):
    hist = [0, 62, 63, 64, 254, 255, 256, 510, 1023, 4095, 8191, 5000]
    _check(Case(hist, [], [], seed=7, kv_fp8=kv_fp8), device)


@pytest.mark.parametrize("kv_fp8", [False, True])
def test_decode_small_blocks_and_step_boundaries(device, kv_fp8):
    # 64-token blocks with pages in random order: an E4M3FN wavefront step is
    # 32 tokens and a workgroup step 128, so a step's wavefronts read two
    # blocks; lengths around 16/32-token halves, steps and 256/512-token items.
    hist = [14, 15, 16, 30, 31, 32, 94, 95, 127, 128, 200, 383, 384, 511, 512, 767, 1100, 2047]
    _check(Case(hist, [], [], bs=64, seed=17, kv_fp8=kv_fp8), device)
    # the same rows beside a prefill chunk (mixed launch)
    _check(Case(hist[:9], [70], [45], bs=64, seed=18, kv_fp8=kv_fp8), device)


def test_prefill_tile_and_prefix_boundaries(device):
    counts = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100]
    prefixes = [0, 1, 63, 64, 255, 256, 257, 0, 511, 3, 700]
    _check(Case([5, 300], prefixes, counts, seed=8), device)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (64, 8), (16, 1), (12, 4), (16, 4)])
def test_gqa_ratios(device, hq, hkv):
    _check(Case([100, 700], [40, 0], [70, 33], hq=hq, hkv=hkv, seed=hq * 10 + hkv), device)


@pytest.mark.parametrize("kv_fp8", [False, True])
@pytest.mark.parametrize("phases", [2, 3])
def test_prefill_rows_split_in_key_halves(device, kv_fp8, phases):
    # prefill-only launches: the rows whose heaviest block spans more key
    # tiles than twice a workgroup's share (and at least 16), after a cached
    # prefix at least as long as their chunk, run as pairs of items over the
    # two halves of each block's keys, merged by the second.  First case: two
    # long-prefix rows split beside unsplit lighter and cold rows (odd tile
    # counts: 4096 + 512 keys end mid-tile).  Second: one row of 1,100 new
    # tokens after 1,100 cached ones, alone.  Every long row splits in both,
    # so the blocks keep 32 positions.  Third: a cold row of 1,024 tokens,
    # as long as a workgroup's share allows but unable to split, beside a
    # long-prefix row that splits: 16-position blocks and split items.
    from slo_attn import workspace_events
    cases = (Case([], [4096, 0, 2900, 1, 130], [512, 700, 96, 33, 5], seed=12, kv_fp8=kv_fp8),
             Case([], [1100], [1100], seed=13, kv_fp8=kv_fp8),
             Case([], [0, 1024], [1024, 256], seed=14, kv_fp8=kv_fp8))
    for case in cases:
        workspace_events(device)
        (mx, mn), got, _ = _check(case, device, phases)
        merged = workspace_events(device)["split_prefill_merges"]
        print(f"split prefill fp8={kv_fp8} phases={phases}: max-abs {mx:.3e} mean-abs {mn:.3e}, "
              f"split pairs merged {merged}")
        # no decode rows: both phase masks make prefill-only launches, which split
        assert merged > 0, "no prefill item was split"
        # the merge's rounding does not depend on which half finishes second
        for _ in range(3):
            again, _ = case.run_gpu(device, phases)
            torch.cuda.synchronize()
            assert torch.equal(again.view(torch.int16), got.view(torch.int16))


@pytest.mark.parametrize("kv_fp8", [False, True])
def test_split_phases_match_fused(device, kv_fp8):
    # Each phase alone against the mixed launch: both pass the gate against
    # the oracle and agree to the gate's bounds; with a bf16 pool the decode
    # phase (the direct kernel, chunks of the mixed launch's length here) and
    # the prefill phase (the same prefill items) are bit-equal to it.
    case = Case([300, 1000, 17], [512], [200], seed=9, kv_fp8=kv_fp8)
    fused, _ = case.run_gpu(device, phases=3)
    dec, _ = case.run_gpu(device, phases=1)
    pre, _ = case.run_gpu(device, phases=2)
    torch.cuda.synchronize()
    want, _ = case.oracle()
    d = 3
    for got in (dec[:d], fused[:d]):
        assert_close_gate(got, want[:d])
    assert_close_gate(dec[:d], fused[:d])
    for got in (pre[d:], fused[d:]):
        assert_close_gate(got, want[d:])
    if not kv_fp8:
        assert torch.equal(fused[:d], dec[:d])
        assert torch.equal(fused[d:], pre[d:])


def test_deterministic_across_launches(device):
    case = Case([3000, 2000, 100], [1024], [300], seed=10)
    a, _ = case.run_gpu(device)
    b, _ = case.run_gpu(device)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("index,kv_fp8,waits", [(0, False, False), (3, False, True), (3, True, True), (4, False, True)])
def test_merge_that_gives_up_is_reported_and_does_not_poison_the_next_launch(device, monkeypatch, index, kv_fp8,
                                                                            waits):
    # A split-K merge task waits a bounded time for the chunks of its (row, kv
    # head).  With the bound set to 0 from the host (SLO_ATTN_MERGE_WAIT_US),
    # tasks whose chunks are not all in give up at once: every kernel still
    # exits, the host's check raises, the tickets are back at zero, and the
    # next launch with the normal bound is bit-identical to an untouched one.
    # Config 0 (16 short decode rows) runs the direct decode kernel, whose
    # last-arriving chunk merges without waiting: the bound changes nothing.
    from slo_attn import check_workspaces, workspace_events
    case = _workload_case(index, kv_fp8)
    clean, _ = case.run_gpu(device)
    check_workspaces()
    monkeypatch.setenv("SLO_ATTN_MERGE_WAIT_US", "0")
    gave_up = 0
    nd = len(case.decode_hist)
    for _ in range(3):
        out, _ = case.run_gpu(device)
        torch.cuda.synchronize()
        try:
            n = workspace_events(device)["merges_gave_up"]
        except RuntimeError as e:
            assert "gave up waiting" in str(e), e
            n = int(str(e).split("workspace_check: ")[1].split()[0])
        gave_up += n
        # a merge that gives up writes NaN to its (row, kv head)'s outputs
        if n:
            assert torch.isnan(out[:nd].float()).any(), "a merge gave up but no decode output is NaN"
    print(f"config {index} fp8={kv_fp8}: merges that gave up over 3 launches: {gave_up}")
    if waits:
        assert gave_up > 0, "no merge task gave up: the bounded wait's exit did not run"
    else:
        assert gave_up == 0
    monkeypatch.delenv("SLO_ATTN_MERGE_WAIT_US")
    again, _ = case.run_gpu(device)
    check_workspaces()
    assert torch.equal(clean.view(torch.int16), again.view(torch.int16))
