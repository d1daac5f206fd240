"""Pins the CPU oracle before it is trusted as the checker (CPU only).

Every oracle function is checked against something it does not compute itself:
* fp8 codec: the reference's known answers (tests/test_v0_quant.py:8-28), the
  torch library converter through the golden table (tests/golden/), and
  exhaustive agreement of the vectorised and scalar forms;
* quantize_kv: closed forms of the scale contract (amax=0, floor, the amax
  element lands on +-448, round-trip error bound);
* dense_suffix_attention: the reference KAT [3, 24.75]
  (tests/test_v1_validation.py:39-47), a brute-force triple loop, the
  uniform-attention closed form, GQA head mapping and input rejection;
* gather_pages / expected_slots: the layer-replay KATs
  (tests/test_layer_replay_diagnostic.py:14-22);
* store_kvcache: a per-token brute-force loop, untouched slots, slot -1;
* mixed / varlen / decode: equal to per-row dense attention on explicitly
  concatenated prefix + chunk, like tests/test_v1_reference_gpu.py:10-45.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import fp8, kvstore, metadata

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------ FP8 codec
def test_all_finite_codes_round_trip():
    codes = [c for c in range(256) if (c & 0x7F) != 0x7F]
    assert len(codes) == 254
    for c in codes:
        assert fp8.encode_e4m3fn(fp8.decode_e4m3fn(c)) == c


def test_ties_to_even_sign_zero_saturation():
    assert fp8.encode_e4m3fn(1.0625) == 56
    assert fp8.encode_e4m3fn(1.1875) == 58
    assert fp8.encode_e4m3fn(-0.0) == 128
    assert fp8.encode_e4m3fn(1e10) == 126
    assert fp8.encode_e4m3fn(-1e10) == 254
    assert fp8.decode_e4m3fn(126) == 448.0


def test_nonfinite_rejected():
    assert math.isnan(fp8.decode_e4m3fn(127))
    for v in (math.nan, math.inf, -math.inf):
        with pytest.raises(ValueError):
            fp8.encode_e4m3fn(v)
    with pytest.raises(ValueError):
        fp8.encode_array(np.array([1.0, np.nan], dtype=np.float32))


def _bf16_values():
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    return bits.float().numpy()


def test_encode_array_matches_golden_torch_table():
    table = np.load(os.path.join(GOLDEN, "e4m3fn_bf16_codes.npy"))
    x = _bf16_values()
    finite = np.isfinite(x)
    got = fp8.encode_array(np.clip(x[finite], -448, 448))
    assert np.array_equal(got, table[finite])


def test_encode_array_matches_scalar_exhaustively_on_bf16():
    x = _bf16_values()
    x = np.clip(x[np.isfinite(x)], -448, 448)
    sample = x[::7]  # scalar path is pure Python; every 7th bf16 value still covers all binades
    want = np.array([fp8.encode_e4m3fn(float(v)) for v in sample], dtype=np.uint8)
    assert np.array_equal(fp8.encode_array(sample), want)


def test_encode_array_midpoints_and_random_fp32():
    mags = np.array(fp8.MAGNITUDES, dtype=np.float64)
    mids = ((mags[:-1] + mags[1:]) / 2).astype(np.float32)  # exact ties (representable in fp32)
    rng = np.random.default_rng(0)
    rand = (rng.standard_normal(20000) * rng.choice([1e-3, 1e-2, 1, 30, 300], 20000)).astype(np.float32)
    for x in (mids, -mids, rand):
        want = torch.from_numpy(np.clip(x, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(fp8.encode_array(x), want)


def test_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = fp8.DECODE_TABLE
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()


# --------------------------------------------------------- quantisation rule
def test_quantize_zero_vector_scale_one():
    x = np.zeros((2, 128), dtype=np.float32)
    x[1] = -0.0
    codes, scale = fp8.quantize_kv(x)
    assert (scale == 1.0).all()
    assert (codes[0] == 0).all() and (codes[1] == 0x80).all()


def test_quantize_scale_is_amax_over_448_and_amax_hits_448():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    codes, scale = fp8.quantize_kv(x)
    amax = np.abs(x).max(-1)
    assert np.array_equal(scale, (amax / np.float32(448)).astype(np.float32))
    arg = np.abs(x).argmax(-1)
    hit = codes[np.arange(64), arg] & 0x7F
    assert (hit == 126).all()  # |x|/scale rounds to 448 (or saturates there)


def test_quantize_floor_applies_to_tiny_amax():
    x = np.full((1, 128), np.float32(2.0 ** -100))
    codes, scale = fp8.quantize_kv(x)
    assert scale[0] == np.float32(2.0 ** -64)
    assert (codes == 0).all()  # 2^-36 of the scale rounds to zero
    big = np.full((1, 128), np.float32(1.0))
    _, s2 = fp8.quantize_kv(big, scale_floor=1.0)
    assert s2[0] == 1.0


def test_quantize_round_trip_error_bound():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((256, 128)) * rng.uniform(0.01, 50, (256, 1))).astype(np.float32)
    codes, scale = fp8.quantize_kv(x)
    xh = fp8.dequantize_kv(codes, scale)
    # E4M3 has 3 mantissa bits: relative rounding error <= 2^-4 for normals,
    # absolute <= 2^-10 * scale in the subnormal range.
    err = np.abs(xh - x)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, scale[:, None] * 2.0 ** -10) * 1.0001
    assert (err <= bound).all()


# ----------------------------------------------------------------- attention
def test_dense_suffix_bottom_right_kat():
    q = torch.zeros(2, 4, 2)
    k = torch.zeros(4, 2, 2)
    v = torch.tensor([0.0, 3.0, 6.0, 90.0])[:, None, None].expand(4, 2, 2)
    out = oatt.dense_suffix_attention(q, k, v, scale=1.0)
    want = torch.tensor([3.0, 24.75])[:, None, None].expand(2, 4, 2)
    torch.testing.assert_close(out, want)


def test_dense_suffix_rejects_invalid():
    with pytest.raises(ValueError):
        oatt.dense_suffix_attention(torch.zeros(3, 2, 2), torch.zeros(2, 1, 2), torch.zeros(2, 1, 2))
    with pytest.raises(ValueError):
        oatt.dense_suffix_attention(torch.full((1, 2, 2), float("nan")), torch.zeros(2, 1, 2),
                                    torch.zeros(2, 1, 2))
    with pytest.raises(ValueError):
        oatt.dense_suffix_attention(torch.zeros(1, 3, 2), torch.zeros(2, 2, 2), torch.zeros(2, 2, 2))


def _brute(q, k, v, scale):
    nq, H, D = q.shape
    nk, Hkv, _ = k.shape
    G = H // Hkv
    out = torch.zeros(nq, H, D, dtype=torch.float64)
    for i in range(nq):
        pos = nk - nq + i
        for h in range(H):
            kh = h // G
            s = [sum(float(q[i, h, d]) * float(k[j, kh, d]) for d in range(D)) * scale
                 for j in range(pos + 1)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            for d in range(D):
                out[i, h, d] = sum(w[j] * float(v[j, kh, d]) for j in range(pos + 1)) / z
    return out


@pytest.mark.parametrize("nq,nk,H,Hkv,D", [(1, 5, 4, 1, 3), (3, 7, 4, 2, 4), (4, 4, 2, 2, 5)])
def test_dense_suffix_matches_brute_force(nq, nk, H, Hkv, D):
    g = torch.Generator().manual_seed(nq * 100 + nk)
    q, k, v = (torch.randn(s, generator=g) for s in ((nq, H, D), (nk, Hkv, D), (nk, Hkv, D)))
    got = oatt.dense_suffix_attention(q, k, v, scale=0.7)
    torch.testing.assert_close(got.double(), _brute(q, k, v, 0.7), atol=1e-5, rtol=1e-5)


def test_uniform_attention_closed_form_and_gqa_mapping():
    # q = 0 makes every visible key equally likely: the output is the mean of
    # the visible values of the query head's own kv head.
    nk, Hkv, G, D = 9, 3, 4, 8
    v = torch.arange(nk * Hkv * D, dtype=torch.float32).view(nk, Hkv, D)
    k = torch.randn(nk, Hkv, D)
    q = torch.zeros(3, Hkv * G, D)
    out = oatt.dense_suffix_attention(q, k, v)
    for i in range(3):
        vis = nk - 3 + i + 1
        for h in range(Hkv * G):
            torch.testing.assert_close(out[i, h], v[:vis, h // G].mean(0))


def test_gather_pages_and_slots_kats():
    cache = torch.arange(12.0).reshape(3, 2, 1, 2)
    got = oatt.gather_pages(cache, [2, 0], 3)
    torch.testing.assert_close(got, torch.tensor([[[8.0, 9.0]], [[10.0, 11.0]], [[0.0, 1.0]]]))
    assert metadata.expected_slots([2, 0], 1, 3, 2) == [5, 0]
    with pytest.raises(ValueError):
        oatt.gather_pages(cache, [-1], 1)
    with pytest.raises(ValueError):
        oatt.gather_pages(cache, [0], 3)


def _flat_offsets(meta):
    """Flat query offsets of a mixed step: each decode row one token, then the
    prefill rows (BatchMetadata.query_offsets, batch_metadata.py:94-118)."""
    d = meta["num_decode"]
    return tuple(range(d + 1)) + tuple(d + c for c in meta["prefill_cu_q"][1:])


def test_flat_offsets_kat():
    # tests/test_v1_state.py:88-101: a 256-token sequence decodes its token at
    # position 256 beside the first 256-token chunk of a 513-token prompt, one
    # step, 256-token blocks: query_offsets (0, 1, 257), positions[:3]
    # (256, 0, 1).
    bs = 256
    tables = [[0, 1], [2, 3, 4]]
    meta = metadata.mixed_metadata([257], tables[:1], [0], [256], tables[1:])
    assert _flat_offsets(meta) == (0, 1, 257)
    step = metadata.padded_step([256, 0], [1, 256], 1, 1, 257, tables, bs)
    assert tuple(step["positions"][:3]) == (256, 0, 1)
    assert step["positions"] == [256] + list(range(256))
    assert step["slot_mapping"][0] == metadata.slot_of(tables[0], 256, bs) == 256
    assert step["slot_mapping"][1:] == metadata.expected_slots(tables[1], 0, 256, bs)
    assert step["decode_lens"] == [257] and step["cu_seqlens_q"] == [0, 256] and step["cu_seqlens_k"] == [0, 256]
    assert not meta["prefill_has_history"]  # the chunk starts at position 0


def test_mixed_oracle_equals_dense_on_concatenated_history():
    # Mirrors tests/test_v1_reference_gpu.py:10-45 on the CPU: decode 256+1,
    # prefill 249+8 across a page boundary, and a cold 17-token prefill.
    g = torch.Generator().manual_seed(101)
    histories, counts = [256, 249, 0], [1, 8, 17]
    tables = [[5, 1], [3, 0], [2]]
    H, Hkv, D, bs = 32, 8, 16, 256
    N = sum(counts)
    q = torch.randn(N, H, D, generator=g)
    k = torch.randn(N, Hkv, D, generator=g)
    v = torch.randn(N, Hkv, D, generator=g)
    ck = torch.full((6, bs, Hkv, D), 19.0)
    cv = torch.full((6, bs, Hkv, D), -23.0)
    expected, slots, off = [], [], 0
    for t, h, n in zip(tables, histories, counts):
        ok = torch.randn(h, Hkv, D, generator=g)
        ov = torch.randn(h, Hkv, D, generator=g)
        for p in range(h):
            ck[t[p // bs], p % bs] = ok[p]
            cv[t[p // bs], p % bs] = ov[p]
        sl = slice(off, off + n)
        expected.append(oatt.dense_suffix_attention(q[sl], torch.cat([ok, k[sl]]), torch.cat([ov, v[sl]])))
        slots.extend(metadata.slot_of(t, p, bs) for p in range(h, h + n))
        off += n
    kvstore.store_kvcache(k.numpy(), v.numpy(), ck.numpy(), cv.numpy(), slots)
    meta = metadata.mixed_metadata([257], [tables[0]], [249, 0], [8, 17], tables[1:])
    got = oatt.mixed(q, k, v, ck, cv, meta, D ** -0.5)
    torch.testing.assert_close(got, torch.cat(expected), atol=1e-5, rtol=1e-5)
    assert meta["prefill_cu_q"] == [0, 8, 25] and meta["prefill_cu_k"] == [0, 257, 274]
    assert meta["decode_tables"] == [[5, 1]] and meta["prefill_tables"] == [[3, 0], [2, -1]]


# ------------------------------------------------------------------ KV store
def test_store_matches_per_token_loop_and_keeps_other_slots():
    rng = np.random.default_rng(3)
    nblk, bs, H, D, N = 4, 8, 2, 4, 10
    key = rng.integers(0, 65535, (N, H, D), dtype=np.uint16)
    val = rng.integers(0, 65535, (N, H, D), dtype=np.uint16)
    slots = rng.permutation(nblk * bs)[:N].astype(np.int64)
    slots[3] = -1
    kc = np.full((nblk, bs, H, D), 99, dtype=np.uint16)
    vc = np.full((nblk, bs, H, D), 77, dtype=np.uint16)
    kc2, vc2 = kc.copy(), vc.copy()
    kvstore.store_kvcache(key, val, kc, vc, slots)
    for i, s in enumerate(slots):
        if s == -1:
            continue
        kc2[s // bs, s % bs] = key[i]
        vc2[s // bs, s % bs] = val[i]
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)
    untouched = np.ones(nblk * bs, bool)
    untouched[slots[slots != -1]] = False
    assert (kc.reshape(nblk * bs, -1)[untouched] == 99).all()


def test_store_fp8_matches_quantize_per_head():
    rng = np.random.default_rng(4)
    nblk, bs, H, D, N = 3, 16, 2, 128, 5
    k = rng.standard_normal((N, H, D)).astype(np.float32)
    v = rng.standard_normal((N, H, D)).astype(np.float32) * 7
    slots = [17, -1, 3, 40, 0]
    kc = np.zeros((nblk, bs, H, D), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros((nblk, bs, H), np.float32)
    vs = np.zeros_like(ks)
    kvstore.store_kvcache_fp8(k, v, kc, vc, ks, vs, slots)
    for i, s in enumerate(slots):
        if s == -1:
            continue
        c, sc = fp8.quantize_kv(k[i])
        assert np.array_equal(kc[s // bs, s % bs], c) and np.array_equal(ks[s // bs, s % bs], sc)
    assert (kc[0, 1] == 0).all()  # slot of the -1 row never written


def test_padded_step_metadata_matches_prepare_mixed_and_slot_kats():
    # unpadded rows agree with mixed_metadata (prepare_mixed) and with expected_slots
    # (layer_replay.py:32-37); padding rows and tokens are inert.
    tables = [[2, 0], [5], [1, 3, 4], [6]]
    dstart = [300, 17]
    rows = [(250, 20), (0, 5)]
    dc, pc, tc, bs = 3, 3, 40, 256
    starts = dstart + [0] + [s for s, _ in rows] + [0]
    toks = [1, 1, 0] + [n for _, n in rows] + [0]
    tabs = tables[:2] + [[]] + tables[2:] + [[]]
    got = metadata.padded_step(starts, toks, dc, pc, tc, tabs, bs)
    ref = metadata.mixed_metadata([301, 18], tables[:2], [250, 0], [20, 5], tables[2:])
    assert got["decode_lens"] == ref["decode_lens"] + [0]
    assert got["cu_seqlens_q"] == ref["prefill_cu_q"] + [25]
    assert got["cu_seqlens_k"] == ref["prefill_cu_k"] + [ref["prefill_cu_k"][-1]]
    assert got["slot_mapping"][:2] == [metadata.slot_of(tables[0], 300, bs), metadata.slot_of(tables[1], 17, bs)]
    assert got["slot_mapping"][2] == -1
    assert got["slot_mapping"][3:23] == metadata.expected_slots(tables[2], 250, 270, bs)
    assert got["slot_mapping"][23:28] == metadata.expected_slots(tables[3], 0, 5, bs)
    assert got["slot_mapping"][28:] == [-1] * 12 and got["positions"][28:] == [0] * 12
    assert got["positions"][3:5] == [250, 251] and got["last_token"] == [0, 1, -1, 22, 27, -1]
