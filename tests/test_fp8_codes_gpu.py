"""Every E4M3FN code through the attention kernels' reads of the pool, bit for bit.

The kernels turn pool code bytes into bf16 with v_cvt_scalef32_pk_bf16_fp8 (two
codes per instruction, one from each byte of a 16-bit pair) in three places:
the direct decode kernel, the work-list decode path of a mixed launch and the
prefill tile.  Every finite E4M3FN value is a bf16 value, so when a query puts
all of its softmax weight on one key with unit scales, its output row is that
key's V codes decoded exactly.  Four V rows hold code (d + 128 * (k // 2) +
k % 2) % 256 at position d, so all 256 codes appear in both bytes of a pair;
the expected values come from the oracle's codec (oracle/fp8.py, which restates
benchmarks/v0/probe_quant_support.py:24-33).  The two NaN codes (0x7f, 0xff)
must come out as NaN, and code 0x80 (-0) as a zero of either sign.

Decode rows hold one cached token (all the weight by construction).  Prefill
rows hold a one-token prefix and one new token; the query is 16 at d = 0, the
prefix key 448 there (code 0x7e) and the new key 0, so the scores differ by
7168 and the new token's weight exp2(-7168 * scale * log2 e) is 0 in fp32.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 4, 1, 128, 64


def _pattern(k):
    return np.array([(d + 128 * (k // 2) + k % 2) % 256 for d in range(D)], dtype=np.uint8)


def _expected(codes):
    vals = np.array([ofp8.decode_e4m3fn(int(c)) for c in codes], dtype=np.float32)
    return torch.from_numpy(vals).to(torch.bfloat16)


def _check_rows(out_rows, patterns):
    for row, k in zip(out_rows, patterns):
        want = _expected(_pattern(k))
        nan = torch.isnan(want.float())
        for h in range(HQ):
            got = row[h].cpu()
            assert torch.isnan(got[nan].float()).all(), f"pattern {k} head {h}: NaN codes not NaN"
            # exact values; +0 and -0 compare equal (code 0x80 is -0, and an
            # accumulator that starts at +0 returns +0 for 1 * -0)
            assert torch.equal(got[~nan].float(), want[~nan].float()), \
                f"pattern {k} head {h}: decoded codes differ from the oracle codec"


def test_every_code_decodes_exactly(device):
    from slo_attn import _lib, ops
    nd, npf = 4, 4
    kc = torch.zeros(nd + npf, BS, HKV, D, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    for b in range(nd):                     # decode row b: block b, one token
        vc[b, 0, 0] = torch.from_numpy(_pattern(b))
    for r in range(npf):                    # prefill row r: block nd + r, prefix token + new token
        vc[nd + r, 0, 0] = torch.from_numpy(_pattern(r))
        kc[nd + r, 0, 0, 0] = 0x7E          # 448 at d = 0; the new token's key stays 0
    ks = torch.ones(nd + npf, BS, HKV, dtype=torch.float32)
    vs = torch.ones_like(ks)
    q = torch.zeros(nd + npf, HQ, D, dtype=torch.bfloat16)
    q[:nd] = torch.randn(nd, HQ, D).to(torch.bfloat16)
    q[nd:, :, 0] = 16.0
    dev = {n: t.to(device) for n, t in dict(kc=kc, vc=vc, ks=ks, vs=vs, q=q).items()}
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=device)  # noqa: E731
    meta = dict(num_decode=nd, decode_lens=i32([1] * nd), decode_tables=i32([[b] for b in range(nd)]),
                num_prefill=npf, prefill_cu_q=i32(list(range(npf + 1))),
                prefill_cu_k=i32([2 * r for r in range(npf + 1)]), max_q=1, max_k=2,
                prefill_tables=i32([[nd + r] for r in range(npf)]))
    for phases in (_lib.PHASE_ALL, _lib.PHASE_DECODE, _lib.PHASE_PREFILL):
        out = ops.paged_attention(dev["q"], dev["kc"], dev["vc"], D ** -0.5, num_kv_heads=HKV, k_scale=dev["ks"],
                                  v_scale=dev["vs"], phases=phases, **meta)
        torch.cuda.synchronize()
        if phases & _lib.PHASE_DECODE:
            _check_rows(out[:nd], range(nd))
        if phases & _lib.PHASE_PREFILL:
            _check_rows(out[nd:], range(npf))
