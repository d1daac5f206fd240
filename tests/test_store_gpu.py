"""KV-cache write on the GPU vs the oracle: bit-exact, bf16 and E4M3FN.

Shapes follow the reference's own store checks (tests/test_v1_attention_gpu.py:
sentinel-filled pools 99/-99, strided V rows from a fused QKV view, exact cache
bytes at :103-104) plus the quantisation edge cases of
docs/project_manual.md:527-537 (zero heads, -0, tiny values, outliers, exact
rounding ties) and an exhaustive pass of every finite bf16 value.
"""
import numpy as np
import pytest
import torch

from oracle import fp8, kvstore
from slo_attn import store_kvcache
from slo_attn import _lib

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _fused_qkv(n, hq, hkv, d, g, device):
    qkv = torch.randn(n, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(device)
    q, k, v = qkv.split([hq * d, hkv * d, hkv * d], dim=-1)
    return q.view(n, hq, d), k.view(n, hkv, d), v.view(n, hkv, d)


@pytest.mark.parametrize("nblk,bs,hkv,d,n", [(6, 256, 8, 128, 37), (4, 256, 2, 128, 300), (3, 64, 4, 64, 50),
                                             (2, 256, 1, 256, 9)])
def test_store_bf16_bit_exact(device, nblk, bs, hkv, d, n):
    g = torch.Generator().manual_seed(n)
    _, k, v = _fused_qkv(n, 4 * hkv, hkv, d, g, device)   # strided rows like qwen3.py:78-81
    assert v.stride(0) == 6 * hkv * d
    slots = torch.randperm(nblk * bs, generator=g)[:n].to(torch.int32)
    slots[::7] = -1
    kc = torch.full((nblk, bs, hkv, d), 99.0, dtype=torch.bfloat16, device=device)
    vc = torch.full_like(kc, -99.0)
    kc_ref, vc_ref = _bits(kc), _bits(vc)
    store_kvcache(k, v, kc, vc, slots.to(device))
    kvstore.store_kvcache(_bits(k), _bits(v), kc_ref, vc_ref, slots.numpy())
    assert np.array_equal(_bits(kc), kc_ref)
    assert np.array_equal(_bits(vc), vc_ref)


def _fp8_pools(nblk, bs, hkv, d, device):
    kc = torch.full((nblk, bs, hkv, d), 0x5A, dtype=torch.uint8, device=device)
    vc = torch.full_like(kc, 0xA5)
    ks = torch.full((nblk, bs, hkv), -3.0, dtype=torch.float32, device=device)
    vs = torch.full_like(ks, -5.0)
    return kc, vc, ks, vs


def _check_fp8(k, v, slots, kc, vc, ks, vs, floor=fp8.SCALE_FLOOR):
    kc_ref, vc_ref = kc.cpu().numpy(), vc.cpu().numpy()
    ks_ref, vs_ref = ks.cpu().numpy(), vs.cpu().numpy()
    store_kvcache(k, v, kc, vc, slots, ks, vs, scale_floor=floor)
    kvstore.store_kvcache_fp8(k.float().cpu().numpy(), v.float().cpu().numpy(), kc_ref, vc_ref, ks_ref, vs_ref,
                              slots.cpu().numpy(), floor)
    assert np.array_equal(kc.cpu().numpy(), kc_ref)
    assert np.array_equal(vc.cpu().numpy(), vc_ref)
    assert np.array_equal(ks.cpu().numpy().view(np.uint32), ks_ref.view(np.uint32))
    assert np.array_equal(vs.cpu().numpy().view(np.uint32), vs_ref.view(np.uint32))


@pytest.mark.parametrize("hkv,d", [(8, 128), (2, 64), (1, 256)])
def test_store_fp8_random_bit_exact(device, hkv, d):
    g = torch.Generator().manual_seed(hkv * d)
    n, nblk, bs = 200, 4, 256
    _, k, v = _fused_qkv(n, 4 * hkv, hkv, d, g, device)
    k = (k.float() * torch.logspace(-3, 2, n, device=device)[:, None, None]).to(torch.bfloat16)
    slots = torch.randperm(nblk * bs, generator=g)[:n].to(torch.int32)
    slots[5] = -1
    _check_fp8(k, v, slots.to(device), *_fp8_pools(nblk, bs, hkv, d, device))


def test_store_fp8_edge_cases(device):
    d, hkv = 128, 8
    rows = []
    rows.append(torch.zeros(hkv, d))                          # amax = 0 -> scale 1
    rows.append(torch.full((hkv, d), -0.0))                   # signed zeros -> 0x80
    tiny = torch.full((hkv, d), 2.0 ** -120)                  # scale hits the floor
    tiny[:, ::2] *= -1
    rows.append(tiny)
    out = torch.randn(hkv, d)
    out[:, 0] = 3.0e4                                          # one outlier per head
    rows.append(out)
    mags = torch.tensor(fp8.MAGNITUDES[1:], dtype=torch.float64)
    ties = torch.zeros(hkv, d)
    ties[:, 0] = 448.0                                         # scale exactly 1
    mids = ((mags[:-1] + mags[1:]) / 2).float()
    ties[:, 1:1 + min(d - 1, mids.numel())] = mids[:d - 1]     # exact rounding ties
    rows.append(ties)
    rows.append(-ties)
    sub = torch.zeros(hkv, d)
    sub[:, 0] = 448.0
    sub[:, 1:] = torch.linspace(-2.0 ** -6, 2.0 ** -6, d - 1)  # subnormal code range
    rows.append(sub)
    k = torch.stack(rows).to(torch.bfloat16)
    v = torch.flip(k, dims=[0]).contiguous()
    n = k.shape[0]
    slots = torch.arange(n, dtype=torch.int32) * 3
    _check_fp8(k.to(device), v.to(device), slots.to(device), *_fp8_pools(2, 256, hkv, d, device))


def test_store_fp8_every_finite_bf16(device):
    # Every finite bf16 value, in heads whose amax is 448 (scale 1: the code
    # is the value's own rounding) and in heads with a random amax.
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits.float()
    x = x[torch.isfinite(x)]
    d, hkv = 128, 8
    per = d - 1
    pad = (-x.numel()) % per
    x = torch.cat([x, torch.zeros(pad)]).view(-1, per)
    # heads with amax 448: clamp the pattern into [-448, 448], first element 448
    a = torch.cat([torch.full((x.shape[0], 1), 448.0), x.clamp(-448, 448)], dim=1)
    # heads with the raw values (amax set by the largest element of the row)
    b = torch.cat([torch.full((x.shape[0], 1), 1.0), x], dim=1)
    heads = torch.cat([a, b]).to(torch.bfloat16)
    rows = (heads.shape[0] + hkv - 1) // hkv
    heads = torch.cat([heads, torch.zeros(rows * hkv - heads.shape[0], d, dtype=torch.bfloat16)])
    k = heads.view(rows, hkv, d)
    v = torch.roll(k, 1, dims=0).contiguous()
    nblk = (rows + 255) // 256
    slots = torch.randperm(nblk * 256, generator=torch.Generator().manual_seed(7))[:rows].to(torch.int32)
    _check_fp8(k.to(device), v.to(device), slots.to(device), *_fp8_pools(nblk, 256, hkv, d, device))


def test_store_empty_and_all_padding(device):
    kc = torch.full((2, 256, 8, 128), 7.0, dtype=torch.bfloat16, device=device)
    vc = kc.clone()
    k = torch.randn(3, 8, 128, device=device).to(torch.bfloat16)
    store_kvcache(k[:0], k[:0], kc, vc, torch.zeros(0, dtype=torch.int32, device=device))
    store_kvcache(k, k, kc, vc, torch.full((3,), -1, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert (kc == 7.0).all() and (vc == 7.0).all()


def test_store_rejects_cpu_and_bad_strides(device):
    k = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    kc = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        store_kvcache(k, k, kc, kc, torch.zeros(2, dtype=torch.int32))
    kg = torch.zeros(2, 8, 256, dtype=torch.bfloat16, device=device)[..., :128]
    with pytest.raises(AssertionError):
        store_kvcache(kg, kg, kc.to(device), kc.to(device), torch.zeros(2, dtype=torch.int32, device=device))
