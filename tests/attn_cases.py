"""Shared builders for the attention parity tests (not collected by pytest).

A case is one mixed step: decode rows (history h -> h + 1 keys) first, then
prefill rows (cached prefix p, chunk of n new tokens).  The pool is filled
with sentinels, the prefixes are written page by page, the new tokens go
through the store kernel, and the oracle replays the same writes on the CPU.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import kvstore, metadata
from slo_attn import MixedAttentionContext, forward_mixed, store_kvcache

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def errors(got: torch.Tensor, want: torch.Tensor):
    diff = (got.float().cpu() - want.float().cpu()).abs()
    return diff.max().item(), diff.mean().item()


def assert_close_gate(got, want, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    got_c = got.float().cpu()
    assert torch.isfinite(got_c).all(), "non-finite attention output"
    mx, mn = errors(got, want)
    assert mx <= max_abs and mn <= mean_abs, f"max-abs {mx:.3e} (<= {max_abs}), mean-abs {mn:.3e} (<= {mean_abs})"
    return mx, mn


class Case:
    def __init__(self, decode_hist, prefill_hist, prefill_count, hq=32, hkv=8, d=128, bs=256,
                 seed=0, kv_fp8=False, num_blocks=None, tables=None, sentinel=(99.0, -99.0)):
        g = torch.Generator().manual_seed(seed)
        self.hq, self.hkv, self.d, self.bs, self.kv_fp8 = hq, hkv, d, bs, kv_fp8
        self.decode_hist = list(decode_hist)
        self.prefill_hist, self.prefill_count = list(prefill_hist), list(prefill_count)
        totals = [h + 1 for h in self.decode_hist] + [h + n for h, n in zip(self.prefill_hist, self.prefill_count)]
        pages = [(t + bs - 1) // bs for t in totals]
        if tables is None:
            nblk = num_blocks or sum(pages) + 3
            perm = torch.randperm(nblk, generator=g).tolist()
            tables, at = [], 0
            for p in pages:
                tables.append(perm[at:at + p])
                at += p
        else:
            nblk = num_blocks or (max(max(t) for t in tables) + 1)
        self.tables, self.nblk = tables, nblk
        nd = len(self.decode_hist)
        n_new = nd + sum(self.prefill_count)
        self.q = torch.randn(n_new, hq, d, generator=g).to(torch.bfloat16)
        self.k = torch.randn(n_new, hkv, d, generator=g).to(torch.bfloat16)
        self.v = torch.randn(n_new, hkv, d, generator=g).to(torch.bfloat16)
        hists = self.decode_hist + self.prefill_hist
        self.old_k = [torch.randn(h, hkv, d, generator=g).to(torch.bfloat16) for h in hists]
        self.old_v = [torch.randn(h, hkv, d, generator=g).to(torch.bfloat16) for h in hists]
        slots = []
        for b, h in enumerate(self.decode_hist):
            slots.append(metadata.slot_of(tables[b], h, bs))
        for r, (h, n) in enumerate(zip(self.prefill_hist, self.prefill_count)):
            slots.extend(metadata.slot_of(tables[nd + r], p, bs) for p in range(h, h + n))
        self.slots = slots
        self.meta_host = metadata.mixed_metadata(
            [h + 1 for h in self.decode_hist], tables[:nd], self.prefill_hist, self.prefill_count, tables[nd:])
        self.sentinel = sentinel
        self.scale = d ** -0.5

    # -------------------------------------------------------------- pools
    def cpu_pools(self):
        """bf16 pools with the prefixes resident (torch CPU, sentinel elsewhere)."""
        kc = torch.full((self.nblk, self.bs, self.hkv, self.d), self.sentinel[0], dtype=torch.bfloat16)
        vc = torch.full_like(kc, self.sentinel[1])
        for t, ok, ov in zip(self.tables, self.old_k, self.old_v):
            for p in range(ok.shape[0]):
                kc[t[p // self.bs], p % self.bs] = ok[p]
                vc[t[p // self.bs], p % self.bs] = ov[p]
        return kc, vc

    def meta(self, device):
        m = self.meta_host

        def i32(x):
            return None if x is None else torch.tensor(x, dtype=torch.int32, device=device)
        nd = m["num_decode"]
        return MixedAttentionContext(
            nd, m["num_prefill_tokens"], i32(m["decode_lens"]) if nd else None,
            i32(m["decode_tables"]) if nd else None,
            i32(m["prefill_cu_q"]) if m["num_prefill_tokens"] else None,
            i32(m["prefill_cu_k"]) if m["num_prefill_tokens"] else None,
            i32(m["prefill_tables"]) if m["num_prefill_tokens"] else None,
            m["max_q"], m["max_k"], m["prefill_has_history"])

    # --------------------------------------------------------------- run
    def run_gpu(self, device, phases=3):
        """Returns (output, device pools) after store + one attention launch."""
        from types import SimpleNamespace
        kc, vc = self.cpu_pools()
        ctx = SimpleNamespace(mixed=self.meta(device),
                              slot_mapping=torch.tensor(self.slots, dtype=torch.int32, device=device))
        q, k, v = self.q.to(device), self.k.to(device), self.v.to(device)
        if not self.kv_fp8:
            kd, vd = kc.to(device), vc.to(device)
            out = forward_mixed(q, k, v, kd, vd, ctx, self.scale, store_kvcache, phases=phases)
            return out, (kd, vd)
        codes, scales = self.fp8_pools(kc, vc)
        kd, vd = torch.from_numpy(codes[0]).to(device), torch.from_numpy(codes[1]).to(device)
        ksd, vsd = torch.from_numpy(scales[0]).to(device), torch.from_numpy(scales[1]).to(device)
        out = forward_mixed(q, k, v, kd, vd, ctx, self.scale, store_kvcache, ksd, vsd, phases=phases)
        return out, (kd, vd, ksd, vsd)

    def fp8_pools(self, kc, vc):
        """Quantise the resident bf16 pool on the CPU (every slot, sentinels too)."""
        kcodes, kscale = ofp8.quantize_kv(kc.float().numpy())
        vcodes, vscale = ofp8.quantize_kv(vc.float().numpy())
        return (kcodes, vcodes), (kscale, vscale)

    def oracle(self):
        """fp32 oracle of the same step; returns (output, pools after the write)."""
        kc, vc = self.cpu_pools()
        if not self.kv_fp8:
            kb = kc.view(torch.int16).numpy()
            vb = vc.view(torch.int16).numpy()
            kvstore.store_kvcache(self.k.view(torch.int16).numpy(), self.v.view(torch.int16).numpy(), kb, vb,
                                  self.slots)
            kf, vf = kc.float(), vc.float()
            pools = (kc, vc)
        else:
            (kcodes, vcodes), (kscale, vscale) = self.fp8_pools(kc, vc)
            kvstore.store_kvcache_fp8(self.k.float().numpy(), self.v.float().numpy(), kcodes, vcodes, kscale,
                                      vscale, self.slots)
            kf = torch.from_numpy(ofp8.dequantize_kv(kcodes, kscale))
            vf = torch.from_numpy(ofp8.dequantize_kv(vcodes, vscale))
            pools = (kcodes, vcodes, kscale, vscale)
        out = oatt.mixed(self.q.float(), self.k.float(), self.v.float(), kf, vf, self.meta_host, self.scale)
        return out, pools


def pool_bytes_equal(gpu_pools, cpu_pools) -> bool:
    for g, c in zip(gpu_pools, cpu_pools):
        gc = g.cpu()
        if gc.dtype == torch.bfloat16:
            if not torch.equal(gc.view(torch.int16), c.view(torch.int16)):
                return False
        else:
            cn = c if isinstance(c, np.ndarray) else c.numpy()
            if not np.array_equal(gc.numpy().view(np.uint8), cn.view(np.uint8)):
                return False
    return True
