"""Seeded synthetic attention-layer workloads (Qwen3-4B head geometry).

Each workload is one layer's attention step as the V1 mixed runner issues it:
new q/k/v for every scheduled token, a paged KV pool whose cached prefixes are
already resident, per-row block tables and a slot mapping, with decode rows
first (nanovllm/engine/batch_metadata.py:72-74, mixed_model_runner.py:66-92).

RNG convention: ``g = torch.Generator().manual_seed(seed)``; integer draws are
``torch.randint(lo, hi + 1, ..., generator=g)``; values are ``torch.randn`` on
the CPU.  q and k are scaled to unit RMS per head (qk-norm), v ~ N(0, 1), the
pool is pre-filled N(0, 1), block tables come from one random permutation of
the pool so no two rows share a page.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

HQ, HKV, HD, BLOCK = 32, 8, 128, 256


@dataclass
class Workload:
    name: str
    q: torch.Tensor            # [N, Hq, D] bf16 (CPU)
    k: torch.Tensor            # [N, Hkv, D] bf16
    v: torch.Tensor
    k_cache: torch.Tensor      # [nblk, block, Hkv, D] bf16, cached prefixes resident
    v_cache: torch.Tensor
    slot_mapping: list[int]
    decode_lens: list[int]     # per decode row, keys incl. the new token
    decode_tables: list[list[int]]
    prefill_q: list[int]       # per prefill row, new tokens
    prefill_prefix: list[int]  # per prefill row, cached tokens before the chunk
    prefill_tables: list[list[int]]
    scale: float = HD ** -0.5
    block_size: int = BLOCK
    extra: dict = field(default_factory=dict)

    @property
    def num_decode(self) -> int:
        return len(self.decode_lens)

    @property
    def num_tokens(self) -> int:
        return self.q.shape[0]

    @property
    def has_history(self) -> bool:
        return any(p > 0 for p in self.prefill_prefix)

    @property
    def cu_q(self) -> list[int]:
        out = [0]
        for n in self.prefill_q:
            out.append(out[-1] + n)
        return out

    @property
    def cu_k(self) -> list[int]:
        out = [0]
        for n, p in zip(self.prefill_q, self.prefill_prefix):
            out.append(out[-1] + n + p)
        return out

    def decode_kv_bytes(self, elem_bytes: float = 2.0, scale_bytes: int = 0) -> int:
        """Algorithmic decode KV bytes: every cached key and value read once."""
        hkv, d = self.k.shape[1], self.k.shape[2]
        return int(sum(self.decode_lens) * hkv * (2 * d * elem_bytes + 2 * scale_bytes))

    def prefill_flops(self) -> int:
        """4*D*Hq per unmasked causal (query, key) pair."""
        hq, d = self.q.shape[1], self.q.shape[2]
        pairs = sum(n * p + n * (n + 1) // 2 for n, p in zip(self.prefill_q, self.prefill_prefix))
        return 4 * d * hq * pairs


def _unit_rms(x: torch.Tensor) -> torch.Tensor:
    return x / x.square().mean(-1, keepdim=True).sqrt()


def _pad(rows: list[list[int]]) -> list[list[int]]:
    width = max(len(r) for r in rows)
    return [list(r) + [-1] * (width - len(r)) for r in rows]


def padded_tables(rows: list[list[int]]) -> list[list[int]]:
    """Block tables padded with -1 to the row maximum (mixed_model_runner.py:62-64)."""
    return _pad(rows)


def build(name: str, seed: int, decode_lens: list[int], prefill_q: list[int],
          prefill_prefix: list[int], num_blocks: int, g: torch.Generator,
          hq: int = HQ, hkv: int = HKV, d: int = HD, block_size: int = BLOCK) -> Workload:
    rows_total = [L for L in decode_lens] + [p + n for p, n in zip(prefill_prefix, prefill_q)]
    pages_needed = [(t + block_size - 1) // block_size for t in rows_total]
    if sum(pages_needed) > num_blocks:
        raise ValueError("pool too small for the workload")
    perm = torch.randperm(num_blocks, generator=g).tolist()
    tables, at = [], 0
    for n in pages_needed:
        tables.append(perm[at:at + n])
        at += n
    num_tokens = len(decode_lens) + sum(prefill_q)
    q = _unit_rms(torch.randn(num_tokens, hq, d, generator=g)).to(torch.bfloat16)
    k = _unit_rms(torch.randn(num_tokens, hkv, d, generator=g)).to(torch.bfloat16)
    v = torch.randn(num_tokens, hkv, d, generator=g).to(torch.bfloat16)
    k_cache = torch.randn(num_blocks, block_size, hkv, d, generator=g).to(torch.bfloat16)
    v_cache = torch.randn(num_blocks, block_size, hkv, d, generator=g).to(torch.bfloat16)
    slots = []
    nd = len(decode_lens)
    for b, L in enumerate(decode_lens):
        pos = L - 1
        slots.append(tables[b][pos // block_size] * block_size + pos % block_size)
    for r, (n, p) in enumerate(zip(prefill_q, prefill_prefix)):
        t = tables[nd + r]
        slots.extend(t[pos // block_size] * block_size + pos % block_size for pos in range(p, p + n))
    return Workload(name=name, q=q, k=k, v=v, k_cache=k_cache, v_cache=v_cache, slot_mapping=slots,
                    decode_lens=list(decode_lens), decode_tables=tables[:nd],
                    prefill_q=list(prefill_q), prefill_prefix=list(prefill_prefix),
                    prefill_tables=tables[nd:], scale=d ** -0.5, block_size=block_size,
                    extra={"seed": seed})


def config(index: int, hq: int = HQ, hkv: int = HKV) -> Workload:
    """The attention-layer workloads of the five benchmark configurations.

    ``hq``/``hkv`` select the heads of one tensor-parallel rank (16 and 4 at
    TP=2, qwen3.py:29-35); row lengths, block tables and slots are drawn
    before the values, so they are the same whatever the head counts."""
    g = torch.Generator().manual_seed(index)
    tag = "" if (hq, hkv) == (HQ, HKV) else f"_{hq}q{hkv}kv"
    if index == 0:
        lens = torch.randint(64, 1025, (16,), generator=g).tolist()
        return build("decode16_ctx64-1024" + tag, 0, lens, [], [], 128, g, hq, hkv)
    if index == 1:
        lens = torch.randint(256, 2049, (4,), generator=g).tolist()
        return build("prefill4_varlen256-2048" + tag, 1, [], lens, [0] * 4, 64, g, hq, hkv)
    if index == 2:
        idx = torch.randint(0, 4, (3,), generator=g).tolist()
        prefixes = [(0, 512, 1024, 2048)[i] for i in idx]
        return build("chunked_prefill3x512_prefix" + tag, 2, [], [512] * 3, prefixes, 96, g, hq, hkv)
    if index == 3:
        lens = torch.randint(256, 4097, (24,), generator=g).tolist()
        return build("mixed_24decode_2x512chunk" + tag, 3, lens, [512, 512], [0, 1024], 512, g, hq, hkv)
    if index == 4:
        lens = torch.randint(512, 4097, (64,), generator=g).tolist()
        return build("qwen3_4b_layer_64decode_1024chunk" + tag, 4, lens, [1024], [0], 681, g, hq, hkv)
    raise ValueError(index)


def to_device(w: Workload, device, kv_fp8: bool = False):
    """Device tensors + MixedAttentionContext for ``w`` (prepare_mixed layout)."""
    from slo_attn import MixedAttentionContext

    def i32(x):
        return torch.tensor(x, dtype=torch.int32, device=device)

    nd = w.num_decode
    meta = MixedAttentionContext(
        nd, sum(w.prefill_q),
        i32(w.decode_lens) if nd else None,
        i32(padded_tables(w.decode_tables)) if nd else None,
        i32(w.cu_q) if w.prefill_q else None,
        i32(w.cu_k) if w.prefill_q else None,
        i32(padded_tables(w.prefill_tables)) if w.prefill_q else None,
        max(w.prefill_q) if w.prefill_q else 0,
        max(n + p for n, p in zip(w.prefill_q, w.prefill_prefix)) if w.prefill_q else 0,
        w.has_history,
    )
    return {
        "q": w.q.to(device), "k": w.k.to(device), "v": w.v.to(device),
        "slot_mapping": i32(w.slot_mapping), "meta": meta,
    }
