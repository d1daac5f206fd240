"""Qwen3-4B mixed forward step with random-init weights (not collected by pytest).

The model restates nanovllm/models/qwen3.py (attention block :14-88, MLP
:91-115, decoder layer :118-159, model and LM head :162-215) in eager torch,
keeping the rounding points of the reference layers:

* RMSNorm (nanovllm/layers/layernorm.py:16-40): statistics in fp32, cast to
  bf16, then the bf16 weight multiply; with a residual, the add is done in fp32
  and the new residual is the bf16 rounding of the sum.
* RoPE (nanovllm/layers/rotary_embedding.py:6-48): fp32 table of
  ``position * inv_freq`` over max_position, rotation of the two halves in
  fp32, one rounding to bf16.
* SiluAndMul (nanovllm/layers/activation.py:8-11): evaluated in fp32 and
  rounded once, as the compiled reference evaluates it.
* Linear layers (nanovllm/layers/linear.py): bf16 ``F.linear``; the fused QKV
  and gate/up projections are single matrices split after the product, so V is
  a strided view of the QKV output.
* LM head (nanovllm/layers/embed_head.py:56-66) on the sampled rows only, tied
  to the embedding as in Qwen3-4B, then greedy argmax
  (nanovllm/engine/mixed_model_runner.py:115-126).

Both runs of a check share every line of this model except the per-layer
attention module: ``slo_attn.Attention`` (the HIP path, a drop-in for
nanovllm.layers.attention.Attention) or ``ReferenceAttention`` (the oracle's
definitions evaluated in fp32 on the same device).  The KV pool is laid out as
the mixed runner allocates it (mixed_model_runner.py:38-47): one
``[2, layers, blocks, 256, kv_heads, head_dim]`` tensor with per-layer views,
plus ``[2, layers, blocks, 256, kv_heads]`` fp32 scales for the E4M3FN pool.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import metadata
from slo_attn import KVPool, MixedAttentionContext, get_context, qk_norm_rope_store, reset_context, set_context


# Residual-branch conditioning of the full config-4 step.  With plain N(0, 0.02)
# weights every MLP adds about 1.2 RMS to a residual that starts at the
# embedding's 0.02, so the final hidden state is close to Gaussian noise: the
# 151936 logits of a row are Gaussian and their top two often share one bf16
# value, and two exact evaluations (fp32, fp64) pick different tokens.  Scaling
# o_proj and down_proj down makes each layer add a few percent of the residual,
# so the embedding keeps most of it: with the tied LM head a row's own token
# then wins by a wide margin (at least 3.6 logits, against 0.25 between the
# exact evaluations), while attention still carries the rest of the logit
# vector (zeroing it changes the logits by 130% in relative L2).
CONDITIONED = dict(o_proj_std=4e-4, down_proj_std=2.6e-5)


@dataclass(frozen=True)
class Geometry:
    """Qwen3-4B (configs/qwen3_4b.json and its HF config)."""
    num_layers: int = 36
    hidden: int = 2560
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 9728
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6
    max_position: int = 40960
    init_std: float = 0.02
    # Residual-branch conditioning of the random init: the std of o_proj and
    # down_proj (the two projections that write into the residual stream),
    # and the q/k norm weights (None: init_std and 1, plain N(0, init_std)).
    o_proj_std: float | None = None
    down_proj_std: float | None = None
    qk_norm_weight: float = 1.0


# ------------------------------------------------------------------ layers
def rms_norm(x, weight, eps):
    """layernorm.py:18-26."""
    dtype = x.dtype
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return xf.to(dtype) * weight


def add_rms_norm(x, residual, weight, eps):
    """layernorm.py:28-40: returns (normalised, new residual)."""
    dtype = x.dtype
    xf = x.float() + residual.float()
    residual = xf.to(dtype)
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return xf.to(dtype) * weight, residual


def rope_table(geom: Geometry, device):
    """rotary_embedding.py:27-35: [max_position, head_dim] fp32 (cos | sin), contiguous."""
    d = geom.head_dim
    inv_freq = 1.0 / (geom.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float, device=device) / d))
    t = torch.arange(geom.max_position, dtype=torch.float, device=device)
    freqs = t[:, None] * inv_freq[None, :]
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).contiguous()


def apply_rope(x, cos, sin):
    """rotary_embedding.py:6-14."""
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)


def silu_and_mul(x):
    """activation.py:8-11, one rounding."""
    a, b = x.float().chunk(2, -1)
    return (F.silu(a) * b).to(x.dtype)


class Qwen3:
    """Weights and the mixed-step forward; ``attn[l]`` is layer l's attention module."""

    def __init__(self, geom: Geometry, device, seed: int = 4):
        self.geom, self.device = geom, device
        g = torch.Generator(device=device).manual_seed(seed)
        std, bf = geom.init_std, torch.bfloat16

        def normal(*shape, s=std):
            return torch.empty(shape, dtype=bf, device=device).normal_(0.0, s, generator=g)

        def ones(n, value=1.0):
            return torch.full((n,), value, dtype=bf, device=device)

        o_std = std if geom.o_proj_std is None else geom.o_proj_std
        down_std = std if geom.down_proj_std is None else geom.down_proj_std

        hq, hkv, d, h = geom.num_heads, geom.num_kv_heads, geom.head_dim, geom.hidden
        self.q_size, self.kv_size = hq * d, hkv * d
        self.embed = normal(geom.vocab, h)
        self.layers = []
        for _ in range(geom.num_layers):
            self.layers.append({
                "qkv": normal(self.q_size + 2 * self.kv_size, h),
                "o": normal(h, self.q_size, s=o_std),
                "gate_up": normal(2 * geom.intermediate, h),
                "down": normal(h, geom.intermediate, s=down_std),
                "input_norm": ones(h), "post_norm": ones(h),
                "q_norm": ones(d, geom.qk_norm_weight), "k_norm": ones(d, geom.qk_norm_weight),
            })
        self.final_norm = ones(h)
        self.rope = rope_table(geom, device)
        self.scale = d ** -0.5
        self.attn: list[nn.Module] = []
        # True: q/k norm, RoPE and the KV write run as one slo_attn launch
        # (qk_norm_rope_store) and the attention module skips its store.
        self.fused = False

    def forward(self, ids, positions):
        geom = self.geom
        hq, hkv, d, eps = geom.num_heads, geom.num_kv_heads, geom.head_dim, geom.eps
        cos, sin = self.rope[positions].unsqueeze(1).chunk(2, dim=-1)
        x = F.embedding(ids, self.embed)
        residual = None
        for w, attn in zip(self.layers, self.attn):
            if residual is None:
                h, residual = rms_norm(x, w["input_norm"], eps), x
            else:
                h, residual = add_rms_norm(x, residual, w["input_norm"], eps)
            qkv = F.linear(h, w["qkv"])
            if self.fused:
                q, k, v = qk_norm_rope_store(qkv, positions, w["q_norm"], w["k_norm"], eps, self.rope, hq, hkv,
                                             attn.k_cache, attn.v_cache, get_context().slot_mapping,
                                             attn.k_scale, attn.v_scale)
                o = attn(q, k, v, kv_stored=True)
            else:
                q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
                q = rms_norm(q.view(-1, hq, d), w["q_norm"], eps)
                k = rms_norm(k.view(-1, hkv, d), w["k_norm"], eps)
                v = v.view(-1, hkv, d)
                q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
                o = attn(q, k, v)
            x = F.linear(o.flatten(1, -1), w["o"])
            h, residual = add_rms_norm(x, residual, w["post_norm"], eps)
            x = F.linear(silu_and_mul(F.linear(h, w["gate_up"])), w["down"])
        h, _ = add_rms_norm(x, residual, self.final_norm, eps)
        return h

    def logits(self, hidden, sample_indices):
        return F.linear(hidden.index_select(0, sample_indices), self.embed)


def quantize_kv(x: np.ndarray):
    """``oracle.fp8.quantize_kv`` over token slices in threads (rows are independent)."""
    with ThreadPoolExecutor(8) as ex:
        parts = list(ex.map(ofp8.quantize_kv, np.array_split(x, 16)))
    return np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])


# ------------------------------------------------------------------- batch
@dataclass
class Batch:
    decode_lens: list[int]        # end_pos of each decode row (keys incl. the new token)
    prefill_count: list[int]
    prefill_start: list[int]
    tables: list[list[int]]       # decode rows first
    input_ids: list[int]
    positions: list[int]
    slots: list[int]
    num_blocks: int
    block_size: int

    @property
    def num_decode(self):
        return len(self.decode_lens)

    @property
    def sample_indices(self):
        """Every decode row and the last token of each prefill chunk."""
        out, at = list(range(self.num_decode)), self.num_decode
        for n in self.prefill_count:
            at += n
            out.append(at - 1)
        return out

    def host_meta(self):
        d = self.num_decode
        return metadata.mixed_metadata(self.decode_lens, self.tables[:d], self.prefill_start,
                                       self.prefill_count, self.tables[d:])

    def device_context(self, device):
        """What prepare_mixed publishes (mixed_model_runner.py:66-92)."""
        m = self.host_meta()

        def i32(x):
            return torch.tensor(x, dtype=torch.int32, device=device)

        d = self.num_decode
        pf = m["num_prefill_tokens"] > 0
        meta = MixedAttentionContext(
            d, m["num_prefill_tokens"], i32(m["decode_lens"]) if d else None,
            i32(m["decode_tables"]) if d else None, i32(m["prefill_cu_q"]) if pf else None,
            i32(m["prefill_cu_k"]) if pf else None, i32(m["prefill_tables"]) if pf else None,
            m["max_q"], m["max_k"], m["prefill_has_history"])
        return i32(self.slots), meta


def config4_batch(vocab: int, seed: int = 4, num_blocks: int = 681, block_size: int = 256,
                  num_decode: int = 64, chunk: int = 1024, prefix: int = 0) -> Batch:
    """64 decode rows with end_pos uniform in [512, 4096] and one 1024-token chunk.

    Lengths and block tables are drawn exactly as the single-layer workload of
    the same step (workloads.config(4)); token ids come after.
    """
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(512, 4097, (num_decode,), generator=g).tolist()
    totals = lens + [prefix + chunk]
    pages = [(t + block_size - 1) // block_size for t in totals]
    perm = torch.randperm(num_blocks, generator=g).tolist()
    tables, at = [], 0
    for n in pages:
        tables.append(perm[at:at + n])
        at += n
    ids = torch.randint(0, vocab, (num_decode + chunk,), generator=g).tolist()
    positions = [L - 1 for L in lens] + list(range(prefix, prefix + chunk))
    slots = [metadata.slot_of(tables[b], L - 1, block_size) for b, L in enumerate(lens)]
    slots += [metadata.slot_of(tables[-1], p, block_size) for p in range(prefix, prefix + chunk)]
    return Batch(lens, [chunk], [prefix], tables, ids, positions, slots, num_blocks, block_size)


# -------------------------------------------------------------------- pools
class Pool:
    """KV pool of every layer (slo_attn.KVPool: bf16, or E4M3FN codes plus fp32
    scales) with cached prefixes filled N(0, 1): bf16 values, or their E4M3FN
    encoding with per-(token, kv head) absmax scales."""

    def __init__(self, geom: Geometry, num_blocks: int, block_size: int, device, fp8: bool,
                 seed: int = 1004):
        self.pool = KVPool(geom.num_layers, num_blocks, block_size, geom.num_kv_heads, geom.head_dim,
                           "fp8_e4m3fn" if fp8 else "bf16", device)
        self.fp8, self.kv, self.scale = fp8, self.pool.kv, self.pool.scale
        shape = self.kv.shape
        g = torch.Generator(device=device).manual_seed(seed)
        for i in range(2):
            for l in range(geom.num_layers):
                if not fp8:
                    self.kv[i, l].normal_(generator=g)
                    continue
                x = torch.empty(shape[2:], dtype=torch.float32, device=device).normal_(generator=g)
                amax = x.abs().amax(dim=-1)
                sc = torch.where(amax == 0, torch.ones_like(amax), amax / ofp8.FP8_MAX)
                self.kv[i, l] = (x / sc[..., None]).clamp(-ofp8.FP8_MAX, ofp8.FP8_MAX) \
                    .to(torch.float8_e4m3fn).view(torch.uint8)
                self.scale[i, l] = sc

    def clone(self):
        other = object.__new__(Pool)
        other.pool = object.__new__(KVPool)
        other.pool.__dict__.update(self.pool.__dict__)
        other.pool.kv = self.kv.clone()
        other.pool.scale = None if self.scale is None else self.scale.clone()
        other.fp8, other.kv, other.scale = self.fp8, other.pool.kv, other.pool.scale
        return other

    def attach(self, modules):
        """Per-layer views, as allocate_kv_cache assigns them (mixed_model_runner.py:43-47)."""
        assert self.pool.attach(modules) == self.pool.num_layers


class ReferenceAttention(nn.Module):
    """The mixed step by the oracle's definitions, on the pool's device.

    Store (attention.py:10-40 and the quantisation contract of
    docs/project_manual.md:527-537, by ``oracle.fp8.quantize_kv``), then decode
    rows through ``oracle.attention.decode`` and prefill rows through
    ``oracle.attention.varlen`` (mixed_attention.py:29-57) in ``dtype`` (fp32,
    the reference's precision, or fp64 for a second exact evaluation); the
    output is rounded to bf16.  ``host_meta`` is the step's metadata as host
    lists.
    """

    def __init__(self, num_heads, head_dim, scale, num_kv_heads, dtype=torch.float32):
        super().__init__()
        self.dtype = dtype
        self.num_heads, self.head_dim, self.scale, self.num_kv_heads = num_heads, head_dim, scale, num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.k_scale = self.v_scale = None
        self.host_meta = None

    def forward(self, q, k, v):
        ctx = get_context()
        slots = ctx.slot_mapping.long()
        live = slots >= 0
        n, hkv, d = k.shape
        if self.k_scale is None:
            self.k_cache.view(-1, hkv * d)[slots[live]] = k.reshape(n, -1)[live]
            self.v_cache.view(-1, hkv * d)[slots[live]] = v.reshape(n, -1)[live]
            kc, vc = self.k_cache, self.v_cache
        else:
            table = torch.from_numpy(ofp8.DECODE_TABLE).to(q.device)
            for src, codes, scales in ((k, self.k_cache, self.k_scale), (v, self.v_cache, self.v_scale)):
                c, s = quantize_kv(src.float().cpu().numpy())
                codes.view(-1, hkv * d)[slots[live]] = torch.from_numpy(c).to(q.device).reshape(n, -1)[live]
                scales.view(-1, hkv)[slots[live]] = torch.from_numpy(s).to(q.device)[live]
            kc = table[self.k_cache.long()] * self.k_scale[..., None]
            vc = table[self.v_cache.long()] * self.v_scale[..., None]
        out = oatt.mixed(q, k, v, kc, vc, self.host_meta, self.scale, self.dtype)
        return out.to(torch.bfloat16)


class Recorder:
    """Wraps an attention module and keeps the K/V it was given, per call.

    Attribute reads and writes go to the wrapped module, so the pool views
    land where the module reads them."""

    def __init__(self, inner):
        object.__setattr__(self, "inner", inner)
        object.__setattr__(self, "seen", [])

    def __getattr__(self, name):
        return getattr(self.inner, name)

    def __setattr__(self, name, value):
        setattr(self.inner, name, value)

    def __call__(self, q, k, v, **kw):
        self.seen.append((k.clone(memory_format=torch.contiguous_format),
                          v.clone(memory_format=torch.contiguous_format)))
        return self.inner(q, k, v, **kw)


@torch.inference_mode()
def run_step(model: Qwen3, batch: Batch, modules, pool: Pool):
    """One mixed forward step; returns (sampled logits fp32, greedy tokens)."""
    device = model.device
    model.attn = list(modules)
    pool.attach(modules)
    host = batch.host_meta()
    for m in modules:
        if hasattr(m, "host_meta"):
            m.host_meta = host
    slots, meta = batch.device_context(device)
    ids = torch.tensor(batch.input_ids, dtype=torch.int64, device=device)
    positions = torch.tensor(batch.positions, dtype=torch.int64, device=device)
    set_context(False, slot_mapping=slots, mixed=meta)
    try:
        hidden = model.forward(ids, positions)
        idx = torch.tensor(batch.sample_indices, dtype=torch.int64, device=device)
        logits = model.logits(hidden, idx).float()
    finally:
        reset_context()
    return logits, logits.argmax(dim=-1)


def numerics_policy(logits: torch.Tensor, ref_logits: torch.Tensor):
    """The reference's acceptance rule on each row's fp32 logits (benchmarks/v1/
    numerics.py:5-18 as check_v1.py:216-236 applies it): top-1 match, relative
    L2 <= 0.02, cosine >= 0.999, max-abs <= 0.5.  Returns (passing rows, top-1
    match, rel-L2, cosine, max-abs), one entry per row."""
    rel = (logits - ref_logits).norm(dim=-1) / ref_logits.norm(dim=-1).clamp_min(1e-12)
    cos = F.cosine_similarity(logits, ref_logits, dim=-1)
    max_abs = (logits - ref_logits).abs().amax(dim=-1)
    top1 = logits.argmax(dim=-1) == ref_logits.argmax(dim=-1)
    ok = top1 & (rel <= 0.02) & (cos >= 0.999) & (max_abs <= 0.5) & torch.isfinite(rel)
    return ok, top1, rel, cos, max_abs


def top2_gaps(logits: torch.Tensor) -> torch.Tensor:
    top = logits.topk(2, dim=-1).values
    return top[:, 0] - top[:, 1]


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy()
