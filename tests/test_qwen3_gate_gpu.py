"""The config-4 acceptance gate rejects wrong attention (planted mistakes).

The full Qwen3-4B mixed step of test_qwen3_step_gpu.py is accepted when every
sampled row passes the reference's numerics policy against the fp32-oracle
model (benchmarks/v1/numerics.py:5-18 as check_v1.py:216-236 applies it).
With the conditioned random init (qwen3_step.CONDITIONED) each row's own
token wins the greedy choice by a wide margin, so top-1 agreement alone says
little about attention; these controls show that the policy as a whole does:
the same step with the oracle's attention mistaken in two plausible ways must
fail it on at least one row.

* Each decode row misses its newest key (attends to end_pos - 1 keys, an
  off-by-one in decode_lens; the KV write itself is right).
* Every score is scaled by 1.02 (a 2% softmax-scale error).

The mistakes are planted in the oracle-side module (the oracle's definitions
evaluated with torch on the step's device, as the unmistaken reference is):
no kernel changes.  A third run with the true reference once more must pass
every row (the control of the controls).
"""
from __future__ import annotations

import pytest
import torch

from qwen3_step import CONDITIONED, Geometry, Pool, Qwen3, ReferenceAttention, config4_batch, numerics_policy, \
    run_step

pytestmark = pytest.mark.gpu


class MistakenReference(ReferenceAttention):
    """ReferenceAttention with its step metadata and softmax scale changed."""

    def __init__(self, *args, decode_len_delta: int = 0, scale_factor: float = 1.0, **kw):
        super().__init__(*args, **kw)
        self.decode_len_delta = decode_len_delta
        self.scale = self.scale * scale_factor

    def forward(self, q, k, v):
        host = self.host_meta
        meta = dict(host)
        meta["decode_lens"] = [L + self.decode_len_delta for L in host["decode_lens"]]
        self.host_meta = meta
        try:
            return super().forward(q, k, v)
        finally:
            self.host_meta = host


@pytest.fixture(scope="module")
def model(device):
    m = Qwen3(Geometry(**CONDITIONED), device, seed=4)
    yield m
    del m
    torch.cuda.empty_cache()


def test_policy_rejects_planted_attention_mistakes(device, model):
    geom = model.geom
    hq, hkv, d, layers = geom.num_heads, geom.num_kv_heads, geom.head_dim, geom.num_layers
    batch = config4_batch(geom.vocab)
    pool = Pool(geom, batch.num_blocks, batch.block_size, device, False)

    def run(make):
        p = pool.clone()
        out = run_step(model, batch, [make() for _ in range(layers)], p)
        del p
        torch.cuda.synchronize()
        return out

    ref_logits, _ = run(lambda: ReferenceAttention(hq, d, model.scale, hkv))
    again, _ = run(lambda: ReferenceAttention(hq, d, model.scale, hkv))
    ok, *_ = numerics_policy(again, ref_logits)
    assert bool(ok.all()), "the reference fails its own policy"
    rows = ref_logits.shape[0]
    mistakes = {
        "decode rows miss their newest key": lambda: MistakenReference(hq, d, model.scale, hkv, decode_len_delta=-1),
        "softmax scale 2% high": lambda: MistakenReference(hq, d, model.scale, hkv, scale_factor=1.02),
    }
    for name, make in mistakes.items():
        logits, _ = run(make)
        ok, top1, rel, cos, max_abs = numerics_policy(logits, ref_logits)
        print(f"{name}: policy fails {int((~ok).sum())}/{rows} rows (top-1 differs on {int((~top1).sum())}; worst "
              f"rel-L2 {rel.max().item():.4f}, cosine {cos.min().item():.6f}, max-abs {max_abs.max().item():.4f})",
              flush=True)
        assert not bool(ok.all()), f"the acceptance policy does not detect: {name}"
    del pool
    torch.cuda.empty_cache()
