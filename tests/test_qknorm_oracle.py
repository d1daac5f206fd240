"""Pins the CPU definitions of q/k RMSNorm + RoPE + KV write (oracle/qknorm.py)
and of the LM head with greedy argmax (oracle/lm_head.py).

* rope: bit-exact against the reference's own formula evaluated by torch on
  the CPU (nanovllm/layers/rotary_embedding.py:6-14, eager: every product and
  sum rounded), on random heads and positions; position 0 is the identity; the
  table's rows are unit (cos, sin) pairs.
* rms_norm: against the reference's RMSNorm evaluated by torch on the CPU
  (nanovllm/layers/layernorm.py:16-26, eager).  The two definitions may round
  the fp32 mean of squares and rsqrt differently (torch's CPU reduction order
  and rsqrt are its own), so agreement is bitwise on all but about 1e-5 of the
  elements and within two bf16 steps (one in n = bf16(x*r), doubled at most by
  the weight product) everywhere;
  closed forms: a constant vector normalises to +-1 times the weight, the
  weight scales the result exactly (a power of two), and scaling x by a power
  of two leaves the result unchanged.
* f32_to_bf16: torch's round-to-nearest-even conversion on random and
  halfway values.
* qkv_step: splits the fused QKV row as qkv.split([q, k, v]) does
  (qwen3.py:79-81) and leaves v untouched.
* lm_head.logits: within one bf16 step of torch's F.linear on the CPU (the
  reference's compute_logits) on all elements, equal on all but ~1%;
  lm_head.greedy: torch.argmax's first-index rule on exact ties.
"""
import numpy as np
import torch

from oracle import qknorm

HD = 128
EPS = 1e-6


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def _table(max_pos=40960, base=1e6):
    inv_freq = 1.0 / (base ** (torch.arange(0, HD, 2, dtype=torch.float) / HD))
    t = torch.arange(max_pos, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(100000, generator=g) * 10
    # exact halfway points between adjacent bf16 values, both parities
    base = torch.randn(2000, generator=g).to(torch.bfloat16).float()
    half = (base.view(torch.int32) + 0x8000).view(torch.float32)
    for v in (x, half):
        assert np.array_equal(qknorm.f32_to_bf16(v.numpy()), _bits(v.to(torch.bfloat16)))


def test_rope_bit_exact_against_reference_formula():
    g = torch.Generator().manual_seed(1)
    table = _table()
    x = torch.randn(300, 8, HD, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, table.shape[0], (300,), generator=g)
    cos, sin = table[pos].unsqueeze(1).chunk(2, dim=-1)
    # rotary_embedding.py:6-14, evaluated eagerly
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    want = torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(torch.bfloat16)
    got = qknorm.rope(_bits(x), table[pos, :HD // 2].numpy(), table[pos, HD // 2:].numpy())
    assert np.array_equal(got, _bits(want))


def test_rope_position_zero_is_identity_and_table_rows_are_unit():
    table = _table(4096)
    assert torch.equal(table[0, :HD // 2], torch.ones(HD // 2)) and torch.equal(table[0, HD // 2:], torch.zeros(HD // 2))
    c, s = table[:, :HD // 2].double(), table[:, HD // 2:].double()
    assert (c * c + s * s - 1).abs().max() < 1e-6
    x = torch.randn(5, 3, HD).to(torch.bfloat16)
    got = qknorm.rope(_bits(x), table[[0] * 5, :HD // 2].numpy(), table[[0] * 5, HD // 2:].numpy())
    assert np.array_equal(got, _bits(x))


def test_rms_norm_against_reference_formula():
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(4000, 8, HD, generator=g) * torch.rand(4000, 8, 1, generator=g) * 4).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    # layernorm.py:18-26, evaluated eagerly
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    want = (xf * torch.rsqrt(var + EPS)).to(torch.bfloat16) * w
    got = qknorm.rms_norm(_bits(x), _bits(w), EPS)
    diff = (_from_bits(got).float() - want.float()).abs()
    ulp = torch.ldexp(torch.ones_like(diff), torch.frexp(want.float().abs().clamp_min(1e-30))[1] - 8)
    # a different rounding of n = bf16(x * r) may move the weighted result by two steps
    assert (diff <= 2 * ulp).all(), "more than two bf16 steps from the reference formula"
    frac = (diff > 0).float().mean().item()
    assert frac < 1e-4, f"{frac:.2e} of elements round differently"


def test_rms_norm_closed_forms():
    w = torch.full((HD,), 1.5).to(torch.bfloat16)
    for c in (1.0, -3.0, 0.125, 1024.0):
        x = torch.full((2, 1, HD), c).to(torch.bfloat16)
        got = _from_bits(qknorm.rms_norm(_bits(x), _bits(w), EPS)).float()
        assert torch.equal(got, torch.full_like(got, 1.5 * np.sign(c)))
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 4, HD, generator=g).to(torch.bfloat16)
    ones = torch.ones(HD).to(torch.bfloat16)
    base = _from_bits(qknorm.rms_norm(_bits(x), _bits(ones), 0.0)).float()
    twice = _from_bits(qknorm.rms_norm(_bits(x), _bits((2 * ones).to(torch.bfloat16)), 0.0)).float()
    assert torch.equal(twice, 2 * base)
    scaled = _from_bits(qknorm.rms_norm(_bits((x.float() * 8).to(torch.bfloat16)), _bits(ones), 0.0)).float()
    assert torch.equal(scaled, base)


def test_qkv_step_splits_rows_and_keeps_v():
    g = torch.Generator().manual_seed(4)
    hq, hkv, n = 4, 2, 6
    qkv = torch.randn(n, (hq + 2 * hkv) * HD, generator=g).to(torch.bfloat16)
    table = _table(64)
    pos = np.arange(n) * 7
    w = torch.ones(HD).to(torch.bfloat16)
    q, k, v = qknorm.qkv_step(_bits(qkv), pos, _bits(w), _bits(w), EPS, table.numpy(), hq, hkv)
    qv, kv_, vv = qkv.split([hq * HD, hkv * HD, hkv * HD], dim=-1)
    assert np.array_equal(v, _bits(vv.reshape(n, hkv, HD)))
    cos, sin = table[pos, :HD // 2].numpy(), table[pos, HD // 2:].numpy()
    assert np.array_equal(q, qknorm.rope(qknorm.rms_norm(_bits(qv.reshape(n, hq, HD)), _bits(w), EPS), cos, sin))
    assert np.array_equal(k, qknorm.rope(qknorm.rms_norm(_bits(kv_.reshape(n, hkv, HD)), _bits(w), EPS), cos, sin))


# ------------------------------------------------- LM head + greedy (oracle/lm_head.py)
def test_lm_head_oracle_against_torch_and_tie_rule():
    from oracle import lm_head
    g = torch.Generator().manual_seed(5)
    h = torch.randn(9, 512, generator=g).to(torch.bfloat16)
    w = (0.05 * torch.randn(3000, 512, generator=g)).to(torch.bfloat16)
    got = lm_head.logits(_bits(h), _bits(w))
    # the reference computation (F.linear in bf16), evaluated by torch on the CPU
    want = torch.nn.functional.linear(h, w)
    diff = (_from_bits(got).float() - want.float()).abs()
    ulp = torch.ldexp(torch.ones_like(diff), torch.frexp(want.float().abs().clamp_min(1e-30))[1] - 8)
    assert (diff <= ulp).all() and (diff > 0).float().mean() < 1e-2
    # ties: identical weight rows give identical logits; the first index wins, as in torch.argmax
    w2 = w.clone()
    w2[2000] = w2[100]
    lg = lm_head.logits(_bits(h), _bits(w2))
    top = lm_head.greedy(lg)
    assert np.array_equal(top, torch.argmax(_from_bits(lg).float(), dim=-1).numpy())
    h3 = w2[100:101].clone() * 4  # row aligned with the duplicated weight row
    t3 = lm_head.greedy(lm_head.logits(_bits(h3.to(torch.bfloat16)), _bits(w2)))
    assert t3[0] == 100
