"""LM head + greedy argmax on the GPU (slo_attn.lm_head_argmax).

Against oracle/lm_head.py on small shapes (rows 1..128, vocab not a multiple of
the 128-row tile, hidden 128..2560): the logits (when requested) are within one
bf16 step of the oracle everywhere (plus 1e-6 of the largest logit, the fp32
summation error of values that cancel to near zero) and equal on all but a
small fraction, and
every token is the oracle's argmax or within one bf16 step of the oracle's
maximum (the only way two fp32 summation orders can disagree); exact ties from
duplicated weight rows resolve to the smaller index.  At the Qwen3-4B shape
(65 sampled rows, vocab 151936, hidden 2560) the tokens agree the same way
with torch's F.linear + argmax on the GPU.
"""
import numpy as np
import pytest
import torch

from oracle import lm_head
from slo_attn import lm_head_argmax

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _f(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _check_tokens(tokens, ref_logits_bits):
    lf = _f(ref_logits_bits)
    mx = lf.max(axis=1)
    mine = lf[np.arange(lf.shape[0]), tokens]
    ulp = np.ldexp(1.0, np.frexp(np.abs(mx) + 1e-30)[1] - 8)
    assert (mine >= mx - ulp).all(), "a token is more than one bf16 step below the maximum"
    return (tokens == np.argmax(lf, axis=1)).mean()


@pytest.mark.parametrize("rows,vocab,hidden", [(1, 1000, 128), (7, 5003, 512), (65, 3000, 2560), (128, 777, 256)])
def test_against_oracle(device, rows, vocab, hidden):
    g = torch.Generator().manual_seed(rows + vocab)
    h = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    w = (torch.randn(vocab, hidden, generator=g) * hidden ** -0.5).to(torch.bfloat16)
    w[vocab - 1] = w[vocab // 3]  # an exact tie between two vocab rows
    tokens, logits = lm_head_argmax(h.to(device), w.to(device), return_logits=True)
    want = lm_head.logits(_bits(h), _bits(w))
    got = _bits(logits)
    diff = np.abs(_f(got) - _f(want))
    ulp = np.ldexp(1.0, np.frexp(np.abs(_f(want)) + 1e-30)[1] - 8)
    # fp32 sums of many products also differ absolutely by ~2^-24 of the summed
    # magnitudes, which is many bf16 steps of a logit that cancels to near zero
    slack = 1e-6 * np.abs(_f(want)).max()
    assert (diff <= ulp + slack).all(), "logits more than one bf16 step (plus fp32 summation slack) from the oracle"
    assert (diff > 0).mean() < 2e-2
    tok = tokens.cpu().numpy()
    _check_tokens(tok, want)
    # the tokens are the argmax of the logits this call wrote, first index on ties
    assert np.array_equal(tok, np.argmax(_f(got), axis=1))
    # a second call (keys were cleared) without logits gives the same tokens
    assert torch.equal(lm_head_argmax(h.to(device), w.to(device)).cpu(), tokens.cpu())


def test_qwen3_shape_against_torch(device):
    g = torch.Generator(device=device).manual_seed(4)
    w = torch.empty(151936, 2560, dtype=torch.bfloat16, device=device).normal_(0, 0.02, generator=g)
    h = torch.empty(65, 2560, dtype=torch.bfloat16, device=device).normal_(0, 1, generator=g)
    tokens = lm_head_argmax(h, w)
    ref = torch.nn.functional.linear(h, w)
    match = _check_tokens(tokens.cpu().numpy(), _bits(ref))
    print(f"tokens equal to torch argmax on {match * 100:.1f}% of rows")


def test_rejects_bad_arguments(device):
    h = torch.zeros(2, 256, dtype=torch.bfloat16, device=device)
    w = torch.zeros(10, 256, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        lm_head_argmax(torch.zeros(129, 256, dtype=torch.bfloat16, device=device), w)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        lm_head_argmax(h[:, :200].contiguous(), w[:, :200].contiguous())
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        lm_head_argmax(h.cpu(), w.cpu())
