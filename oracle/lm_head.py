"""LM head on sampled rows and greedy argmax -- CPU definition (numpy).

Restates ParallelLMHead.forward at TP=1 (nanovllm/layers/embed_head.py:56-66:
logits = F.linear(x, weight), bf16 out) on the sampled rows and the greedy
choice of run_mixed (nanovllm/engine/mixed_model_runner.py:115-126:
logits.argmax(dim=-1), the first index among equal maxima).  The dot product
is taken exactly (float64, exact for the bf16 products and their sums at these
lengths up to the final rounding) and rounded once to fp32, then to bf16;
a GPU kernel summing in fp32 may differ from it by one bf16 step where the
fp32 sum sits next to a rounding boundary.
"""
from __future__ import annotations

import numpy as np

from .qknorm import bf16_to_f32, f32_to_bf16


def logits(hidden_bits: np.ndarray, weight_bits: np.ndarray) -> np.ndarray:
    """[rows, H] and [V, H] bf16 bits -> [rows, V] bf16 bits."""
    h = bf16_to_f32(hidden_bits).astype(np.float64)
    w = bf16_to_f32(weight_bits).astype(np.float64)
    return f32_to_bf16((h @ w.T).astype(np.float32))


def greedy(logits_bits: np.ndarray) -> np.ndarray:
    """First index of the largest bf16 value per row."""
    return np.argmax(bf16_to_f32(logits_bits), axis=-1).astype(np.int64)
