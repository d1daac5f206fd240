"""The documented drop-in route for the metadata side channel, on the CPU.

The drop-in route replaces nanovllm/utils/context.py (reference lines 1-28) by
a re-export of slo_attn.context.  This test writes that module into a scratch
``nanovllm`` package, publishes a step through it as the reference runners do
(positional ``set_context``, mixed_model_runner.py:71,91 and
model_runner.py:169,187) and checks that ``slo_attn.Attention`` sees the same
``Context``: with a mixed context and no KV pool its forward raises the
reference's own error for that case (nanovllm/layers/mixed_attention.py:31-32),
and after ``reset_context`` it no longer takes the mixed branch.
"""
import importlib
import sys

import pytest
import torch

from slo_attn import Attention, MixedAttentionContext
from slo_attn import context as slo_context

REEXPORT = "from slo_attn.context import Context, get_context, reset_context, set_context\n"


@pytest.fixture
def nanovllm_context(tmp_path, monkeypatch):
    pkg = tmp_path / "nanovllm"
    (pkg / "utils").mkdir(parents=True)
    (pkg / "__init__.py").write_text("")
    (pkg / "utils" / "__init__.py").write_text("")
    (pkg / "utils" / "context.py").write_text(REEXPORT)
    monkeypatch.syspath_prepend(str(tmp_path))
    for name in ("nanovllm", "nanovllm.utils", "nanovllm.utils.context"):
        monkeypatch.delitem(sys.modules, name, raising=False)
    mod = importlib.import_module("nanovllm.utils.context")
    yield mod
    slo_context.reset_context()


def test_runner_context_reaches_the_attention_layer(nanovllm_context):
    ctx = nanovllm_context
    assert ctx.get_context is slo_context.get_context
    slots = torch.tensor([3, 4], dtype=torch.int32)
    meta = MixedAttentionContext(1, 1, None, None, None, None, None, 1, 1, False)
    # positional call, as prepare_mixed publishes the step
    ctx.set_context(False, None, None, 0, 0, slots, None, None, meta)
    seen = slo_context.get_context()
    assert seen.mixed is meta and seen.slot_mapping is slots and seen.is_prefill is False
    attn = Attention(32, 128, 128 ** -0.5, 8)   # no pool attached: k_cache / v_cache are empty
    q = torch.zeros(2, 32, 128, dtype=torch.bfloat16)
    k = v = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="mixed forward requires an allocated KV pool"):
        attn(q, k, v)
    ctx.reset_context()
    assert slo_context.get_context().mixed is None
    # without the mixed context the V0 branches run, which refuse CPU tensors (no CPU fallback)
    ctx.set_context(False, None, None, 0, 0, slots, torch.tensor([1, 1], dtype=torch.int32),
                    torch.zeros(2, 1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        attn(q, k, v)
