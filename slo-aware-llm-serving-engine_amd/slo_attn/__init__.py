"""MI355X (gfx950) attention hot path for the SLO-aware nano-vLLM engine.

Host layer in Python over hand-written HIP kernels behind a C-ABI
(include/slo_attn.h, built into libslo_attn.so next to this file):
``store_kvcache`` (slot-mapped KV write, optional E4M3FN quantisation) and one
ragged mixed prefill/decode paged-attention launch, exposed through the same
``Attention`` / ``forward_mixed`` / ``Context`` interfaces as the reference.
"""
from .context import Context, get_context, reset_context, set_context
from .mixed_attention import MixedAttentionContext, forward_mixed
from .ops import check_workspaces, lm_head_argmax, workspace_events, paged_attention, qk_norm_rope_store, reserve_workspace, rope_cos_sin, store_kvcache
from .attention import Attention
from .kv_pool import KVPool, kv_block_bytes, num_kv_blocks
from .graph import MixedStepBuffers, MixedStepGraph
from . import _lib

__all__ = [
    "Attention", "KVPool", "MixedStepBuffers", "MixedStepGraph", "kv_block_bytes", "num_kv_blocks", "Context",
    "MixedAttentionContext", "check_workspaces", "forward_mixed", "get_context",
    "lm_head_argmax", "paged_attention", "qk_norm_rope_store", "reserve_workspace", "reset_context", "rope_cos_sin",
    "set_context", "store_kvcache", "workspace_events",
]
