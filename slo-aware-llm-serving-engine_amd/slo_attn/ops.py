"""Host wrappers around the C-ABI: argument checks, workspace, stream plumbing.

Every function here launches hand-written HIP kernels through libslo_attn.so on
the current PyTorch stream.  Nothing allocates device memory except the output
tensor and the one-time, per-device workspace (grown outside graph capture), so
calls may be captured into a HIP graph once the workspace is reserved.
There is no CPU path: CPU tensors are rejected.
"""
from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib

_FP8_DTYPES = (torch.uint8,) + ((torch.float8_e4m3fn,) if hasattr(torch, "float8_e4m3fn") else ())


def kv_dtype_code(cache: torch.Tensor) -> int:
    if cache.dtype == torch.bfloat16:
        return _lib.KV_BF16
    if cache.dtype in _FP8_DTYPES:
        return _lib.KV_FP8_E4M3FN
    raise TypeError(f"KV cache dtype {cache.dtype} is not bf16 or E4M3FN bytes")


def _require_gpu(*tensors) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("slo_attn kernels need GPU tensors; there is no CPU fallback")
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"tensors on different devices: {device} vs {t.device}")
    return device


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _int32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32, got {t.dtype}")
    if t.dim() == 1 and t.stride(0) != 1:
        raise ValueError(f"{name} must be contiguous")
    return t


# ------------------------------------------------------------------ KV write
def check_store(key, value, k_cache, v_cache, slot_mapping, k_scale=None, v_scale=None):
    """The store's argument checks (nanovllm/layers/attention.py:36-39 and the
    formats); returns ``(device, kv_dtype code)``."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    # Same stride contract as the reference store (attention.py:36-39).
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    device = _require_gpu(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale)
    if key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        raise TypeError("key/value must be bf16")
    if value.shape != key.shape:
        raise ValueError("key/value shapes differ")
    code = kv_dtype_code(k_cache)
    if kv_dtype_code(v_cache) != code:
        raise TypeError("k_cache and v_cache formats differ")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV pool views must be contiguous")
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    if code == _lib.KV_FP8_E4M3FN:
        if k_scale is None or v_scale is None:
            raise ValueError("an E4M3FN pool needs k_scale and v_scale")
        for s in (k_scale, v_scale):
            if s.dtype != torch.float32 or not s.is_contiguous() or s.numel() != num_slots * num_heads:
                raise ValueError("scale pools must be contiguous fp32 [num_blocks, block_size, num_kv_heads]")
    _int32(slot_mapping, "slot_mapping")
    return device, code


def foldable(key: torch.Tensor, value: torch.Tensor) -> bool:
    """Whether the attention launch can carry the KV write of these new rows:
    bf16 ``[N, num_kv_heads, head_dim]`` rows stored back to back."""
    row = key.shape[1] * key.shape[2]
    return (key.dim() == 3 and key.dtype == torch.bfloat16 and value.dtype == torch.bfloat16
            and key.stride(0) == row and value.stride(0) == row and key.stride(2) == 1 and value.stride(2) == 1
            and key.stride(1) == key.shape[2] and value.stride(1) == value.shape[2])


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                  k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None,
                  scale_floor: float = _lib.FP8_SCALE_FLOOR) -> None:
    """Slot-mapped KV write (nanovllm/layers/attention.py:33-40), bf16 or E4M3FN.

    ``key``/``value``: ``[N, num_kv_heads, head_dim]`` bf16 whose rows may be
    strided (a view of the fused QKV output).  ``k_cache``/``v_cache``:
    ``[num_blocks, block_size, num_kv_heads, head_dim]``; for E4M3FN caches
    (uint8 or float8_e4m3fn) ``k_scale``/``v_scale`` are the fp32
    ``[num_blocks, block_size, num_kv_heads]`` scale pools.
    """
    device, code = check_store(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale)
    N, num_heads, head_dim = key.shape
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    lib = _lib.load()
    _lib.check(lib.slo_store_kvcache(
        _ptr(key), key.stride(0), _ptr(value), value.stride(0), _ptr(slot_mapping), N, num_heads,
        head_dim, code, _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), num_slots,
        float(scale_floor), _stream(device)), "slo_store_kvcache")


# ------------------------------------------- fused q/k norm + RoPE + KV write
def rope_cos_sin(head_dim: int, max_position: int, base: float, device) -> torch.Tensor:
    """fp32 [max_position, head_dim] table: cos(p * inv_freq) then sin(p * inv_freq).

    The cos_sin_cache of RotaryEmbedding (nanovllm/layers/rotary_embedding.py:27-35),
    built with the same torch operations on ``device``.
    """
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float, device=device) / head_dim))
    t = torch.arange(max_position, dtype=torch.float, device=device)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).contiguous()


def qk_norm_rope_store(qkv: torch.Tensor, positions: torch.Tensor, q_norm_weight: torch.Tensor,
                       k_norm_weight: torch.Tensor, eps: float, cos_sin: torch.Tensor, num_heads: int,
                       num_kv_heads: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       slot_mapping: torch.Tensor, k_scale: torch.Tensor | None = None,
                       v_scale: torch.Tensor | None = None, head_dim: int = 128,
                       scale_floor: float = _lib.FP8_SCALE_FLOOR):
    """q_norm, k_norm, rotary_emb and the KV write of one layer in one launch.

    Covers nanovllm/models/qwen3.py:80-86 up to the attention call, and the
    store_kvcache that Attention.forward would issue (attention.py:59-66).
    ``qkv``: ``[N, (num_heads + 2*num_kv_heads) * head_dim]`` bf16 (the fused
    projection output; rows may be strided).  Returns ``(q, k, v)``: q and k
    normalised and rotated (new contiguous bf16 tensors), v a view of ``qkv``.
    The pool receives the rotated k and v at ``slot_mapping`` (bf16 or
    E4M3FN with ``k_scale``/``v_scale``), as ``store_kvcache`` writes them.
    """
    if qkv.dim() != 2 or qkv.stride(-1) != 1:
        raise ValueError("qkv must be a [tokens, width] tensor with contiguous rows")
    N = qkv.shape[0]
    width = (num_heads + 2 * num_kv_heads) * head_dim
    if qkv.shape[1] != width:
        raise ValueError(f"qkv rows must hold {width} elements")
    device = _require_gpu(qkv, positions, q_norm_weight, k_norm_weight, cos_sin, k_cache, v_cache,
                          slot_mapping, k_scale, v_scale)
    if qkv.dtype != torch.bfloat16:
        raise TypeError("qkv must be bf16")
    if positions.dtype != torch.int64 or positions.numel() != N or not positions.is_contiguous():
        raise ValueError("positions must be a contiguous int64 [tokens] tensor")
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w.dtype != torch.bfloat16 or w.numel() != head_dim or not w.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bf16 [head_dim] tensor")
    if cos_sin.dtype != torch.float32 or cos_sin.dim() != 2 or cos_sin.shape[1] != head_dim or \
            not cos_sin.is_contiguous():
        raise ValueError("cos_sin must be a contiguous fp32 [max_position, head_dim] table")
    code = kv_dtype_code(k_cache)
    if kv_dtype_code(v_cache) != code:
        raise TypeError("k_cache and v_cache formats differ")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV pool views must be contiguous")
    if k_cache.shape[-2:] != (num_kv_heads, head_dim) or v_cache.shape != k_cache.shape:
        raise ValueError("KV pool must be [num_blocks, block_size, num_kv_heads, head_dim]")
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    if code == _lib.KV_FP8_E4M3FN:
        if k_scale is None or v_scale is None:
            raise ValueError("an E4M3FN pool needs k_scale and v_scale")
        for sc in (k_scale, v_scale):
            if sc.dtype != torch.float32 or not sc.is_contiguous() or sc.numel() != num_slots * num_kv_heads:
                raise ValueError("scale pools must be contiguous fp32 [num_blocks, block_size, num_kv_heads]")
    _int32(slot_mapping, "slot_mapping")
    if slot_mapping.numel() != N:
        raise ValueError("slot_mapping must hold one slot per token")
    q = torch.empty((N, num_heads, head_dim), dtype=torch.bfloat16, device=qkv.device)
    k = torch.empty((N, num_kv_heads, head_dim), dtype=torch.bfloat16, device=qkv.device)
    _lib.check(_lib.load().slo_qk_norm_rope_store(
        _ptr(qkv), qkv.stride(0), _ptr(positions), N, num_heads, num_kv_heads, head_dim, _ptr(q_norm_weight),
        _ptr(k_norm_weight), float(eps), _ptr(cos_sin), cos_sin.shape[0], _ptr(q), _ptr(k), _ptr(slot_mapping),
        code, _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), num_slots, float(scale_floor),
        _stream(device)), "slo_qk_norm_rope_store")
    v = qkv[:, (num_heads + num_kv_heads) * head_dim:].view(N, num_kv_heads, head_dim)
    return q, k, v


# ------------------------------------------------------ LM head + greedy argmax
_keys: dict[int, torch.Tensor] = {}
LM_HEAD_MAX_ROWS = 128


def lm_head_argmax(hidden: torch.Tensor, weight: torch.Tensor, return_logits: bool = False):
    """Greedy next tokens of the sampled rows: argmax_v bf16(hidden[r] . weight[v]).

    compute_logits + argmax of run_mixed (nanovllm/engine/mixed_model_runner.py:
    115-126, nanovllm/layers/embed_head.py:56-66) in one pass over the weight.
    ``hidden``: ``[rows, hidden_size]`` bf16 (the already-selected sampled rows,
    at most 128); ``weight``: ``[vocab, hidden_size]`` bf16.  Returns int64
    ``[rows]`` tokens (ties: the smallest index), and the bf16 logits
    ``[rows, vocab]`` as well when ``return_logits``.
    """
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("hidden must be [rows, hidden_size] and weight [vocab, hidden_size]")
    device = _require_gpu(hidden, weight)
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("hidden and weight must be bf16")
    if hidden.stride(-1) != 1 or weight.stride(-1) != 1:
        raise ValueError("hidden and weight rows must be contiguous")
    rows, vocab = hidden.shape[0], weight.shape[0]
    if rows > LM_HEAD_MAX_ROWS:
        raise ValueError(f"at most {LM_HEAD_MAX_ROWS} sampled rows per call")
    index = device.index if device.index is not None else torch.cuda.current_device()
    keys = _keys.get(index)
    if keys is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("call lm_head_argmax once before graph capture")
        keys = torch.zeros(LM_HEAD_MAX_ROWS, dtype=torch.int64, device=device)
        _keys[index] = keys
    tokens = torch.empty(rows, dtype=torch.int64, device=device)
    logits = torch.empty(rows, vocab, dtype=torch.bfloat16, device=device) if return_logits else None
    _lib.check(_lib.load().slo_lm_head_argmax(
        _ptr(hidden), hidden.stride(0), rows, _ptr(weight), weight.stride(0), vocab, hidden.shape[1], _ptr(logits),
        vocab, _ptr(keys), _ptr(tokens), _stream(device)), "slo_lm_head_argmax")
    return (tokens, logits) if return_logits else tokens


# ---------------------------------------------------------------- workspace
_ws_lock = threading.Lock()
_workspaces: dict[int, torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device zero-initialised workspace of at least ``nbytes`` bytes.

    The kernels leave the control words and split-K tickets at zero when they
    finish, so the buffer is zero-filled only when it is (re)allocated.
    Growing is refused while a graph is being captured.
    """
    index = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        ws = _workspaces.get(index)
        if ws is not None and ws.numel() >= nbytes:
            return ws
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("attention workspace must be reserved before graph capture "
                               "(call reserve_workspace)")
        size = max(nbytes, int((ws.numel() if ws is not None else 0) * 1.5), 1 << 20)
        ws = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", index))
        _workspaces[index] = ws
        return ws


def check_workspaces() -> None:
    """Raise if any device's attention workspace is not in the state every
    launch leaves it in (work-list counters and split-K tickets zero), or if a
    split-K merge gave up waiting since the last check (its decode outputs were
    not written).  Synchronises the current stream of each device; call it
    outside graph capture, e.g. every few hundred steps of a serving loop."""
    for index, ws in list(_workspaces.items()):
        device = torch.device("cuda", index)
        _lib.check(_lib.load().slo_attention_workspace_check(ws.data_ptr(), ws.numel(), None, _stream(device)),
                   "slo_attention_workspace_check")


def workspace_events(device) -> dict:
    """Reads and clears the attention workspace's event counters on ``device``
    (after checking its zero invariants): ``merges_gave_up`` (split-K merge
    tasks that stopped waiting) and ``split_prefill_merges`` (split prefill
    item pairs merged).  Raises like ``check_workspaces`` when a merge gave up.
    Synchronises; a diagnostic for tests and tuning."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    ws = _workspaces.get(index)
    if ws is None:
        return {"merges_gave_up": 0, "split_prefill_merges": 0}
    ev = (ctypes.c_uint32 * 4)()
    _lib.check(_lib.load().slo_attention_workspace_check(ws.data_ptr(), ws.numel(), ev, _stream(device)),
               "slo_attention_workspace_check")
    return {"merges_gave_up": int(ev[0]), "split_prefill_merges": int(ev[1])}


def reserve_workspace(device, max_decode_rows: int, max_decode_len: int, num_heads: int,
                      num_kv_heads: int, head_dim: int) -> torch.Tensor:
    nbytes = _lib.workspace_bytes(max_decode_rows, max_decode_len, num_heads, num_kv_heads, head_dim)
    return workspace(torch.device(device), nbytes)


# ---------------------------------------------------------------- attention
def paged_attention(q: torch.Tensor, k_cache: torch.Tensor | None, v_cache: torch.Tensor | None,
                    softmax_scale: float, *, num_kv_heads: int,
                    k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None,
                    num_decode: int = 0, decode_lens: torch.Tensor | None = None,
                    decode_tables: torch.Tensor | None = None,
                    num_prefill: int = 0, prefill_cu_q: torch.Tensor | None = None,
                    prefill_cu_k: torch.Tensor | None = None, max_q: int = 0, max_k: int = 0,
                    prefill_tables: torch.Tensor | None = None,
                    k: torch.Tensor | None = None, v: torch.Tensor | None = None,
                    phases: int = _lib.PHASE_ALL, out: torch.Tensor | None = None,
                    store_slot_mapping: torch.Tensor | None = None, new_k: torch.Tensor | None = None,
                    new_v: torch.Tensor | None = None, noalloc: bool = False,
                    store_scale_floor: float = _lib.FP8_SCALE_FLOOR) -> torch.Tensor:
    """One ragged launch: decode rows ``q[:num_decode]``, then prefill rows.

    Decode row b attends to ``decode_lens[b]`` cached tokens through
    ``decode_tables[b]``.  Prefill row r owns query rows
    ``num_decode + [cu_q[r], cu_q[r+1])`` and attends causally, bottom-right
    aligned, to ``cu_k[r+1]-cu_k[r]`` keys from the pool (``prefill_tables``)
    or, with ``prefill_tables=None``, from the contiguous ``k``/``v`` rows
    starting at ``cu_k[r]``.  Returns ``out`` ``[q rows, num_heads, head_dim]``.

    With ``store_slot_mapping``, the same launch also writes ``new_k``/``new_v``
    (one row per query row: decode tokens, then prefill tokens) to their slots,
    the store of forward_mixed folded in, and reads the step's new tokens from
    those rows; the result is the separate store followed by the launch, bit
    for bit.  With an E4M3FN pool the write is ``store_kvcache``'s quantising
    store (``store_scale_floor``), the new tokens are read as its codes and
    scales, and at most 8 query heads may share a kv head.

    ``noalloc=True`` launches through ``slo_paged_attention_noalloc``, which
    uses the library's static per-GPU scratch instead of this module's
    workspace (pass ``out`` as well and nothing is allocated).
    """
    if q.dim() != 3:
        raise ValueError("q must be [tokens, num_heads, head_dim]")
    T, num_heads, head_dim = q.shape
    device = _require_gpu(q, k_cache, v_cache, k_scale, v_scale, decode_lens, decode_tables,
                          prefill_cu_q, prefill_cu_k, prefill_tables, k, v, out)
    if q.dtype != torch.bfloat16:
        raise TypeError("q must be bf16")
    if q.stride(-1) != 1 or q.stride(1) != head_dim:
        raise ValueError("q rows must hold contiguous heads")
    if out is None:
        out = torch.empty((T, num_heads, head_dim), dtype=torch.bfloat16, device=q.device)
    elif out.shape != (T, num_heads, head_dim) or out.stride(-1) != 1 or out.stride(1) != head_dim:
        raise ValueError("out must be [tokens, num_heads, head_dim] with contiguous heads")
    args = _lib.PagedAttentionArgs()
    args.q, args.q_row_stride = q.data_ptr(), q.stride(0)
    args.out, args.out_row_stride = out.data_ptr(), out.stride(0)
    args.num_q_rows = T
    code = _lib.KV_BF16
    if k_cache is not None and k_cache.numel():
        code = kv_dtype_code(k_cache)
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("KV pool views must be contiguous")
        if k_cache.dim() != 4 or k_cache.shape[2] != num_kv_heads or k_cache.shape[3] != head_dim:
            raise ValueError("KV pool must be [num_blocks, block_size, num_kv_heads, head_dim]")
        args.k_cache, args.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
        args.num_blocks, args.block_size = k_cache.shape[0], k_cache.shape[1]
        if code == _lib.KV_FP8_E4M3FN:
            if k_scale is None or v_scale is None:
                raise ValueError("an E4M3FN pool needs k_scale and v_scale")
            args.k_scale, args.v_scale = k_scale.data_ptr(), v_scale.data_ptr()
    args.kv_dtype = code
    decode_cap_len = 0
    if num_decode:
        _int32(decode_lens, "decode_lens")
        _int32(decode_tables, "decode_tables")
        if decode_tables.dim() != 2 or decode_tables.stride(1) != 1:
            raise ValueError("decode_tables must be a row-major [rows, width] int32 tensor")
        if decode_lens.numel() < num_decode or decode_tables.shape[0] < num_decode:
            raise ValueError("decode metadata has fewer rows than num_decode")
        args.num_decode = num_decode
        args.decode_lens = decode_lens.data_ptr()
        args.decode_tables = decode_tables.data_ptr()
        args.decode_table_stride = decode_tables.stride(0)
        args.decode_table_width = decode_tables.shape[1]
        decode_cap_len = decode_tables.shape[1] * args.block_size
    if num_prefill:
        _int32(prefill_cu_q, "cu_seqlens_q")
        _int32(prefill_cu_k, "cu_seqlens_k")
        if prefill_cu_q.numel() < num_prefill + 1 or prefill_cu_k.numel() < num_prefill + 1:
            raise ValueError("cu_seqlens shorter than num_prefill + 1")
        args.num_prefill = num_prefill
        args.prefill_cu_q, args.prefill_cu_k = prefill_cu_q.data_ptr(), prefill_cu_k.data_ptr()
        args.max_q, args.max_k = int(max_q), int(max_k)
        if prefill_tables is not None:
            _int32(prefill_tables, "block_tables")
            if prefill_tables.dim() != 2 or prefill_tables.stride(1) != 1:
                raise ValueError("block_tables must be a row-major [rows, width] int32 tensor")
            args.prefill_tables = prefill_tables.data_ptr()
            args.prefill_table_stride = prefill_tables.stride(0)
            args.prefill_table_width = prefill_tables.shape[1]
        else:
            if k is None or v is None:
                raise ValueError("prefill without block tables needs contiguous k and v")
            for name, t in (("k", k), ("v", v)):
                if t.dtype != torch.bfloat16 or t.stride(-1) != 1 or t.stride(1) != head_dim:
                    raise ValueError(f"{name} must be bf16 [tokens, num_kv_heads, head_dim] rows")
            args.k, args.k_row_stride = k.data_ptr(), k.stride(0)
            args.v, args.v_row_stride = v.data_ptr(), v.stride(0)
            args.num_kv_rows = min(k.shape[0], v.shape[0])
    if store_slot_mapping is not None:
        check_store(new_k, new_v, k_cache, v_cache, store_slot_mapping, k_scale, v_scale)
        if code != _lib.KV_BF16 and num_heads > 8 * num_kv_heads:
            raise ValueError("the E4M3FN KV write in the attention launch needs <= 8 query heads per kv head")
        if new_k.shape[0] != T or new_k.shape[1] != num_kv_heads or new_k.shape[2] != head_dim:
            raise ValueError("new_k/new_v must hold one [num_kv_heads, head_dim] row per query row")
        args.k_cache, args.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
        args.num_blocks, args.block_size = k_cache.shape[0], k_cache.shape[1]
        args.store_slot_mapping = store_slot_mapping.data_ptr()
        args.new_k, args.new_k_row_stride = new_k.data_ptr(), new_k.stride(0)
        args.new_v, args.new_v_row_stride = new_v.data_ptr(), new_v.stride(0)
        args.num_new_rows = T
        args.store_scale_floor = float(store_scale_floor)
    args.num_heads, args.num_kv_heads, args.head_dim = num_heads, num_kv_heads, head_dim
    args.softmax_scale = float(softmax_scale)
    args.phases = int(phases)
    if noalloc:
        args.workspace, args.workspace_bytes = None, 0
        _lib.check(_lib.load().slo_paged_attention_noalloc(ctypes.byref(args), _stream(device)),
                   "slo_paged_attention_noalloc")
        return out
    need = _lib.workspace_bytes(num_decode if (phases & _lib.PHASE_DECODE) else 0,
                                decode_cap_len, num_heads, num_kv_heads, head_dim)
    ws = workspace(device, need)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(_lib.load().slo_paged_attention(ctypes.byref(args), _stream(device)),
               "slo_paged_attention")
    return out
