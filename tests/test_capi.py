"""The C-ABI library on the CPU: it loads, exports every declared symbol,
validates arguments without touching a GPU, and the host layer refuses to run
without it (no CPU fallback)."""
import ctypes
import os
import re

import pytest
import torch

from slo_attn import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "slo_attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(slo_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert set(names) == set(_lib.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name


def test_args_struct_layout_matches_header():
    lib = _lib.load()
    assert lib.slo_paged_attention_args_size() == ctypes.sizeof(_lib.PagedAttentionArgs)


def test_workspace_bytes_and_errors():
    n1 = _lib.workspace_bytes(24, 4096, 32, 8, 128)
    n2 = _lib.workspace_bytes(48, 4096, 32, 8, 128)
    n0 = _lib.workspace_bytes(0, 0, 32, 8, 128)
    # control lines + trash line + ticket array are fixed; partials grow with rows x chunks x heads:
    # one record of G x (128 accumulators + m + l + 2 pad) floats per chunk of at least 128 tokens
    per_item = 4 * (128 + 4) * 4
    assert n2 - n1 == 24 * (4096 // 128) * 8 * per_item
    # control lines, trash and event line, 65536 tickets and 48 MiB of split prefill records
    assert n0 == 24 * 128 + 1024 + 4 * 65536 + (48 << 20)
    with pytest.raises(RuntimeError, match="head_dim"):
        _lib.workspace_bytes(1, 1, 32, 8, 64)
    with pytest.raises(RuntimeError):
        _lib.workspace_bytes(1, 1, 30, 8, 128)


def test_entry_points_reject_bad_arguments_without_a_gpu():
    lib = _lib.load()
    assert lib.slo_paged_attention(None, None) == 1
    assert "null args" in lib.slo_last_error().decode()
    args = _lib.PagedAttentionArgs()
    args.head_dim, args.num_heads, args.num_kv_heads = 64, 32, 8
    assert lib.slo_paged_attention(ctypes.byref(args), None) == 4
    args.head_dim, args.num_heads = 128, 31
    assert lib.slo_paged_attention(ctypes.byref(args), None) == 1
    args.num_heads, args.kv_dtype = 32, 0
    # nothing to do -> OK with no device work
    assert lib.slo_paged_attention(ctypes.byref(args), None) == 0
    # a pooled decode row with a block size that is not a multiple of 64 is refused
    # before any pointer is touched (the pointers below are never dereferenced)
    args.num_decode, args.num_q_rows, args.block_size, args.num_blocks, args.phases = 1, 1, 100, 1, 3
    args.q = args.out = args.k_cache = args.v_cache = 4096
    args.workspace = 8192
    assert lib.slo_paged_attention(ctypes.byref(args), None) == 4
    assert "block_size" in lib.slo_last_error().decode()
    # a contiguous prefill row whose K rows are closer than num_kv_heads * 128
    # elements is refused (the pointers are never dereferenced)
    cu = (ctypes.c_int32 * 2)(0, 64)
    args.num_decode, args.num_prefill, args.num_q_rows, args.phases = 0, 1, 64, 3
    args.prefill_cu_q = args.prefill_cu_k = ctypes.cast(cu, ctypes.c_void_p).value
    args.k = args.v = 4096
    args.k_row_stride, args.v_row_stride = 8 * 128 - 8, 8 * 128
    assert lib.slo_paged_attention(ctypes.byref(args), None) == 1
    assert "num_kv_heads * 128" in lib.slo_last_error().decode()
    args.num_prefill, args.num_decode = 0, 1
    # the workspace check refuses a missing or too small workspace before any HIP call
    assert lib.slo_attention_workspace_check(None, 1 << 20, None, None) == 1
    assert lib.slo_attention_workspace_check(8192, 1024, None, None) == 1
    assert "control area" in lib.slo_last_error().decode()
    assert lib.slo_store_kvcache(None, 0, None, 0, None, 0, 8, 128, 0, None, None, None, None, 0, 1.0, None) == 0
    assert lib.slo_store_kvcache(None, 0, None, 0, None, 4, 8, 96, 0, None, None, None, None, 0, 1.0, None) == 4
    assert lib.slo_store_kvcache(None, 0, None, 0, None, 4, 8, 128, 0, None, None, None, None, 0, 1.0, None) == 1


def test_host_layer_refuses_cpu_tensors():
    from slo_attn import paged_attention, store_kvcache
    q = torch.zeros(2, 32, 128, dtype=torch.bfloat16)
    kc = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        paged_attention(q, kc, kc, 0.1, num_kv_heads=8, num_decode=2,
                        decode_lens=torch.ones(2, dtype=torch.int32),
                        decode_tables=torch.zeros(2, 1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        store_kvcache(torch.zeros(2, 8, 128, dtype=torch.bfloat16), torch.zeros(2, 8, 128, dtype=torch.bfloat16),
                      kc, kc, torch.zeros(2, dtype=torch.int32))


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libslo_attn.so")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()
