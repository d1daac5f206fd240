"""KV pool allocation for bf16 or E4M3FN caches, and the block lifecycle helpers.

The runner's allocate_kv_cache (nanovllm/engine/model_runner.py:103-121,
nanovllm/engine/mixed_model_runner.py:17-47) sizes the pool by

    block_bytes = 2 * layers * block_size * kv_heads * head_dim * itemsize
    blocks = (total * gpu_memory_utilization - used - peak + current) // block_bytes

and hands each attention layer the views ``pool[0, l]`` / ``pool[1, l]`` of
one ``[2, layers, blocks, block_size, kv_heads, head_dim]`` tensor.  The
quantised pool of docs/project_manual.md:527-563,583 keeps that layout with
E4M3FN code bytes and adds one fp32 scale per (token, kv head), K and V each:
``[2, layers, blocks, block_size, kv_heads]`` (the scale layout of
docs/project_manual.md:174-189), so a block costs
``2 * layers * block_size * kv_heads * (head_dim + 4)`` bytes instead of
``... * head_dim * 2`` -- 264 against 512 bytes per token and kv head at
head_dim 128 (docs/project_manual.md:548-556).

Lifecycle (docs/project_manual.md:591-602): a block's code bytes and scales
are one cache object, so copying a block (copy-on-write of a shared tail) or
snapshotting it moves both, and a block taken back into use has its scales
reset with its bytes.  The store kernels write every (token, kv head) scale
together with its codes, and attention reads only tokens below a row's
length, so stale scales beyond a row's valid tokens are never read.
"""
from __future__ import annotations

import torch

from . import _lib

_KV_FORMATS = {"bf16": _lib.KV_BF16, "fp8_e4m3fn": _lib.KV_FP8_E4M3FN}


def kv_block_bytes(num_layers: int, block_size: int, num_kv_heads: int, head_dim: int,
                   kv_format: str = "bf16") -> int:
    """Bytes of one block across all layers, K and V, scales included."""
    if kv_format == "bf16":
        return 2 * num_layers * block_size * num_kv_heads * head_dim * 2
    if kv_format == "fp8_e4m3fn":
        return 2 * num_layers * block_size * num_kv_heads * (head_dim + 4)
    raise ValueError(f"unknown KV format {kv_format!r}")


def num_kv_blocks(total: int, used: int, peak: int, current: int, gpu_memory_utilization: float,
                  block_bytes: int, cap: int | None = None) -> int:
    """Block count of allocate_kv_cache (mixed_model_runner.py:20-33), optionally capped."""
    count = int(total * gpu_memory_utilization - used - peak + current) // block_bytes
    if cap is not None:
        count = min(count, cap)
    return count


class KVPool:
    """One pool for all layers: codes or bf16 values, and fp32 scales for E4M3FN.

    ``kv``    ``[2, layers, blocks, block_size, kv_heads, head_dim]`` bf16 or uint8
    ``scale`` ``[2, layers, blocks, block_size, kv_heads]`` fp32 (E4M3FN only)
    """

    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                 kv_format: str = "bf16", device=None):
        if kv_format not in _KV_FORMATS:
            raise ValueError(f"unknown KV format {kv_format!r}")
        if num_blocks <= 0:
            raise RuntimeError("no KV blocks available")
        self.kv_format = kv_format
        self.num_layers, self.num_blocks, self.block_size = num_layers, num_blocks, block_size
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim
        shape = (2, num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        if kv_format == "bf16":
            self.kv = torch.empty(shape, dtype=torch.bfloat16, device=device)
            self.scale = None
        else:
            self.kv = torch.zeros(shape, dtype=torch.uint8, device=device)
            self.scale = torch.ones(shape[:-1], dtype=torch.float32, device=device)

    @classmethod
    def for_memory(cls, num_layers: int, block_size: int, num_kv_heads: int, head_dim: int, kv_format: str,
                   gpu_memory_utilization: float = 0.9, cap: int | None = None, device=None) -> "KVPool":
        """Sizes the pool from the device's free memory like allocate_kv_cache."""
        device = torch.device(device if device is not None else "cuda")
        free, total = torch.cuda.mem_get_info(device)
        stats = torch.cuda.memory_stats(device)
        count = num_kv_blocks(total, total - free, stats["allocated_bytes.all.peak"],
                              stats["allocated_bytes.all.current"], gpu_memory_utilization,
                              kv_block_bytes(num_layers, block_size, num_kv_heads, head_dim, kv_format), cap)
        return cls(num_layers, count, block_size, num_kv_heads, head_dim, kv_format, device)

    @property
    def fp8(self) -> bool:
        return self.scale is not None

    def layer(self, l: int):
        """(k_cache, v_cache, k_scale, v_scale) views of layer ``l`` (scales None for bf16)."""
        if self.scale is None:
            return self.kv[0, l], self.kv[1, l], None, None
        return self.kv[0, l], self.kv[1, l], self.scale[0, l], self.scale[1, l]

    def attach(self, model) -> int:
        """Assigns each layer's views to the modules that have ``k_cache``/``v_cache``, in order
        (mixed_model_runner.py:43-47); E4M3FN pools also set ``k_scale``/``v_scale``.
        Returns the number of layers attached."""
        layer = 0
        modules = model.modules() if hasattr(model, "modules") else model
        for module in modules:
            if hasattr(module, "k_cache") and hasattr(module, "v_cache"):
                if layer >= self.num_layers:
                    raise ValueError("more attention layers than pool layers")
                module.k_cache, module.v_cache, k_scale, v_scale = self.layer(layer)
                if self.scale is not None or hasattr(module, "k_scale"):
                    module.k_scale, module.v_scale = k_scale, v_scale
                layer += 1
        return layer

    # ------------------------------------------------------------- lifecycle
    def copy_blocks(self, src: list[int], dst: list[int]) -> None:
        """Copies whole blocks (codes and scales, every layer): copy-on-write of a shared block."""
        if len(src) != len(dst) or len(set(dst)) != len(dst) or set(src) & set(dst):
            raise ValueError("copy_blocks needs distinct destination blocks, disjoint from the sources")
        s = torch.as_tensor(src, dtype=torch.long, device=self.kv.device)
        d = torch.as_tensor(dst, dtype=torch.long, device=self.kv.device)
        self.kv[:, :, d] = self.kv[:, :, s]
        if self.scale is not None:
            self.scale[:, :, d] = self.scale[:, :, s]

    def reset_blocks(self, blocks: list[int]) -> None:
        """Returns blocks to the initial state (codes 0, scales 1) before reuse."""
        b = torch.as_tensor(blocks, dtype=torch.long, device=self.kv.device)
        self.kv[:, :, b] = 0
        if self.scale is not None:
            self.scale[:, :, b] = 1.0

    def snapshot(self, blocks: list[int]) -> dict:
        """Host copy of whole blocks, codes and scales (the geometry-aware form of
        diagnostics/online_token_replay/tensors.py:11-35)."""
        b = torch.as_tensor(blocks, dtype=torch.long, device=self.kv.device)
        return {"block_ids": list(blocks), "kv_format": self.kv_format,
                "kv": self.kv[:, :, b].cpu(), "scale": None if self.scale is None else self.scale[:, :, b].cpu(),
                "pool_shape": list(self.kv.shape)}

    def restore(self, image: dict) -> None:
        if image["kv_format"] != self.kv_format or image["pool_shape"] != list(self.kv.shape):
            raise ValueError("snapshot geometry or format differs from this pool")
        b = torch.as_tensor(image["block_ids"], dtype=torch.long, device=self.kv.device)
        self.kv[:, :, b] = image["kv"].to(self.kv.device)
        if self.scale is not None:
            self.scale[:, :, b] = image["scale"].to(self.kv.device)
