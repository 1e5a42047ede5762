"""Physical paged KV pool (reference: mini_vllm/cache/pool.py:38-278).

One K tensor and one V tensor per layer, each
``[num_blocks, num_kv_heads, block_size, head_dim]`` and contiguous, so that
the (block, kv head) tile of ``block_size * head_dim`` elements the decode
kernel streams is one contiguous run of HBM. Dimension 0 is the physical
block id that block tables and slot mappings refer to. Storage comes from
``torch.empty``: only slots named by a slot mapping are ever written and
the kernels read only the first ``kv_len`` tokens of a sequence.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch

MIN_BLOCKS = 16
"""Smallest pool ``compute_num_gpu_blocks`` returns (reference pool.py:26)."""

_WORKSPACE_RESERVE = 256 * 1024 * 1024


def _default_device() -> torch.device:
    return torch.device("cuda" if torch.cuda.is_available() else "cpu")


@dataclass
class KVCachePool:
    key_caches: List[torch.Tensor]
    value_caches: List[torch.Tensor]
    num_blocks: int
    block_size: int
    num_layers: int
    num_kv_heads: int
    head_dim: int
    device: torch.device
    dtype: torch.dtype

    @staticmethod
    def allocate(
        num_layers: int,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype = torch.float16,
        device: Optional[torch.device] = None,
    ) -> "KVCachePool":
        """Allocate uninitialised per-layer K/V tensors (reference pool.py:64-114).

        Raises ``ValueError`` naming the first non-positive size.
        """
        for name, value in (
            ("num_blocks", num_blocks),
            ("num_layers", num_layers),
            ("block_size", block_size),
            ("num_kv_heads", num_kv_heads),
            ("head_dim", head_dim),
        ):
            if value <= 0:
                raise ValueError(f"{name} must be > 0, got {value}")
        dev = torch.device(device) if device is not None else _default_device()
        shape = (num_blocks, num_kv_heads, block_size, head_dim)
        keys = [torch.empty(shape, dtype=dtype, device=dev) for _ in range(num_layers)]
        values = [torch.empty(shape, dtype=dtype, device=dev) for _ in range(num_layers)]
        return KVCachePool(keys, values, num_blocks, block_size, num_layers,
                           num_kv_heads, head_dim, dev, dtype)

    def get_key_cache(self, layer_idx: int) -> torch.Tensor:
        return self.key_caches[layer_idx]

    def get_value_cache(self, layer_idx: int) -> torch.Tensor:
        return self.value_caches[layer_idx]

    def reset(self) -> None:
        """Zero every layer's K and V."""
        for t in (*self.key_caches, *self.value_caches):
            t.zero_()

    @property
    def total_slots(self) -> int:
        """Token slots per layer: ``num_blocks * block_size``."""
        return self.num_blocks * self.block_size

    @property
    def bytes_per_block_per_layer(self) -> int:
        """K plus V bytes of one block in one layer."""
        itemsize = torch.empty((), dtype=self.dtype).element_size()
        return 2 * self.num_kv_heads * self.block_size * self.head_dim * itemsize

    @property
    def bytes_per_block_total(self) -> int:
        return self.num_layers * self.bytes_per_block_per_layer

    @property
    def total_bytes(self) -> int:
        return self.num_blocks * self.bytes_per_block_total


def compute_num_gpu_blocks(
    num_layers: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    dtype: torch.dtype = torch.float16,
    device: Optional[torch.device] = None,
    gpu_memory_utilization: float = 0.90,
    peak_runtime_estimate: int = 0,
    workspace_reserve: int = _WORKSPACE_RESERVE,
    num_gpu_blocks_override: Optional[int] = None,
) -> int:
    """Number of pool blocks that fit in free device memory.

    Same budget rule as the reference (pool.py:174-278): the free bytes
    reported by the device, minus the runtime estimate and a fixed
    workspace reserve, times ``gpu_memory_utilization``, divided by the K+V
    bytes of one block across all layers; never below ``MIN_BLOCKS``. On a
    CPU device it returns ``MIN_BLOCKS``. On one MI355X (288 GB HBM3E) the
    Qwen2-0.5B pool (24 layers, 2 kv heads, head_dim 64, block 16, bf16:
    196608 bytes per block) holds about 1.3 M blocks, i.e. 21 M tokens.
    """
    if not 0 < gpu_memory_utilization <= 1.0:
        raise ValueError(
            f"gpu_memory_utilization must be in (0, 1], got {gpu_memory_utilization}"
        )
    if num_gpu_blocks_override is not None:
        if num_gpu_blocks_override < MIN_BLOCKS:
            raise RuntimeError(
                f"num_gpu_blocks_override ({num_gpu_blocks_override}) < minimum ({MIN_BLOCKS})"
            )
        return num_gpu_blocks_override
    dev = torch.device(device) if device is not None else _default_device()
    if dev.type != "cuda":
        return MIN_BLOCKS
    free_bytes, _ = torch.cuda.mem_get_info(dev)
    usable = free_bytes - peak_runtime_estimate - workspace_reserve
    if usable <= 0:
        raise RuntimeError(
            f"GPU memory exhausted after deductions: free={free_bytes}, "
            f"peak={peak_runtime_estimate}, workspace={workspace_reserve}"
        )
    itemsize = torch.empty((), dtype=dtype).element_size()
    per_block = num_layers * 2 * num_kv_heads * block_size * head_dim * itemsize
    return max(MIN_BLOCKS, int(usable * gpu_memory_utilization) // per_block)
