"""Attention plugin interface (reference: mini_vllm/attention/backend.py:12-113).

The model runner talks to attention only through this ABC, created by
``AttentionBackend.create(model_config, backend=config.attention_backend)``
(reference call site: mini_vllm/executor/paged_executor.py:47-49):

* ``allocate_pool``  — the physical paged KV pool, once at start-up;
* ``write_kv_cache`` — scatter of the step's new K/V rows by slot, per layer;
* ``decode_attention`` — paged decode over each sequence's block table;
* ``prefill_attention`` — attention of prefill chunks over prefix + chunk.

This package implements one backend, the HIP backend for gfx950
(``AttentionBackendGPU``). ``"hip"`` is its name and ``"triton"`` — the name
the reference's configs and tests use for the GPU backend — selects the same
class. ``"reference"`` / ``"ref"`` keep the reference's meaning: the PyTorch
test backend ``AttentionBackendRef``, imported lazily from the sibling module
``paged_attention_ref`` that the reference tree provides (this package does
not ship that module; where it is absent the import error propagates).
There is no fallback: an unknown name raises ``ValueError`` and a missing GPU
or kernel library raises ``RuntimeError`` at creation.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING, Any

import torch

if TYPE_CHECKING:
    from ..model_runner.base import AttentionMetadata, ModelConfig

GPU_BACKEND_NAMES = ("hip", "triton")
REFERENCE_BACKEND_NAMES = ("reference", "ref")


class AttentionBackend(ABC):
    @abstractmethod
    def allocate_pool(
        self,
        num_layers: int,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device,
    ) -> Any:
        """Allocate the per-layer K/V pool; returns a ``KVCachePool``."""

    @abstractmethod
    def write_kv_cache(
        self,
        layer_idx: int,
        key: torch.Tensor,           # [num_tokens, num_kv_heads, head_dim]
        value: torch.Tensor,         # [num_tokens, num_kv_heads, head_dim]
        slot_mapping: torch.Tensor,  # [num_tokens] int64, -1 = skip
    ) -> None:
        """Scatter-write the tokens' K/V rows into layer ``layer_idx``."""

    @abstractmethod
    def decode_attention(
        self,
        layer_idx: int,
        query: torch.Tensor,  # [num_decode_tokens, num_heads, head_dim]
        attn_metadata: "AttentionMetadata",
        pool: Any,
    ) -> torch.Tensor:
        """Paged decode attention; returns ``[num_decode, num_heads, head_dim]``."""

    @abstractmethod
    def prefill_attention(
        self,
        layer_idx: int,
        query: torch.Tensor,  # [num_prefill_tokens, num_heads, head_dim]
        key: torch.Tensor,    # [num_prefill_tokens, num_kv_heads, head_dim]
        value: torch.Tensor,  # [num_prefill_tokens, num_kv_heads, head_dim]
        attn_metadata: "AttentionMetadata",
        pool: Any,
    ) -> torch.Tensor:
        """Causal attention of prefill chunks over the cached prefix + chunk."""

    @staticmethod
    def create(config: "ModelConfig", backend: str = "hip") -> "AttentionBackend":
        """Backend factory (reference backend.py:95-118).

        ``"reference"`` / ``"ref"``: the reference's PyTorch backend, from the
        module ``paged_attention_ref`` beside this one (reference :106-108;
        ``Config.attention_backend`` defaults to it, reference config.py:76).
        ``"hip"`` / ``"triton"``: the HIP backend. Anything else:
        ``ValueError`` (reference :117-118).
        """
        if backend in REFERENCE_BACKEND_NAMES:
            from .paged_attention_ref import AttentionBackendRef  # the reference tree's module

            return AttentionBackendRef(config)
        if backend in GPU_BACKEND_NAMES:
            from .paged_attention_gpu import AttentionBackendGPU

            return AttentionBackendGPU(config)
        raise ValueError(f"Unknown AttentionBackend: {backend!r}")
