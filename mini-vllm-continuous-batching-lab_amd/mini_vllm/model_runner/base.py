"""Per-step metadata types consumed by the attention backend.

Field names, types and meaning follow mini_vllm/model_runner/base.py:14-106
of the reference so that metadata built by its ``ModelInputBuilder``
(mini_vllm/engine/input_builder.py:48-196) and rebased by
``QwenModelRunner._build_decode_meta`` (qwen_runner.py:213-251) can be handed
to this package's backend unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import torch


def _empty_long() -> torch.Tensor:
    return torch.tensor([], dtype=torch.long)


@dataclass
class ModelConfig:
    """Model dimensions (reference: model_runner/base.py:14-40).

    Only ``num_heads``, ``num_kv_heads`` and ``head_dim`` matter to the
    attention backend; the remaining fields keep the reference's
    constructor signature.
    """

    model_type: str = ""
    num_layers: int = 0
    hidden_size: int = 0
    num_heads: int = 0
    num_kv_heads: int = 0
    head_dim: int = 0
    vocab_size: int = 0
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    max_position_embeddings: int = 32768
    hidden_act: str = "silu"
    intermediate_size: int = 0
    tie_word_embeddings: bool = True
    rope_scaling: Optional[dict] = None
    dtype: torch.dtype = torch.float16
    activation_dtype: torch.dtype = torch.float16


@dataclass
class AttentionGroup:
    """Sequences of one attention type (reference: base.py:47-59).

    ``attention_type`` is ``"decode_gpu"`` for decode rows and
    ``"prefill_gpu"`` / ``"prefill_ref"`` for prefill rows. The three length
    tensors are int64, one entry per sequence of the group, with
    ``kv_len_after == cached_len_before + query_len``.
    """

    seq_indices: List[int]
    attention_type: str
    cached_len_before: torch.Tensor
    query_len: torch.Tensor
    kv_len_after: torch.Tensor


@dataclass
class AttentionMetadata:
    """Per-step attention metadata (reference: base.py:62-84).

    Block tables are ``[num_seqs, max_blocks]`` int64, padded with -1 at the
    tail of each row; slot mappings are int64 flat slot indices.
    """

    groups: List[AttentionGroup] = field(default_factory=list)
    prefill_slot_mapping: torch.Tensor = field(default_factory=_empty_long)
    prefill_block_tables: torch.Tensor = field(default_factory=_empty_long)
    prefill_positions: torch.Tensor = field(default_factory=_empty_long)
    decode_block_tables: torch.Tensor = field(default_factory=_empty_long)
    decode_slot_mapping: torch.Tensor = field(default_factory=_empty_long)
    decode_positions: torch.Tensor = field(default_factory=_empty_long)
    block_size: int = 0
    num_kv_heads: int = 0
    head_dim: int = 0

    def decode_group(self) -> Optional[AttentionGroup]:
        """First group with ``attention_type == "decode_gpu"`` (or None)."""
        for g in self.groups:
            if g.attention_type == "decode_gpu":
                return g
        return None


@dataclass
class ModelInput:
    """Inputs of one model step (reference: base.py:87-105)."""

    input_ids: torch.Tensor = field(default_factory=_empty_long)
    positions: torch.Tensor = field(default_factory=_empty_long)
    slot_mapping: torch.Tensor = field(default_factory=_empty_long)
    attn_metadata: AttentionMetadata = field(default_factory=AttentionMetadata)
    sample_token_indices: torch.Tensor = field(default_factory=_empty_long)
    sequence_info: Tuple = field(default_factory=tuple)
