from .backend import AttentionBackend
from .paged_attention_gpu import AttentionBackendGPU

__all__ = ["AttentionBackend", "AttentionBackendGPU"]
