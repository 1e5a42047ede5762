from .base import AttentionGroup, AttentionMetadata, ModelConfig, ModelInput

__all__ = ["AttentionGroup", "AttentionMetadata", "ModelConfig", "ModelInput"]
