from .base import BaseAttentionBackend, BaseAttentionMetadata, HybridAttentionBackend
from .backend import (
    SUPPORTED_HEAD_DIMS,
    Mi355xAttentionBackend,
    Mi355xAttentionMetadata,
)

__all__ = [
    "BaseAttentionBackend",
    "BaseAttentionMetadata",
    "HybridAttentionBackend",
    "Mi355xAttentionBackend",
    "Mi355xAttentionMetadata",
    "SUPPORTED_HEAD_DIMS",
]
