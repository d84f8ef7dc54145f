from .base import BaseAttentionBackend, BaseAttentionMetadata, HybridAttentionBackend
from .backend import (
    SUPPORTED_HEAD_DIMS,
    Mi355xAttentionBackend,
    Mi355xAttentionMetadata,
    Mi355xStaticDecodeMetadata,
    Mi355xStaticPrefillMetadata,
    check_decode_preconditions,
)

__all__ = [
    "BaseAttentionBackend",
    "BaseAttentionMetadata",
    "HybridAttentionBackend",
    "Mi355xAttentionBackend",
    "Mi355xAttentionMetadata",
    "Mi355xStaticDecodeMetadata",
    "Mi355xStaticPrefillMetadata",
    "SUPPORTED_HEAD_DIMS",
    "check_decode_preconditions",
]
