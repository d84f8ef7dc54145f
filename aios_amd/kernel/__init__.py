from .store import store_cache

__all__ = ["store_cache"]
