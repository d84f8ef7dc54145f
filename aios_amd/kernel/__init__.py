from .attnres import attnres_mix, attnres_mix_step
from .store import store_cache

__all__ = ["attnres_mix", "attnres_mix_step", "store_cache"]
