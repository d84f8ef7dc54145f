"""aios_amd — MI355X-native (gfx950 HIP) attention backend for AIOS-IME.

Drop-in for the reference's attention backend and paged KV-store op:
``aios_amd.attention.Mi355xAttentionBackend`` (prepare_metadata / forward),
``aios_amd.kvcache.MHAKVCache`` (k_cache / v_cache / store_kv) and
``aios_amd.kernel.store_cache``; the kernels sit behind the C ABI in
``include/aios_attn.h`` (libaios_attn.so, loaded by ``aios_amd._lib``).
"""
from __future__ import annotations

__version__ = "0.1.0"
