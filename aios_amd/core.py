"""Runtime data model read by the attention backend.

Mirrors python/aios/core.py:14-124 (SamplingParams, Req, Batch, Context and
the process-global context) so that callers written against the reference
drive this backend unchanged.  Two fields are added, both set only by callers
that guarantee what they state (the CandidateGroup engine here):

* ``Batch.shared_prefix_len`` (default 0): the number of leading KV positions
  whose pages every row of a decode batch shares (the reference creates that
  sharing at python/aios/ime.py:1155 but never tells the backend);
* ``Batch.fused_append`` (default False): every decode row's ``out_loc`` entry
  is that row's last page, ``page_table[row, device_len - 1]`` (as in
  ime.py:1228-1229), so the backend may append the new K/V inside the decode
  launch instead of running ``store_kv`` first (flashinfer.py:389).
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import TYPE_CHECKING, List, Literal, Optional

import torch

if TYPE_CHECKING:
    from aios_amd.attention import BaseAttentionBackend, BaseAttentionMetadata
    from aios_amd.kvcache import MHAKVCache


@dataclass
class SamplingParams:
    """python/aios/core.py:14-24."""

    temperature: float = 0.0
    top_k: int = -1
    top_p: float = 1.0
    ignore_eos: bool = False
    max_tokens: int = 1024

    @property
    def is_greedy(self) -> bool:
        return (self.temperature <= 0.0 or self.top_k == 1) and self.top_p == 1.0


@dataclass(eq=False)
class Req:
    """Per-request runtime state (python/aios/core.py:27-59)."""

    input_ids: torch.Tensor
    cached_len: int
    output_len: int
    uid: int
    sampling_params: SamplingParams
    table_idx: int | None = None
    generated: List[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        self.device_len = len(self.input_ids)
        self.max_device_len = len(self.input_ids) + self.output_len
        assert 0 <= self.cached_len <= self.device_len <= self.max_device_len

    @property
    def remain_len(self) -> int:
        return self.max_device_len - self.device_len

    @property
    def extend_len(self) -> int:
        return self.device_len - self.cached_len

    def complete_one(self) -> None:
        self.cached_len = self.device_len
        self.device_len += 1

    @property
    def can_decode(self) -> bool:
        return self.remain_len > 0


@dataclass
class Batch:
    """One forward pass worth of requests (python/aios/core.py:62-88)."""

    reqs: List[Req]
    phase: Literal["prefill", "decode"]
    input_ids: torch.Tensor = field(init=False)
    positions: torch.Tensor = field(init=False)
    out_loc: torch.Tensor = field(init=False)
    attn_metadata: "BaseAttentionMetadata" = field(init=False)
    return_all_logits: bool = False
    shared_prefix_len: int = 0
    fused_append: bool = False
    # The rows' embeddings when the caller has gathered them already (a
    # captured CandidateGroup step does it with its step preparation).
    input_embeds: Optional[torch.Tensor] = None

    @property
    def is_prefill(self) -> bool:
        return self.phase == "prefill"

    @property
    def is_decode(self) -> bool:
        return self.phase == "decode"

    @property
    def size(self) -> int:
        return len(self.reqs)


@dataclass
class Context:
    """python/aios/core.py:91-111."""

    page_size: int
    page_table: torch.Tensor = field(init=False)
    attn_backend: "BaseAttentionBackend" = field(init=False)
    kv_cache: "MHAKVCache" = field(init=False)
    _batch: Batch | None = field(default=None, init=False)

    @property
    def batch(self) -> Batch:
        assert self._batch is not None, "No active batch in context"
        return self._batch

    @contextmanager
    def forward_batch(self, batch: Batch):
        assert self._batch is None, "Nested forward_batch is not allowed"
        try:
            self._batch = batch
            yield
        finally:
            self._batch = None


_GLOBAL_CTX: Context | None = None


def set_global_ctx(ctx: Context) -> None:
    global _GLOBAL_CTX
    assert _GLOBAL_CTX is None, "Global context is already set"
    _GLOBAL_CTX = ctx


def get_global_ctx() -> Context:
    assert _GLOBAL_CTX is not None, "Global context is not set"
    return _GLOBAL_CTX


def reset_global_ctx() -> None:
    """Drop the process-global context (tests and benches build several)."""
    global _GLOBAL_CTX
    _GLOBAL_CTX = None
