"""MI355X paged attention backend (drop-in for FlashInferAttentionBackend).

Public surface follows python/aios/attention/flashinfer.py:94-394:

* ``prepare_metadata(batch)`` builds cu_seqlens (pinned host int32), the flat
  page-index list ``indices`` (device int32, identical to the reference's
  ``torch.cat([page_table[row, :device_len] ...])``) and sets
  ``batch.attn_metadata``; here it also builds the per-batch plan on the host
  (the reference plans lazily on the first layer, flashinfer.py:252-289; both
  happen once per batch and are reused by every layer).
* ``forward(q, k, v, kv_cache, layer_id, batch)`` appends the new K/V rows
  (kernel (a)) and then runs prefill (kernel (b)) or decode (kernels (c),
  (d) and the combine) through the C ABI, returning ``[tokens, Hq*D]``; a
  decode batch marked ``fused_append`` appends inside the decode launch
  (aios_attn_append_decode).
* ``metadata.get_last_indices(bs)`` = ``cu_seqlens_q[1:bs+1] - 1``.

There is one code path for every supported head dim (64, 96, 128), so the
reference's torch-SDPA fallback for head_dim 96 (flashinfer.py:19-24,
328-372) has no counterpart here.

Two caller guarantees change what a decode does, and both are opt-in on the
batch: ``Batch.shared_prefix_len`` lets the prefix pages be read once per
kv-head (the cascade), and ``Batch.fused_append`` lets the K/V append run
inside the decode launch.  ``validate=True`` (or ``AIOS_VALIDATE=1``) checks
both on the first layer of every eagerly run decode batch
(:func:`check_decode_preconditions`, one host synchronisation) and raises
``ValueError`` when the batch breaks them; captured graphs skip the check.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import TYPE_CHECKING

import torch

from aios_amd import _lib, paged
from aios_amd.core import get_global_ctx

from .base import BaseAttentionBackend, BaseAttentionMetadata

if TYPE_CHECKING:
    from aios_amd.core import Batch
    from aios_amd.kvcache import MHAKVCache

SUPPORTED_HEAD_DIMS = frozenset({64, 96, 128})
SUPPORTED_GROUPS = frozenset({1, 2, 3, 4, 6, 8})


@dataclass
class Mi355xAttentionMetadata(BaseAttentionMetadata):
    cu_seqlens_q_cpu: torch.Tensor
    cu_seqlens_k_cpu: torch.Tensor
    cu_seqlens_q_gpu: torch.Tensor
    cu_seqlens_k_gpu: torch.Tensor
    indices: torch.Tensor
    last_page_len_cpu: torch.Tensor
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    pos_encoding_mode: str
    seq_lens_cpu: torch.Tensor
    dtype: torch.dtype
    plan: _lib.AttnPlan
    shared_prefix_len: int
    host_staging: torch.Tensor
    initialized: bool = True

    def get_last_indices(self, bs: int) -> torch.Tensor:
        return self.cu_seqlens_q_gpu[1 : 1 + bs].to(torch.long) - 1


@dataclass
class Mi355xStaticDecodeMetadata(Mi355xAttentionMetadata):
    """Decode metadata on fixed device buffers, for steps replayed from a HIP graph.

    The plan is built once for ``max_kv_len`` positions per row; the kernels
    read each row's actual length from ``cu_seqlens_k_gpu``, so one plan (and
    one captured graph) serves every step whose rows are at most that long.
    ``refresh(kv_len)`` rewrites cu_seqlens_k and the flat page indices on the
    device from a device scalar, with no host synchronisation (all rows of the
    batch have the same length, as in an uncompacted CandidateGroup).
    """

    row_ids_gpu: torch.Tensor | None = None
    page_table: torch.Tensor | None = None
    max_kv_len: int = 0
    _ramp: torch.Tensor | None = None

    def refresh(self, kv_len: torch.Tensor) -> None:
        bs = self.row_ids_gpu.numel()
        torch.mul(self._ramp, kv_len, out=self.cu_seqlens_k_gpu)
        _lib.check(
            _lib.lib().aios_build_indices(
                self.page_table.data_ptr(), self.page_table.stride(0), self.row_ids_gpu.data_ptr(),
                self.cu_seqlens_k_gpu.data_ptr(), bs, bs * self.max_kv_len,
                self.indices.data_ptr(), torch.cuda.current_stream(self.indices.device).cuda_stream),
            "aios_build_indices",
        )


@dataclass
class Mi355xStaticPrefillMetadata(Mi355xAttentionMetadata):
    """Prefill metadata of one request (page-table row ``row_id``) on fixed
    device buffers, for a prefill or LCP extension replayed from a HIP graph.

    ``q_len`` new tokens; the plan is built for ``max_kv_len`` positions and
    the kernel reads the request's actual KV length (cached + new) from
    ``cu_seqlens_k_gpu``; ``refresh(kv_len)`` rewrites it and the flat page
    indices on the device from a device scalar, with no host synchronisation.
    """

    row_ids_gpu: torch.Tensor | None = None
    page_table: torch.Tensor | None = None
    max_kv_len: int = 0
    _ramp: torch.Tensor | None = None

    def refresh(self, kv_len: torch.Tensor) -> None:
        torch.mul(self._ramp, kv_len, out=self.cu_seqlens_k_gpu)
        _lib.check(
            _lib.lib().aios_build_indices(
                self.page_table.data_ptr(), self.page_table.stride(0), self.row_ids_gpu.data_ptr(),
                self.cu_seqlens_k_gpu.data_ptr(), 1, self.max_kv_len, self.indices.data_ptr(),
                torch.cuda.current_stream(self.indices.device).cuda_stream),
            "aios_build_indices",
        )


def check_decode_preconditions(indices: torch.Tensor, cu_seqlens_k: torch.Tensor,
                               out_loc: torch.Tensor | None, shared_prefix_len: int) -> None:
    """Raise ``ValueError`` unless the decode batch keeps the caller
    guarantees the backend relies on: every row's first
    ``shared_prefix_len`` page ids equal row 0's, and (``out_loc`` given, the
    fused append) ``out_loc[b]`` is row b's last page id,
    ``indices[cu_seqlens_k[b + 1] - 1]``.  Works on CPU or device tensors;
    one host synchronisation for device tensors."""
    cu = cu_seqlens_k.to(torch.long)
    bs = cu.numel() - 1
    if bs <= 0:
        return
    lens = cu[1:] - cu[:-1]
    if shared_prefix_len > 0:
        if bool((lens < shared_prefix_len).any()):
            raise ValueError(f"shared_prefix_len {shared_prefix_len} exceeds a row's KV length")
        ar = torch.arange(shared_prefix_len, device=indices.device)
        rows = indices[cu[:-1, None] + ar[None, :]]
        if not bool((rows == rows[:1]).all()):
            raise ValueError(f"rows do not share their first {shared_prefix_len} pages "
                             "(Batch.shared_prefix_len)")
    if out_loc is not None:
        if bool((lens < 1).any()):
            raise ValueError("a decode row has no KV position for its new token")
        last = indices[cu[1:] - 1]
        if not bool((out_loc.to(last.dtype) == last).all()):
            raise ValueError("out_loc[b] must be row b's last page id (Batch.fused_append)")


class Mi355xAttentionBackend(BaseAttentionBackend):
    """Paged prefill/decode on hand-written gfx950 HIP kernels."""

    def __init__(
        self,
        config,
        workspace_size: int = 128 * 1024 * 1024,
        prefix_chunk_len: int = 0,
        suffix_split_len: int = 0,
        validate: bool | None = None,
    ) -> None:
        self.num_heads = config.num_qo_heads
        self.num_kv_heads = config.num_kv_heads
        self.head_dim = config.head_dim
        self.sm_scale = config.head_dim ** -0.5
        if self.head_dim not in SUPPORTED_HEAD_DIMS:
            raise ValueError(
                f"head_dim {self.head_dim} is not supported (built: {sorted(SUPPORTED_HEAD_DIMS)})"
            )
        if self.num_heads % self.num_kv_heads:
            raise ValueError("query head count must be divisible by KV head count")
        if self.num_heads // self.num_kv_heads not in SUPPORTED_GROUPS:
            raise ValueError("GQA group size is not supported")
        self.prefill_kernel_backend = "hip-mfma"
        self.decode_kernel_backend = "hip-cascade"
        self.backend_name = "mi355x-paged-prefill-hip-mfma-decode-hip-cascade"
        self.workspace_size = workspace_size
        self.prefix_chunk_len = prefix_chunk_len
        self.suffix_split_len = suffix_split_len
        self.validate = (os.environ.get("AIOS_VALIDATE", "0") not in ("", "0")
                         if validate is None else bool(validate))
        self._workspace: torch.Tensor | None = None
        self._cached_ones_cpu: torch.Tensor = torch.tensor([], dtype=torch.int32)

    # -- helpers ---------------------------------------------------------------
    def _get_workspace(self, device: torch.device) -> torch.Tensor:
        if self._workspace is None or self._workspace.numel() != self.workspace_size:
            self._workspace = torch.empty(self.workspace_size, dtype=torch.uint8, device=device)
        return self._workspace

    def _get_ones_cpu(self, bs: int) -> torch.Tensor:
        if bs <= len(self._cached_ones_cpu):
            return self._cached_ones_cpu[:bs]
        next_len = 1 << max(bs - 1, 0).bit_length()
        self._cached_ones_cpu = torch.ones(next_len, dtype=torch.int32, pin_memory=True)
        return self._cached_ones_cpu[:bs]

    # -- interface -------------------------------------------------------------
    def prepare_metadata(self, batch: Batch) -> Mi355xAttentionMetadata:
        ctx = get_global_ctx()
        page_table = ctx.page_table
        assert page_table.is_cuda, "the MI355X backend requires a GPU page table"
        assert page_table.dtype == torch.int32, "page_table must be int32"
        reqs = batch.reqs
        bs = len(reqs)
        seqlens_q = [req.extend_len for req in reqs]
        seqlens_k = [req.device_len for req in reqs]
        row_ids = [int(req.table_idx) for req in reqs]
        if any(r < 0 or r >= page_table.shape[0] for r in row_ids):
            raise ValueError("request table_idx outside the page table")
        if seqlens_k and max(seqlens_k) > page_table.shape[1]:
            raise ValueError("device_len exceeds the page-table row length")
        device = page_table.device

        # One pinned staging buffer -> one host-to-device copy per batch:
        # [cu_q (bs+1) | cu_k (bs+1) | row_ids (bs)].
        host = torch.empty(3 * bs + 2, dtype=torch.int32, pin_memory=True)
        cu_q = host[: bs + 1]
        cu_k = host[bs + 1 : 2 * bs + 2]
        rows = host[2 * bs + 2 :]
        cu_q[0] = 0
        cu_k[0] = 0
        if bs:
            cu_q[1:] = torch.tensor(seqlens_q, dtype=torch.int32).cumsum_(0)
            cu_k[1:] = torch.tensor(seqlens_k, dtype=torch.int32).cumsum_(0)
            rows.copy_(torch.tensor(row_ids, dtype=torch.int32))
        dev = host.to(device, non_blocking=True)
        cu_q_gpu = dev[: bs + 1]
        cu_k_gpu = dev[bs + 1 : 2 * bs + 2]
        rows_gpu = dev[2 * bs + 2 :]
        total_kv = int(cu_k[bs]) if bs else 0

        shared = int(getattr(batch, "shared_prefix_len", 0)) if batch.is_decode else 0
        plan = _lib.AttnPlan()
        _lib.check(
            _lib.lib().aios_attn_plan(
                _lib.PHASE_DECODE if batch.is_decode else _lib.PHASE_PREFILL,
                cu_q.data_ptr(),
                cu_k.data_ptr(),
                bs,
                self.num_heads,
                self.num_kv_heads,
                self.head_dim,
                1,
                shared,
                self.workspace_size,
                self.prefix_chunk_len,
                self.suffix_split_len,
                plan,
            ),
            "aios_attn_plan",
        )

        indices = torch.empty(total_kv, dtype=torch.int32, device=device)
        if total_kv:
            stream = torch.cuda.current_stream(device).cuda_stream
            _lib.check(
                _lib.lib().aios_build_indices(
                    page_table.data_ptr(),
                    page_table.stride(0),
                    rows_gpu.data_ptr(),
                    cu_k_gpu.data_ptr(),
                    bs,
                    total_kv,
                    indices.data_ptr(),
                    stream,
                ),
                "aios_build_indices",
            )

        metadata = Mi355xAttentionMetadata(
            cu_seqlens_q_cpu=cu_q,
            cu_seqlens_k_cpu=cu_k,
            cu_seqlens_q_gpu=cu_q_gpu,
            cu_seqlens_k_gpu=cu_k_gpu,
            indices=indices,
            last_page_len_cpu=self._get_ones_cpu(bs),
            num_qo_heads=self.num_heads,
            num_kv_heads=self.num_kv_heads,
            head_dim=self.head_dim,
            page_size=1,
            pos_encoding_mode="NONE",
            seq_lens_cpu=torch.tensor(seqlens_k, dtype=torch.int32),
            dtype=ctx.kv_cache.dtype,
            plan=plan,
            shared_prefix_len=shared,
            host_staging=host,
        )
        if plan.ws_bytes:
            self._get_workspace(device)
        batch.attn_metadata = metadata
        return metadata

    def prepare_static_decode(self, row_ids: torch.Tensor, max_kv_len: int, shared_prefix_len: int,
                              page_table: torch.Tensor) -> Mi355xStaticDecodeMetadata:
        """Fixed-buffer decode metadata for graph-replayed steps (see
        :class:`Mi355xStaticDecodeMetadata`); ``shared_prefix_len`` may be any
        length up to the prefix every row really shares."""
        bs = row_ids.numel()
        device = page_table.device
        if page_table.dtype != torch.int32 or max_kv_len > page_table.shape[1]:
            raise ValueError("max_kv_len exceeds the page-table row length")
        cu_q = torch.arange(bs + 1, dtype=torch.int32)
        cu_k = cu_q * max_kv_len
        plan = _lib.AttnPlan()
        _lib.check(
            _lib.lib().aios_attn_plan(_lib.PHASE_DECODE, cu_q.data_ptr(), cu_k.data_ptr(), bs,
                                      self.num_heads, self.num_kv_heads, self.head_dim, 1,
                                      shared_prefix_len, self.workspace_size,
                                      self.prefix_chunk_len, self.suffix_split_len, plan),
            "aios_attn_plan",
        )
        if plan.ws_bytes:
            self._get_workspace(device)
        ramp = torch.arange(bs + 1, dtype=torch.int32, device=device)
        return Mi355xStaticDecodeMetadata(
            cu_seqlens_q_cpu=cu_q,
            cu_seqlens_k_cpu=cu_k,
            cu_seqlens_q_gpu=ramp.clone(),
            cu_seqlens_k_gpu=torch.zeros(bs + 1, dtype=torch.int32, device=device),
            indices=torch.zeros(bs * max_kv_len, dtype=torch.int32, device=device),
            last_page_len_cpu=self._get_ones_cpu(bs),
            num_qo_heads=self.num_heads,
            num_kv_heads=self.num_kv_heads,
            head_dim=self.head_dim,
            page_size=1,
            pos_encoding_mode="NONE",
            seq_lens_cpu=torch.full((bs,), max_kv_len, dtype=torch.int32),
            dtype=torch.bfloat16,
            plan=plan,
            shared_prefix_len=shared_prefix_len,
            host_staging=cu_q,
            row_ids_gpu=row_ids.to(device=device, dtype=torch.int32).contiguous(),
            page_table=page_table,
            max_kv_len=max_kv_len,
            _ramp=ramp,
        )

    def prepare_static_prefill(self, q_len: int, max_kv_len: int, page_table: torch.Tensor,
                               row_id: int = 0) -> Mi355xStaticPrefillMetadata:
        """Fixed-buffer prefill metadata for graph-replayed prefills of
        ``q_len`` tokens against at most ``max_kv_len`` positions (see
        :class:`Mi355xStaticPrefillMetadata`)."""
        device = page_table.device
        if page_table.dtype != torch.int32 or max_kv_len > page_table.shape[1]:
            raise ValueError("max_kv_len exceeds the page-table row length")
        if not 1 <= q_len <= max_kv_len:
            raise ValueError("q_len must be within 1..max_kv_len")
        cu_q = torch.tensor([0, q_len], dtype=torch.int32)
        cu_k = torch.tensor([0, max_kv_len], dtype=torch.int32)
        plan = _lib.AttnPlan()
        _lib.check(
            _lib.lib().aios_attn_plan(_lib.PHASE_PREFILL, cu_q.data_ptr(), cu_k.data_ptr(), 1,
                                      self.num_heads, self.num_kv_heads, self.head_dim, 1, 0,
                                      self.workspace_size, self.prefix_chunk_len,
                                      self.suffix_split_len, plan),
            "aios_attn_plan",
        )
        ramp = torch.arange(2, dtype=torch.int32, device=device)
        return Mi355xStaticPrefillMetadata(
            cu_seqlens_q_cpu=cu_q,
            cu_seqlens_k_cpu=cu_k,
            cu_seqlens_q_gpu=cu_q.to(device),
            cu_seqlens_k_gpu=torch.zeros(2, dtype=torch.int32, device=device),
            indices=torch.zeros(max_kv_len, dtype=torch.int32, device=device),
            last_page_len_cpu=self._get_ones_cpu(1),
            num_qo_heads=self.num_heads,
            num_kv_heads=self.num_kv_heads,
            head_dim=self.head_dim,
            page_size=1,
            pos_encoding_mode="NONE",
            seq_lens_cpu=torch.tensor([max_kv_len], dtype=torch.int32),
            dtype=torch.bfloat16,
            plan=plan,
            shared_prefix_len=0,
            host_staging=cu_q,
            row_ids_gpu=torch.tensor([row_id], dtype=torch.int32, device=device),
            page_table=page_table,
            max_kv_len=max_kv_len,
            _ramp=ramp,
        )

    def forward(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        paged_kv_cache: MHAKVCache,
        layer_id: int,
        batch: Batch,
    ) -> torch.Tensor:
        if batch.is_prefill:
            return self._prefill(q, k, v, paged_kv_cache, layer_id, batch)
        return self._decode(q, k, v, paged_kv_cache, layer_id, batch)

    # Head sizes whose decoder layers take the q/k norm + rotation inside the
    # decode launch.  Measured on MI355X (graph-replayed CandidateGroup step,
    # the two forms back to back): 64 (MiniMind-IME 0.1B) 441 -> 430 us;
    # 96 (MiniMind 0.1B) 403.3 -> 400.8 us.  With the suffix items' rotation
    # in the pair layout (half the registers of the 16-row tile layout),
    # 128 (Qwen3-0.6B) 996 -> 981.5 us; in the tile layout it had pushed the
    # decode kernel past the register file (1304 -> 1339 us).
    ROPE_IN_DECODE_HEAD_DIMS = (64, 96, 128)

    def decode_rope_applies(self, batch: Batch) -> bool:
        """Whether forward_rope takes this batch: an appending decode batch
        (Batch.fused_append) whose new tokens lie after the shared prefix,
        at a head size listed in ROPE_IN_DECODE_HEAD_DIMS."""
        if self.head_dim not in self.ROPE_IN_DECODE_HEAD_DIMS:
            return False
        if not batch.is_decode or not batch.fused_append:
            return False
        md = batch.attn_metadata
        return (isinstance(md, Mi355xAttentionMetadata)
                and md.plan.prefix_len < md.plan.min_kv_len
                and batch.out_loc.dtype == torch.int32)

    def forward_rope(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     q_norm: torch.Tensor, k_norm: torch.Tensor, cos: torch.Tensor,
                     sin: torch.Tensor, positions: torch.Tensor, eps: float,
                     paged_kv_cache: MHAKVCache, layer_id: int, batch: Batch) -> torch.Tensor:
        """The q/k RMSNorm + rotary embedding of Qwen3Attention.forward
        (python/aios/models/qwen3.py:52-67), store_kv and the decode run
        (python/aios/attention/flashinfer.py:374-394) in one launch, for a
        batch decode_rope_applies accepts; q and k are the raw projections,
        cos / sin the rotary tables rounded to bf16."""
        if not (batch.is_decode and batch.fused_append
                and isinstance(batch.attn_metadata, Mi355xAttentionMetadata)
                and batch.attn_metadata.plan.prefix_len < batch.attn_metadata.plan.min_kv_len
                and batch.out_loc.dtype == torch.int32):
            raise ValueError("forward_rope needs an appending decode batch (Batch.fused_append) "
                             "whose new tokens lie after the shared prefix")
        bsz = batch.size
        metadata = batch.attn_metadata
        self._check_q(q)
        if q.size(0) != bsz:
            raise ValueError("decode batch must contain one flat token per request")
        if k.shape != v.shape or k.shape[1:] != (self.num_kv_heads, self.head_dim):
            raise ValueError("K/V input shape does not match the cache layout")
        plan = metadata.plan
        out_loc = batch.out_loc.view(-1)
        if out_loc.numel() != k.shape[0]:
            raise ValueError("KV write indices and K/V tensors must have matching token counts")
        if self.validate and layer_id == 0 and not torch.cuda.is_current_stream_capturing():
            check_decode_preconditions(metadata.indices, metadata.cu_seqlens_k_gpu, out_loc,
                                       metadata.shared_prefix_len)
        ws = self._get_workspace(q.device) if plan.ws_bytes else None
        k_cache, v_cache = self._layer_caches(paged_kv_cache, layer_id)
        out = paged.append_decode_rope(plan, q, k, v, out_loc.contiguous(),
                                       k_cache.view(-1, self.num_kv_heads, self.head_dim),
                                       v_cache.view(-1, self.num_kv_heads, self.head_dim),
                                       metadata.indices, metadata.cu_seqlens_k_gpu, q_norm, k_norm,
                                       cos, sin, positions, eps, workspace=ws,
                                       sm_scale=self.sm_scale)
        return out.reshape(bsz, -1)

    def _check_q(self, q: torch.Tensor) -> None:
        if q.ndim != 3 or q.shape[1] != self.num_heads or q.shape[2] != self.head_dim:
            raise ValueError("q must have shape (tokens, num_qo_heads, head_dim)")
        if q.dtype != torch.bfloat16:
            raise ValueError("the MI355X attention kernels compute in bfloat16")
        if q.stride(2) != 1 or q.stride(1) != self.head_dim:
            raise ValueError("q must have contiguous (heads, head_dim) rows")

    def _layer_caches(self, paged_kv_cache: MHAKVCache, layer_id: int):
        k_cache = paged_kv_cache.k_cache(layer_id)
        v_cache = paged_kv_cache.v_cache(layer_id)
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("per-layer KV caches must be contiguous")
        if k_cache.dtype != torch.bfloat16:
            raise ValueError("the MI355X attention kernels read a bfloat16 KV cache")
        return k_cache, v_cache

    def _prefill(self, q, k, v, paged_kv_cache, layer_id, batch) -> torch.Tensor:
        assert batch.is_prefill, "prefill backend expects a prefill batch"
        metadata = batch.attn_metadata
        assert isinstance(metadata, Mi355xAttentionMetadata)
        self._check_q(q)
        if q.shape[0] != metadata.plan.total_q:
            raise RuntimeError("prefill request lengths do not match flat Q tokens")
        paged_kv_cache.store_kv(k, v, batch.out_loc.view(-1), layer_id)
        k_cache, v_cache = self._layer_caches(paged_kv_cache, layer_id)
        out = paged.prefill(metadata.plan, q, k_cache.view(-1, self.num_kv_heads, self.head_dim),
                            v_cache.view(-1, self.num_kv_heads, self.head_dim), metadata.indices,
                            metadata.cu_seqlens_q_gpu, metadata.cu_seqlens_k_gpu,
                            sm_scale=self.sm_scale)
        return out.reshape(q.size(0), -1)

    def _decode(self, q, k, v, paged_kv_cache, layer_id, batch) -> torch.Tensor:
        assert batch.is_decode, "decode backend expects a decode batch"
        bsz = batch.size
        assert q.size(0) == bsz, "decode batch must contain one flat token per request"
        metadata = batch.attn_metadata
        assert isinstance(metadata, Mi355xAttentionMetadata)
        self._check_q(q)
        plan = metadata.plan
        out_loc = batch.out_loc.view(-1)
        ws = self._get_workspace(q.device) if plan.ws_bytes else None
        fused = (batch.fused_append and plan.prefix_len < plan.min_kv_len
                 and out_loc.dtype == torch.int32)
        if self.validate and layer_id == 0 and not torch.cuda.is_current_stream_capturing():
            check_decode_preconditions(metadata.indices, metadata.cu_seqlens_k_gpu,
                                       out_loc if fused else None, metadata.shared_prefix_len)
        if fused:
            # The store_kv of flashinfer.py:389 runs inside the decode launch:
            # the caller guarantees (Batch.fused_append) that each row's new
            # token goes to its last KV position's page.
            if k.shape != v.shape or k.shape[1:] != (self.num_kv_heads, self.head_dim):
                raise ValueError("K/V input shape does not match the cache layout")
            if out_loc.numel() != k.shape[0]:
                raise ValueError("KV write indices and K/V tensors must have matching token counts")
            k_cache, v_cache = self._layer_caches(paged_kv_cache, layer_id)
            out = paged.append_decode(plan, q, k, v, out_loc.contiguous(),
                                      k_cache.view(-1, self.num_kv_heads, self.head_dim),
                                      v_cache.view(-1, self.num_kv_heads, self.head_dim),
                                      metadata.indices, metadata.cu_seqlens_k_gpu, workspace=ws,
                                      sm_scale=self.sm_scale)
            return out.reshape(bsz, -1)
        paged_kv_cache.store_kv(k, v, out_loc, layer_id)
        k_cache, v_cache = self._layer_caches(paged_kv_cache, layer_id)
        out = paged.decode(plan, q, k_cache.view(-1, self.num_kv_heads, self.head_dim),
                           v_cache.view(-1, self.num_kv_heads, self.head_dim), metadata.indices,
                           metadata.cu_seqlens_k_gpu, workspace=ws, sm_scale=self.sm_scale)
        return out.reshape(bsz, -1)
