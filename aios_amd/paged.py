"""Functional wrappers over the C ABI (plan / prefill / decode / kv_append).

These take torch tensors, check the layouts the kernels assume, and pass raw
device pointers plus the current HIP stream to libaios_attn.so.  The
reference-shaped backend (``aios_amd.attention``) is built on them.
"""
from __future__ import annotations

import torch

from aios_amd import _lib

DEFAULT_WORKSPACE = 128 * 1024 * 1024


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _host_i32(x) -> torch.Tensor:
    t = torch.as_tensor(x, dtype=torch.int32)
    if t.device.type != "cpu":
        raise ValueError("cu_seqlens for planning must be host tensors")
    return t.contiguous()


def plan(phase: str, cu_q, cu_k, num_qo_heads: int, num_kv_heads: int, head_dim: int, *,
         shared_prefix_len: int = 0, workspace_bytes: int = DEFAULT_WORKSPACE,
         prefix_chunk_len: int = 0, suffix_split_len: int = 0) -> _lib.AttnPlan:
    """Host-only schedule for one batch (aios_attn_plan)."""
    cu_q = _host_i32(cu_q)
    cu_k = _host_i32(cu_k)
    if cu_q.numel() != cu_k.numel() or cu_q.numel() < 1:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have batch_size + 1 entries")
    p = _lib.AttnPlan()
    code = _lib.PHASE_DECODE if phase == "decode" else _lib.PHASE_PREFILL
    _lib.check(
        _lib.lib().aios_attn_plan(code, cu_q.data_ptr(), cu_k.data_ptr(), cu_q.numel() - 1,
                                  num_qo_heads, num_kv_heads, head_dim, 1, shared_prefix_len,
                                  workspace_bytes, prefix_chunk_len, suffix_split_len, p),
        "aios_attn_plan",
    )
    return p


def _check_q(q: torch.Tensor, p: _lib.AttnPlan) -> None:
    if q.dtype != torch.bfloat16 or not q.is_cuda:
        raise ValueError("q must be a bfloat16 GPU tensor")
    if q.ndim != 3 or q.shape[1] != p.num_qo_heads or q.shape[2] != p.head_dim:
        raise ValueError("q must have shape (tokens, num_qo_heads, head_dim)")
    if q.stride(2) != 1 or q.stride(1) != p.head_dim:
        raise ValueError("q must have contiguous (heads, head_dim) rows")


def _check_cache(c: torch.Tensor, p: _lib.AttnPlan) -> None:
    if c.dtype != torch.bfloat16 or not c.is_cuda or not c.is_contiguous():
        raise ValueError("KV cache must be a contiguous bfloat16 GPU tensor")
    if c.shape[-1] != p.head_dim or c.shape[-2] != p.num_kv_heads:
        raise ValueError("KV cache must end in (num_kv_heads, head_dim)")
    if c.numel() != c.shape[0] * p.num_kv_heads * p.head_dim:
        raise ValueError("KV cache must be (num_pages, [1,] num_kv_heads, head_dim)")


def _check_i32(t: torch.Tensor, name: str, n: int) -> None:
    if t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous() or t.numel() < n:
        raise ValueError(f"{name} must be a contiguous int32 GPU tensor of >= {n} entries")


def decode(p: _lib.AttnPlan, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
           indices: torch.Tensor, cu_k: torch.Tensor, *, out: torch.Tensor | None = None,
           workspace: torch.Tensor | None = None, sm_scale: float | None = None) -> torch.Tensor:
    """Paged decode attention of one layer: returns [B, Hq, D] bf16."""
    if p.phase != _lib.PHASE_DECODE:
        raise ValueError("plan was not built for decode")
    _check_q(q, p)
    if q.shape[0] != p.batch_size:
        raise ValueError("decode batch must contain one flat token per request")
    _check_cache(k_cache, p)
    _check_cache(v_cache, p)
    _check_i32(indices, "indices", p.total_kv)
    _check_i32(cu_k, "cu_k", p.batch_size + 1)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if p.ws_bytes and (workspace is None or workspace.numel() < p.ws_bytes):
        raise RuntimeError(f"decode needs a workspace of {p.ws_bytes} bytes")
    scale = p.head_dim ** -0.5 if sm_scale is None else sm_scale
    _lib.check(
        _lib.lib().aios_attn_decode(
            p, q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.shape[0], indices.data_ptr(), cu_k.data_ptr(), out.data_ptr(),
            workspace.data_ptr() if workspace is not None else None,
            workspace.numel() if workspace is not None else 0, scale, _stream(q.device)),
        "aios_attn_decode",
    )
    return out


def decode_noalloc(p: _lib.AttnPlan, q: torch.Tensor, k_cache: torch.Tensor,
                   v_cache: torch.Tensor, indices: torch.Tensor, cu_k: torch.Tensor, *,
                   out: torch.Tensor, sm_scale: float | None = None) -> torch.Tensor:
    """``decode`` with the partial states in the library's built-in device
    array (aios_attn_decode_noalloc): no workspace and no allocation, so the
    caller passes ``out``.  Calls overlapping on one GPU race."""
    if p.phase != _lib.PHASE_DECODE:
        raise ValueError("plan was not built for decode")
    _check_q(q, p)
    if q.shape[0] != p.batch_size:
        raise ValueError("decode batch must contain one flat token per request")
    _check_cache(k_cache, p)
    _check_cache(v_cache, p)
    _check_i32(indices, "indices", p.total_kv)
    _check_i32(cu_k, "cu_k", p.batch_size + 1)
    if out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 tensor shaped like q")
    scale = p.head_dim ** -0.5 if sm_scale is None else sm_scale
    _lib.check(
        _lib.lib().aios_attn_decode_noalloc(
            p, q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.shape[0], indices.data_ptr(), cu_k.data_ptr(), out.data_ptr(), scale,
            _stream(q.device)),
        "aios_attn_decode_noalloc",
    )
    return out


def _check_new_kv(k: torch.Tensor, v: torch.Tensor, out_loc: torch.Tensor, p: _lib.AttnPlan) -> None:
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16 or not k.is_cuda or not v.is_cuda:
        raise ValueError("new K/V rows must be bfloat16 GPU tensors")
    shape = (p.batch_size, p.num_kv_heads, p.head_dim)
    if tuple(k.shape) != shape or tuple(v.shape) != shape:
        raise ValueError("K/V input shape does not match the cache layout")
    for t in (k, v):
        if t.stride(2) != 1 or t.stride(1) != p.head_dim:
            raise ValueError("new K/V rows must have contiguous (heads, head_dim) rows")
    _check_i32(out_loc, "out_loc", p.batch_size)


def append_decode(p: _lib.AttnPlan, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  out_loc: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  indices: torch.Tensor, cu_k: torch.Tensor, *, out: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None,
                  sm_scale: float | None = None) -> torch.Tensor:
    """Append each row's new K/V (k[b], v[b] -> page out_loc[b]) and decode, in
    one launch (aios_attn_append_decode); row b's last KV position must be
    out_loc[b].  Returns [B, Hq, D] bf16."""
    if p.phase != _lib.PHASE_DECODE:
        raise ValueError("plan was not built for decode")
    _check_q(q, p)
    if q.shape[0] != p.batch_size:
        raise ValueError("decode batch must contain one flat token per request")
    _check_cache(k_cache, p)
    _check_cache(v_cache, p)
    _check_i32(indices, "indices", p.total_kv)
    _check_i32(cu_k, "cu_k", p.batch_size + 1)
    _check_new_kv(k, v, out_loc, p)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if p.ws_bytes and (workspace is None or workspace.numel() < p.ws_bytes):
        raise RuntimeError(f"decode needs a workspace of {p.ws_bytes} bytes")
    scale = p.head_dim ** -0.5 if sm_scale is None else sm_scale
    _lib.check(
        _lib.lib().aios_attn_append_decode(
            p, q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
            out_loc.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0],
            indices.data_ptr(), cu_k.data_ptr(), out.data_ptr(),
            workspace.data_ptr() if workspace is not None else None,
            workspace.numel() if workspace is not None else 0, scale, _stream(q.device)),
        "aios_attn_append_decode",
    )
    return out


def append_decode_rope(p: _lib.AttnPlan, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       out_loc: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       indices: torch.Tensor, cu_k: torch.Tensor, q_norm: torch.Tensor,
                       k_norm: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                       positions: torch.Tensor, eps: float, *, out: torch.Tensor | None = None,
                       workspace: torch.Tensor | None = None,
                       sm_scale: float | None = None) -> torch.Tensor:
    """append_decode with the per-head q/k RMSNorm and rotary embedding
    applied on load (aios_attn_append_decode_rope): q [B, Hq, D] and k
    [B, Hkv, D] are the raw projections (views into the qkv rows), q_norm /
    k_norm bf16 [D], cos / sin the fp32 rotary tables rounded to bf16
    [positions, D], positions int32 [B].  Returns [B, Hq, D] bf16."""
    if p.phase != _lib.PHASE_DECODE:
        raise ValueError("plan was not built for decode")
    _check_q(q, p)
    if q.shape[0] != p.batch_size:
        raise ValueError("decode batch must contain one flat token per request")
    _check_cache(k_cache, p)
    _check_cache(v_cache, p)
    _check_i32(indices, "indices", p.total_kv)
    _check_i32(cu_k, "cu_k", p.batch_size + 1)
    _check_new_kv(k, v, out_loc, p)
    for w, name in ((q_norm, "q_norm"), (k_norm, "k_norm")):
        if w.dtype != torch.bfloat16 or w.numel() != p.head_dim or not w.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bfloat16 [head_dim] tensor")
    if (cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16 or cos.shape != sin.shape
            or cos.ndim != 2 or cos.shape[1] != p.head_dim or not cos.is_contiguous()
            or not sin.is_contiguous()):
        raise ValueError("cos/sin tables must be contiguous bfloat16 [positions, head_dim]")
    _check_i32(positions, "positions", p.batch_size)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if p.ws_bytes and (workspace is None or workspace.numel() < p.ws_bytes):
        raise RuntimeError(f"decode needs a workspace of {p.ws_bytes} bytes")
    scale = p.head_dim ** -0.5 if sm_scale is None else sm_scale
    _lib.check(
        _lib.lib().aios_attn_append_decode_rope(
            p, q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
            out_loc.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0],
            indices.data_ptr(), cu_k.data_ptr(), q_norm.data_ptr(), k_norm.data_ptr(),
            cos.data_ptr(), sin.data_ptr(), cos.shape[0], positions.data_ptr(), float(eps),
            out.data_ptr(), workspace.data_ptr() if workspace is not None else None,
            workspace.numel() if workspace is not None else 0, scale, _stream(q.device)),
        "aios_attn_append_decode_rope",
    )
    return out


def prefill(p: _lib.AttnPlan, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
            indices: torch.Tensor, cu_q: torch.Tensor, cu_k: torch.Tensor, *,
            out: torch.Tensor | None = None, sm_scale: float | None = None) -> torch.Tensor:
    """Varlen causal paged prefill of one layer: returns [total_q, Hq, D] bf16."""
    if p.phase != _lib.PHASE_PREFILL:
        raise ValueError("plan was not built for prefill")
    _check_q(q, p)
    if q.shape[0] != p.total_q:
        raise RuntimeError("prefill request lengths do not match flat Q tokens")
    _check_cache(k_cache, p)
    _check_cache(v_cache, p)
    _check_i32(indices, "indices", p.total_kv)
    _check_i32(cu_q, "cu_q", p.batch_size + 1)
    _check_i32(cu_k, "cu_k", p.batch_size + 1)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    scale = p.head_dim ** -0.5 if sm_scale is None else sm_scale
    _lib.check(
        _lib.lib().aios_attn_prefill(
            p, q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.shape[0], indices.data_ptr(), cu_q.data_ptr(), cu_k.data_ptr(), out.data_ptr(),
            scale,
            _stream(q.device)),
        "aios_attn_prefill",
    )
    return out


def build_indices(page_table: torch.Tensor, row_ids: torch.Tensor, cu_k: torch.Tensor,
                  total_kv: int) -> torch.Tensor:
    """Device gather of the flat page-index list (aios_build_indices)."""
    if page_table.dtype != torch.int32 or page_table.stride(1) != 1:
        raise ValueError("page_table must be int32 with contiguous rows")
    _check_i32(row_ids, "row_ids", 0)
    _check_i32(cu_k, "cu_k", row_ids.numel() + 1)
    out = torch.empty(total_kv, dtype=torch.int32, device=page_table.device)
    _lib.check(
        _lib.lib().aios_build_indices(page_table.data_ptr(), page_table.stride(0),
                                      row_ids.data_ptr(), cu_k.data_ptr(), row_ids.numel(),
                                      total_kv, out.data_ptr(), _stream(page_table.device)),
        "aios_build_indices",
    )
    return out


def greedy_select(logits: torch.Tensor,
                  out: tuple[torch.Tensor, torch.Tensor] | None = None
                  ) -> tuple[torch.Tensor, torch.Tensor]:
    """Greedy token per row and its raw log-probability (aios_greedy_select):
    (argmax(logits, -1) as int64, log_softmax(logits.float())[token] as fp32),
    written into ``out`` (int64 [rows], fp32 [rows]) when given."""
    if logits.ndim != 2 or logits.stride(1) != 1 or not logits.is_cuda:
        raise ValueError("logits must be a 2-D GPU tensor with contiguous rows")
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("logits must be bfloat16 or float32")
    rows, vocab = logits.shape
    if out is not None:
        tok, lp = out
        if (tok.dtype != torch.int64 or lp.dtype != torch.float32 or tok.numel() != rows
                or lp.numel() != rows or not tok.is_contiguous() or not lp.is_contiguous()):
            raise ValueError("out must be (int64 [rows], float32 [rows]) contiguous tensors")
    else:
        tok = torch.empty(rows, dtype=torch.int64, device=logits.device)
        lp = torch.empty(rows, dtype=torch.float32, device=logits.device)
    _lib.check(
        _lib.lib().aios_greedy_select(logits.data_ptr(), logits.stride(0), rows, vocab,
                                      logits.element_size(), tok.data_ptr(), lp.data_ptr(),
                                      _stream(logits.device)),
        "aios_greedy_select",
    )
    return tok, lp


class BoundCall:
    """A C-ABI launch with its arguments converted once.

    For loops that replay the same launch on fixed buffers (benchmarks, graph
    capture): calling the bound function skips the per-call tensor checks and
    ctypes conversions of :func:`decode` / :func:`prefill`.
    """

    def __init__(self, fn, args, keep):
        self._fn = fn
        self._args = args
        self._keep = keep  # tensors and plans the pointers refer to

    def __call__(self) -> None:
        _lib.check(self._fn(*self._args), self._fn.__name__)


def bind_decode(p: _lib.AttnPlan, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                indices: torch.Tensor, cu_k: torch.Tensor, out: torch.Tensor,
                workspace: torch.Tensor | None, sm_scale: float | None = None,
                stream: torch.cuda.Stream | None = None) -> BoundCall:
    """Checked once, then launched many times on the same buffers."""
    import ctypes

    _check_q(q, p)
    _check_cache(k_cache, p)
    _check_cache(v_cache, p)
    _check_i32(indices, "indices", p.total_kv)
    _check_i32(cu_k, "cu_k", p.batch_size + 1)
    if out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like q")
    if p.ws_bytes and (workspace is None or workspace.numel() < p.ws_bytes):
        raise RuntimeError(f"decode needs a workspace of {p.ws_bytes} bytes")
    scale = p.head_dim ** -0.5 if sm_scale is None else sm_scale
    s = stream.cuda_stream if stream is not None else _stream(q.device)
    args = (ctypes.byref(p), q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.shape[0], indices.data_ptr(), cu_k.data_ptr(), out.data_ptr(),
            workspace.data_ptr() if workspace is not None else None,
            workspace.numel() if workspace is not None else 0, ctypes.c_float(scale), s)
    return BoundCall(_lib.lib().aios_attn_decode, args,
                     (p, q, k_cache, v_cache, indices, cu_k, out, workspace))


def bind_append_decode(p: _lib.AttnPlan, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       out_loc: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       indices: torch.Tensor, cu_k: torch.Tensor, out: torch.Tensor,
                       workspace: torch.Tensor | None, sm_scale: float | None = None,
                       stream: torch.cuda.Stream | None = None) -> BoundCall:
    """Checked once, then launched many times: aios_attn_append_decode."""
    import ctypes

    _check_q(q, p)
    _check_cache(k_cache, p)
    _check_cache(v_cache, p)
    _check_i32(indices, "indices", p.total_kv)
    _check_i32(cu_k, "cu_k", p.batch_size + 1)
    _check_new_kv(k, v, out_loc, p)
    if out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like q")
    if p.ws_bytes and (workspace is None or workspace.numel() < p.ws_bytes):
        raise RuntimeError(f"decode needs a workspace of {p.ws_bytes} bytes")
    scale = p.head_dim ** -0.5 if sm_scale is None else sm_scale
    s = stream.cuda_stream if stream is not None else _stream(q.device)
    args = (ctypes.byref(p), q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(),
            v.stride(0), out_loc.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.shape[0], indices.data_ptr(), cu_k.data_ptr(), out.data_ptr(),
            workspace.data_ptr() if workspace is not None else None,
            workspace.numel() if workspace is not None else 0, ctypes.c_float(scale), s)
    return BoundCall(_lib.lib().aios_attn_append_decode, args,
                     (p, q, k, v, out_loc, k_cache, v_cache, indices, cu_k, out, workspace))


def bind_kv_append(k_cache: torch.Tensor, v_cache: torch.Tensor, out_loc: torch.Tensor,
                   k: torch.Tensor, v: torch.Tensor,
                   stream: torch.cuda.Stream | None = None) -> BoundCall:
    """Checked once, then launched many times: store_cache on fixed buffers."""
    if k_cache.ndim != 3 or k.shape[1:] != k_cache.shape[1:] or k.shape != v.shape:
        raise ValueError("K/V input shape does not match the cache layout")
    if out_loc.dtype != torch.int32 or not out_loc.is_contiguous() or out_loc.numel() != k.shape[0]:
        raise ValueError("out_loc must be a contiguous int32 tensor with one entry per token")
    s = stream.cuda_stream if stream is not None else _stream(k.device)
    width = k_cache.shape[1] * k_cache.shape[2]
    args = (k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0], k_cache.stride(0),
            out_loc.data_ptr(), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), k.shape[0],
            width, k.element_size(), s)
    return BoundCall(_lib.lib().aios_kv_append, args, (k_cache, v_cache, out_loc, k, v))
