"""aios_attn_decode_noalloc, the allocation-free decode entry point: its
partial states live in the library's built-in device array instead of a
caller workspace.  Checked through the C ABI against aios_attn_decode on the
same plan (the same kernels: bit-equal outputs) and against the float64
oracle, on two calls in a row, the second with a smaller batch, and for the
rejection of a plan whose partial states exceed the built-in array."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aios_amd import _lib, paged
from aios_amd.workloads import LONG_CONTEXT, OP_TEST, make_decode_workload
from oracle import attention as oatt
from tests.util import BF16_TOL, to_np64

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(shape, seed, chunk):
    """Plan and device buffers of one decode layer (held by name until the
    calls that read them have run)."""
    wl = make_decode_workload(shape, seed=seed, layers=1, extra_token=True)
    n = shape.num_rows
    p = paged.plan("decode", torch.arange(n + 1, dtype=torch.int32), wl.cu_k,
                   shape.num_qo_heads, shape.num_kv_heads, shape.head_dim,
                   shared_prefix_len=shape.prefix_len, workspace_bytes=64 << 20,
                   prefix_chunk_len=chunk)
    bufs = dict(q=wl.q[0].to(DEV), kc=wl.k_cache[0].to(DEV), vc=wl.v_cache[0].to(DEV),
                idx=wl.indices.to(DEV), cu_k=wl.cu_k.to(DEV))
    return wl, p, bufs


def _abi_decode(p, b, ws):
    out = torch.full_like(b["q"], float("nan"))
    rc = _lib.lib().aios_attn_decode(
        p, b["q"].data_ptr(), b["q"].stride(0), b["kc"].data_ptr(), b["vc"].data_ptr(),
        b["kc"].shape[0], b["idx"].data_ptr(), b["cu_k"].data_ptr(), out.data_ptr(),
        ws.data_ptr(), ws.numel(), p.head_dim ** -0.5,
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.lib().aios_last_error()
    return out


def _abi_noalloc(p, b):
    out = torch.full_like(b["q"], float("nan"))
    rc = _lib.lib().aios_attn_decode_noalloc(
        p, b["q"].data_ptr(), b["q"].stride(0), b["kc"].data_ptr(), b["vc"].data_ptr(),
        b["kc"].shape[0], b["idx"].data_ptr(), b["cu_k"].data_ptr(), out.data_ptr(),
        p.head_dim ** -0.5, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.lib().aios_last_error()
    return out


def test_noalloc_matches_workspace_decode_on_two_calls():
    # call 1: the long-context layer (32 prefix chunks + suffix parts, ~7 MB
    # of partial states); call 2: the op-test layer with a forced cascade
    # (5 parts per row and head, a much smaller batch)
    cases = [(LONG_CONTEXT, 20260814, 0), (OP_TEST, 7, 32)]
    for shape, seed, chunk in cases:
        wl, p, b = _case(shape, seed, chunk)
        assert 0 < p.ws_bytes <= _lib.DECODE_NOALLOC_MAX_BYTES and p.num_parts > 1
        ws = torch.empty(p.ws_bytes, dtype=torch.uint8, device=DEV)
        ref = _abi_decode(p, b, ws)
        got = _abi_noalloc(p, b)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), shape.name
        if shape is OP_TEST:
            expect = oatt.decode_attention(to_np64(wl.q[0]), to_np64(wl.k_cache[0]),
                                           to_np64(wl.v_cache[0]), wl.indices.numpy(),
                                           wl.cu_k.numpy(), shape.head_dim ** -0.5)
            np.testing.assert_allclose(to_np64(got), expect, **BF16_TOL)
        del b, ws


def test_noalloc_wrapper_and_repeat():
    """The Python wrapper gives the same result, and a repeated call on the
    same inputs (the array keeps the previous call's contents) too."""
    wl, p, b = _case(OP_TEST, 11, 32)
    ws = torch.empty(p.ws_bytes, dtype=torch.uint8, device=DEV)
    ref = _abi_decode(p, b, ws)
    out = torch.empty_like(b["q"])
    for _ in range(2):
        paged.decode_noalloc(p, b["q"], b["kc"], b["vc"], b["idx"], b["cu_k"], out=out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_noalloc_rejects_plan_beyond_its_array():
    """A plan needing more partial-state bytes than the built-in array is
    refused before any launch."""
    wl, _, b = _case(LONG_CONTEXT, 20260814, 0)
    n = LONG_CONTEXT.num_rows
    p = paged.plan("decode", torch.arange(n + 1, dtype=torch.int32), wl.cu_k,
                   LONG_CONTEXT.num_qo_heads, LONG_CONTEXT.num_kv_heads, LONG_CONTEXT.head_dim,
                   shared_prefix_len=LONG_CONTEXT.prefix_len, workspace_bytes=64 << 20,
                   suffix_split_len=16)
    assert p.ws_bytes > _lib.DECODE_NOALLOC_MAX_BYTES
    out = torch.zeros_like(b["q"])
    rc = _lib.lib().aios_attn_decode_noalloc(
        p, b["q"].data_ptr(), b["q"].stride(0), b["kc"].data_ptr(), b["vc"].data_ptr(),
        b["kc"].shape[0], b["idx"].data_ptr(), b["cu_k"].data_ptr(), out.data_ptr(),
        p.head_dim ** -0.5, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.AIOS_ERR_WORKSPACE
    assert "built-in" in _lib.lib().aios_last_error().decode()
    torch.cuda.synchronize()
    assert not out.any()
