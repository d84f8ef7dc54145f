"""Paged decode (cascade kernel (c) + suffix kernel (d) + LSE combine) vs the oracle.

The oracle (oracle/attention.py) is float64 offset-causal GQA attention over
the gathered pages (the reference's flashinfer.py:33-91 / :374-394 math);
bf16 kernel outputs must match within atol = rtol = 1e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aios_amd import paged
from aios_amd.workloads import (LONG_CONTEXT, OP_TEST, DecodeShape,
                                make_decode_workload)
from oracle import attention as oatt
from tests.util import BF16_TOL, to_np64

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(wl, layer=0, shared=None, chunk=0, split=0, ws_bytes=64 << 20):
    shape = wl.shape
    n = shape.num_rows
    cu_q = torch.arange(n + 1, dtype=torch.int32)
    p = paged.plan("decode", cu_q, wl.cu_k, shape.num_qo_heads, shape.num_kv_heads,
                   shape.head_dim, shared_prefix_len=shape.prefix_len if shared is None else shared,
                   workspace_bytes=ws_bytes, prefix_chunk_len=chunk, suffix_split_len=split)
    ws = torch.empty(max(p.ws_bytes, 1), dtype=torch.uint8, device=DEV)
    q = wl.q[layer].to(DEV)
    kc = wl.k_cache[layer].to(DEV)
    vc = wl.v_cache[layer].to(DEV)
    out = paged.decode(p, q, kc, vc, wl.indices.to(DEV), wl.cu_k.to(DEV), workspace=ws)
    torch.cuda.synchronize()
    return out, p


def _oracle(wl, layer=0, rows=None):
    shape = wl.shape
    q = to_np64(wl.q[layer])
    kc = to_np64(wl.k_cache[layer])
    vc = to_np64(wl.v_cache[layer])
    ref = oatt.decode_attention(q, kc, vc, wl.indices.numpy(), wl.cu_k.numpy(),
                                shape.head_dim ** -0.5)
    return ref


def test_op_test_config_default_plan():
    wl = make_decode_workload(OP_TEST, seed=20260814)
    out, p = _run(wl)
    assert p.num_parts == 1  # short prefix: one launch, rows read it directly
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


def test_op_test_config_cascade():
    wl = make_decode_workload(OP_TEST, seed=20260814)
    out, p = _run(wl, chunk=32)
    assert p.prefix_len == 24 and p.num_prefix_chunks == 1
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


def test_op_test_golden_fixture():
    """HIP output on the committed op-test fixture's inputs vs its stored
    float64 output (tests/golden/op_test_decode.npz)."""
    import os

    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "op_test_decode.npz"))
    t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(DEV)
    n = len(fx["cu_k"]) - 1
    cu_k = torch.from_numpy(fx["cu_k"])
    for chunk in (0, 32):
        p = paged.plan("decode", torch.arange(n + 1, dtype=torch.int32), cu_k, 8, 2, 96,
                       shared_prefix_len=24, workspace_bytes=16 << 20, prefix_chunk_len=chunk)
        ws = torch.empty(max(p.ws_bytes, 1), dtype=torch.uint8, device=DEV)
        out = paged.decode(p, t(fx["q_bits"]), t(fx["k_bits"]), t(fx["v_bits"]),
                           torch.from_numpy(fx["indices"]).to(DEV), cu_k.to(DEV), workspace=ws)
        torch.cuda.synchronize()
        np.testing.assert_allclose(to_np64(out), fx["out"], **BF16_TOL)


def test_op_test_config_without_shared_prefix():
    wl = make_decode_workload(OP_TEST, seed=20260814)
    out, p = _run(wl, shared=0)
    assert p.prefix_len == 0
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_cascade_and_plain_paths_agree(seed):
    wl = make_decode_workload(OP_TEST, seed=seed)
    a, pa = _run(wl, chunk=32)
    assert pa.prefix_len == 24
    b, _ = _run(wl, shared=0)
    ref = _oracle(wl)
    np.testing.assert_allclose(to_np64(a), ref, **BF16_TOL)
    np.testing.assert_allclose(to_np64(b), ref, **BF16_TOL)
    np.testing.assert_allclose(to_np64(a), to_np64(b), atol=1e-2, rtol=1e-2)


def test_all_suffixes_empty():
    shape = DecodeShape("empty_suffix", 1, 8, 40, 0, 8, 2, 96, 256)
    wl = make_decode_workload(shape, seed=5)
    assert all(s == 0 for s in wl.suffix_lens)
    out, p = _run(wl, chunk=32)
    assert p.prefix_len == 40
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)
    # every row attends to the same prefix with its own query
    out0, _ = _run(wl, shared=0)
    np.testing.assert_allclose(to_np64(out), to_np64(out0), **BF16_TOL)


@pytest.mark.parametrize("chunk,split", [(32, 0), (64, 8), (0, 4), (32, 3)])
def test_forced_chunking_and_splits(chunk, split):
    shape = DecodeShape("chunked", 1, 8, 200, 40, 8, 2, 96, 1024)
    wl = make_decode_workload(shape, seed=11)
    out, p = _run(wl, chunk=chunk, split=split)
    if split:
        assert p.num_suffix_splits > 1
    if chunk:
        assert p.num_prefix_chunks == -(-200 // chunk)
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 64), (16, 8, 128), (32, 8, 128), (12, 4, 64),
                                      (8, 8, 96), (16, 2, 128), (24, 4, 96)])
def test_head_shapes(hq, hkv, d):
    shape = DecodeShape(f"h{hq}_{hkv}_{d}", 1, 8, 75, 20, hq, hkv, d, 512)
    wl = make_decode_workload(shape, seed=hq * 100 + d)
    ref = _oracle(wl)
    out, _ = _run(wl)
    np.testing.assert_allclose(to_np64(out), ref, **BF16_TOL)
    out0, _ = _run(wl, shared=0)
    np.testing.assert_allclose(to_np64(out0), ref, **BF16_TOL)
    out1, _ = _run(wl, chunk=32)
    np.testing.assert_allclose(to_np64(out1), ref, **BF16_TOL)


def test_single_row_and_kv_len_one():
    shape = DecodeShape("one", 1, 1, 1, 0, 8, 2, 96, 16)
    wl = make_decode_workload(shape, seed=2)
    out, p = _run(wl)
    # one visible key: the output is that key's value row (closed form)
    v = wl.v_cache[0][wl.indices.long()[0]].float()  # [Hkv, D]
    expect = v.repeat_interleave(4, dim=0)
    torch.testing.assert_close(out[0].float().cpu(), expect, atol=1e-2, rtol=1e-2)


def test_many_rows_multiple_mgroups():
    shape = DecodeShape("wide", 1, 48, 96, 12, 16, 4, 64, 2048)  # M = 48*4 = 192 rows
    wl = make_decode_workload(shape, seed=21)
    out, p = _run(wl, chunk=32)
    assert p.cascade_mgroups == 2
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


def test_long_context_single_layer():
    wl = make_decode_workload(LONG_CONTEXT, seed=20260814, layers=1, extra_token=True)
    out, p = _run(wl)
    assert p.num_prefix_chunks > 1
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


def _oracle_rows(wl, layer, rows, k_cache, v_cache):
    """Float64 oracle outputs of `rows` of one layer, over only their pages."""
    shape = wl.shape
    spans = [wl.indices[int(wl.cu_k[r]):int(wl.cu_k[r + 1])].long() for r in rows]
    pages, inv = torch.unique(torch.cat(spans), return_inverse=True)
    lens = [len(s) for s in spans]
    cu = np.zeros(len(rows) + 1, dtype=np.int64)
    cu[1:] = np.cumsum(lens)
    dev_pages = pages.to(k_cache.device)
    kc = to_np64(k_cache[layer].index_select(0, dev_pages))
    vc = to_np64(v_cache[layer].index_select(0, dev_pages))
    q = to_np64(wl.q[layer][list(rows)])
    return oatt.decode_attention(q, kc, vc, inv.numpy().astype(np.int64), cu,
                                 shape.head_dim ** -0.5)


def test_long_context_step_every_layer():
    # The whole 36-layer long-context step as bench.py times it: one HIP
    # graph of 36 x (fused KV append + cascade main launch, combine),
    # replayed twice.  Every layer's output is checked against the plain
    # (unshared) decode of the appended caches, and two rows of every layer
    # (all 24 rows over the 36 layers) against the float64 oracle.
    shape = LONG_CONTEXT
    wl = make_decode_workload(shape, seed=20260814, device=DEV, extra_token=True)
    n, nl = shape.num_rows, shape.num_layers
    hq, hkv, d = shape.num_qo_heads, shape.num_kv_heads, shape.head_dim
    g = torch.Generator(device=DEV).manual_seed(20260821)
    k_new = (torch.randn(nl, n, hkv, d, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    v_new = (torch.randn(nl, n, hkv, d, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    last = wl.indices[(wl.cu_k[1:] - 1).long()].to(DEV)
    indices = wl.indices.to(DEV)
    cu_k = wl.cu_k.to(DEV)
    cu_q = torch.arange(n + 1, dtype=torch.int32)
    main_plan = paged.plan("decode", cu_q, wl.cu_k, hq, hkv, d, shared_prefix_len=shape.prefix_len)
    assert main_plan.num_prefix_chunks > 1 and main_plan.num_parts > 1
    comb_plan = paged.plan("decode", cu_q, wl.cu_k, hq, hkv, d, shared_prefix_len=shape.prefix_len)
    main_plan.stage_mask = 1
    comb_plan.stage_mask = 2
    ws = torch.empty(main_plan.ws_bytes, dtype=torch.uint8, device=DEV)
    out = torch.empty(nl, n, hq, d, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()
    calls = []
    for layer in range(nl):
        calls.append(paged.bind_append_decode(main_plan, wl.q[layer], k_new[layer], v_new[layer],
                                              last, wl.k_cache[layer], wl.v_cache[layer],
                                              indices, cu_k, out[layer], ws, stream=s))
        calls.append(paged.bind_decode(comb_plan, wl.q[layer], wl.k_cache[layer],
                                       wl.v_cache[layer], indices, cu_k, out[layer], ws, stream=s))
    graph = torch.cuda.CUDAGraph()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls:  # eager once (also the warm-up the capture needs)
            c()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=s):
        for c in calls:
            c()
    outs = []
    for _ in range(2):
        with torch.cuda.stream(s):
            out.zero_()
            graph.replay()
        torch.cuda.synchronize()
        outs.append(out.clone())
    assert torch.equal(outs[0], outs[1])

    plain = paged.plan("decode", cu_q, wl.cu_k, hq, hkv, d, shared_prefix_len=0)
    ws_plain = torch.empty(max(plain.ws_bytes, 1), dtype=torch.uint8, device=DEV)
    for layer in range(nl):
        # the appended rows are in the caches, as the step left them
        assert torch.equal(wl.k_cache[layer][last.long()], k_new[layer])
        assert torch.equal(wl.v_cache[layer][last.long()], v_new[layer])
        ref = paged.decode(plain, wl.q[layer], wl.k_cache[layer], wl.v_cache[layer], indices,
                           cu_k, workspace=ws_plain)
        np.testing.assert_allclose(to_np64(out[layer]), to_np64(ref), **BF16_TOL)
        rows = (layer % n, (layer + n // 2) % n)
        np.testing.assert_allclose(to_np64(out[layer][list(rows)]),
                                   _oracle_rows(wl, layer, rows, wl.k_cache, wl.v_cache),
                                   **BF16_TOL)


@pytest.mark.parametrize("rows,hq,hkv,d,prefix,shared", [(24, 32, 8, 128, 1024, True),
                                                          (16, 16, 8, 128, 512, True),
                                                          (8, 8, 2, 96, 300, True),
                                                          (6, 32, 8, 128, 700, False)])
def test_growing_logits_move_the_softmax_reference(rows, hq, hkv, d, prefix, shared):
    # K rows scaled up along the positions (x1 at position 0 to x51 at the
    # longest row's end) make a row's running max grow by ~60 log2 units, so
    # the softmax reference moves several times inside the prefix chunks
    # (each move rescales O and the row sums) instead of only at the first
    # sub-tile, as it does with unit-scale data.
    shape = DecodeShape("growing", 1, rows, prefix, 64, hq, hkv, d, 8192)
    wl = make_decode_workload(shape, seed=20260903 + rows)
    kv_max = int((wl.cu_k[1:] - wl.cu_k[:-1]).max())
    scale = torch.ones(shape.num_pages)
    for b in range(rows):
        lo, hi = int(wl.cu_k[b]), int(wl.cu_k[b + 1])
        pos = torch.arange(hi - lo, dtype=torch.float32)
        scale[wl.indices[lo:hi].long()] = 1.0 + 50.0 * pos / kv_max
    wl.k_cache = (wl.k_cache.float() * scale.view(1, -1, 1, 1)).to(torch.bfloat16)
    out, p = _run(wl, shared=None if shared else 0)
    assert (p.num_prefix_chunks > 1) == shared
    # row 0's running max (log2 units, its first query head) climbs by
    # more than twice the reference's 2^8 slack along its positions
    idx0 = wl.indices[int(wl.cu_k[0]):int(wl.cu_k[1])].long()
    sc = to_np64(wl.k_cache[0][idx0, 0]) @ to_np64(wl.q[0][0, 0]) * d ** -0.5 * np.log2(np.e)
    run = np.maximum.accumulate(sc)
    assert run[-1] - run[0] > 16.0
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


def test_page_permutation_invariance():
    # Relabelling physical pages (and moving their rows) must not change the output.
    wl = make_decode_workload(OP_TEST, seed=8)
    out, _ = _run(wl)
    g = torch.Generator().manual_seed(99)
    perm = torch.randperm(OP_TEST.num_pages, generator=g)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(len(perm))
    wl.k_cache = wl.k_cache[:, perm]
    wl.v_cache = wl.v_cache[:, perm]
    wl.indices = inv[wl.indices.long()].to(torch.int32)
    out2, _ = _run(wl)
    assert torch.equal(out.cpu(), out2.cpu())


@pytest.mark.parametrize("hq,hkv,d,rows,lo,hi", [(16, 8, 128, 3, 1500, 3000),
                                                 (32, 8, 128, 4, 4000, 4160),
                                                 (8, 2, 96, 3, 2000, 2500)])
def test_long_rows_without_shared_prefix(hq, hkv, d, rows, lo, hi):
    # Generic paged decode (no shared prefix): long rows are split and merged.
    shape = DecodeShape("long_rows", 1, rows, 0, hi, hq, hkv, d, 32768, min_suffix=lo)
    wl = make_decode_workload(shape, seed=31)
    out, p = _run(wl, shared=0)
    assert p.num_suffix_splits > 1 and p.num_parts > 1
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


@pytest.mark.parametrize("max_suffix", [33, 64, 65, 128, 129, 200])
def test_single_launch_row_lengths(max_suffix):
    # Rows of up to two passes of one suffix wavefront are covered by one item
    # (no partials, no combine); longer rows are split and merged.
    shape = DecodeShape("rows", 1, 6, 0, max_suffix, 8, 2, 96, 2048, min_suffix=max_suffix)
    wl = make_decode_workload(shape, seed=max_suffix)
    out, p = _run(wl, shared=0)
    assert (p.num_parts == 1) == (max_suffix <= 2 * 4 * p.suffix_tpg)
    np.testing.assert_allclose(to_np64(out), _oracle(wl), **BF16_TOL)


def _append_decode_case(shape, seed, shared=None, chunk=0, split=0, oob_row=None):
    wl = make_decode_workload(shape, seed=seed, extra_token=True)
    n, hkv, d = shape.num_rows, shape.num_kv_heads, shape.head_dim
    g = torch.Generator().manual_seed(seed + 99)
    k_new = (torch.randn(n, hkv, d, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    # v as a strided view, the way it leaves the fused qkv projection
    v_big = (torch.randn(n, 3 * hkv, d, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    v_new = v_big[:, hkv:2 * hkv]
    last = torch.tensor([int(wl.indices[int(wl.cu_k[i + 1]) - 1]) for i in range(n)],
                        dtype=torch.int32)
    if oob_row is not None:
        last[oob_row] = shape.num_pages + 5
        wl.indices[int(wl.cu_k[oob_row + 1]) - 1] = shape.num_pages + 5
    out_loc = last.to(DEV)
    cu_q = torch.arange(n + 1, dtype=torch.int32)
    p = paged.plan("decode", cu_q, wl.cu_k, shape.num_qo_heads, hkv, d,
                   shared_prefix_len=shape.prefix_len if shared is None else shared,
                   workspace_bytes=64 << 20, prefix_chunk_len=chunk, suffix_split_len=split)
    ws = torch.empty(max(p.ws_bytes, 256), dtype=torch.uint8, device=DEV)
    q = wl.q[0].to(DEV)
    idx = wl.indices.to(DEV)
    cuk = wl.cu_k.to(DEV)
    # separate calls: store_cache then decode
    ka, va = wl.k_cache[0].to(DEV), wl.v_cache[0].to(DEV)
    from aios_amd.kernel import store_cache
    store_cache(ka, va, out_loc, k_new, v_new)
    out_a = paged.decode(p, q, ka, va, idx, cuk, workspace=ws)
    # one launch
    kb, vb = wl.k_cache[0].to(DEV), wl.v_cache[0].to(DEV)
    out_b = paged.append_decode(p, q, k_new, v_new, out_loc, kb, vb, idx, cuk, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(bits_t(ka), bits_t(kb)) and torch.equal(bits_t(va), bits_t(vb))
    assert torch.equal(out_a, out_b)
    if oob_row is None:  # (the oracle has no out-of-range page semantics)
        ref = oatt.decode_attention(to_np64(q), to_np64(ka), to_np64(va), wl.indices.numpy(),
                                    wl.cu_k.numpy(), d ** -0.5)
        np.testing.assert_allclose(to_np64(out_b), ref, **BF16_TOL)
    return p


def bits_t(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("case", ["op_test", "cascade", "splits", "long_context_layer",
                                  "h64_g3", "h128_g2", "no_shared"])
def test_append_decode_matches_separate_calls(case):
    """KV append inside the decode launch: caches bit-identical and outputs
    bitwise equal to store_cache followed by decode."""
    if case == "op_test":
        p = _append_decode_case(OP_TEST, 20260814)
        assert p.num_parts == 1
    elif case == "cascade":
        p = _append_decode_case(OP_TEST, 3, chunk=32)
        assert p.prefix_len == 24
    elif case == "splits":
        p = _append_decode_case(DecodeShape("sp", 1, 8, 200, 40, 8, 2, 96, 1024), 11, chunk=64,
                                split=8)
        assert p.num_suffix_splits > 1
    elif case == "long_context_layer":
        shape = DecodeShape("lc1", 1, 24, 4096, 64, 32, 8, 128, 65536)
        p = _append_decode_case(shape, 20260814)
        assert p.num_prefix_chunks > 1
    elif case == "h64_g3":
        _append_decode_case(DecodeShape("h64", 1, 8, 150, 20, 12, 4, 64, 512), 5)
    elif case == "h128_g2":
        _append_decode_case(DecodeShape("h128", 1, 8, 140, 24, 16, 8, 128, 512), 6)
    else:
        _append_decode_case(OP_TEST, 9, shared=0)


def _append_decode_rope_case(shape, seed, shared=None, chunk=0, split=0):
    """aios_attn_append_decode_rope against aios_qk_norm_rope followed by
    aios_attn_append_decode on the same raw qkv rows: V rows bitwise equal;
    each new K element equal or one bf16 unit apart (the head's fp32 sum of
    squares is taken in another order) and almost all equal; attention
    outputs within the bf16 tolerance of the separate path's and of the
    float64 oracle over the fused path's cache."""
    from aios_amd.layers import HipOps
    from aios_amd.qwen3 import RotaryEmbedding

    wl = make_decode_workload(shape, seed=seed, extra_token=True)
    n, hq, hkv, d = shape.num_rows, shape.num_qo_heads, shape.num_kv_heads, shape.head_dim
    g = torch.Generator().manual_seed(seed + 7)
    qkv = torch.randn(n, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(DEV)
    qw = (1.0 + 0.2 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV)
    kw = (1.0 + 0.2 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV)
    rot = RotaryEmbedding(d, 8192, 1e6, DEV)
    kv_len = (wl.cu_k[1:] - wl.cu_k[:-1]).to(torch.int32)
    positions = (kv_len - 1).to(DEV)
    eps = 1e-6
    last = torch.tensor([int(wl.indices[int(wl.cu_k[i + 1]) - 1]) for i in range(n)],
                        dtype=torch.int32)
    out_loc = last.to(DEV)
    cu_q = torch.arange(n + 1, dtype=torch.int32)
    p = paged.plan("decode", cu_q, wl.cu_k, hq, hkv, d,
                   shared_prefix_len=shape.prefix_len if shared is None else shared,
                   workspace_bytes=64 << 20, prefix_chunk_len=chunk, suffix_split_len=split)
    ws = torch.empty(max(p.ws_bytes, 256), dtype=torch.uint8, device=DEV)
    idx = wl.indices.to(DEV)
    cuk = wl.cu_k.to(DEV)
    v = qkv[:, (hq + hkv) * d:].view(n, hkv, d)
    # separate: q/k norm + rotation, then append + decode
    q_a, k_a = HipOps.qk_norm_rope(qkv, qw, kw, rot.cos, rot.sin, positions, hq, hkv, d, eps)
    ka, va = wl.k_cache[0].to(DEV), wl.v_cache[0].to(DEV)
    out_a = paged.append_decode(p, q_a, k_a, v, out_loc, ka, va, idx, cuk, workspace=ws)
    # one launch from the raw projections
    q_raw = qkv[:, :hq * d].view(n, hq, d)
    k_raw = qkv[:, hq * d:(hq + hkv) * d].view(n, hkv, d)
    kb, vb = wl.k_cache[0].to(DEV), wl.v_cache[0].to(DEV)
    out_b = paged.append_decode_rope(p, q_raw, k_raw, v, out_loc, kb, vb, idx, cuk, qw, kw,
                                     rot.cos_bf16, rot.sin_bf16, positions, eps, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(bits_t(va), bits_t(vb))
    rest = torch.ones(ka.shape[0], dtype=torch.bool)
    rest[last.long()] = False
    assert torch.equal(bits_t(ka[rest.to(DEV)]), bits_t(kb[rest.to(DEV)]))
    new_a, new_b = ka[out_loc.long()].float(), kb[out_loc.long()].float()
    # one unit of the normalised element moves the rotated one by at most
    # about one unit of the head's largest element
    scale = new_a.abs().amax(dim=-1, keepdim=True)
    assert bool(((new_a - new_b).abs() <= scale * 2.0 ** -6).all())
    assert float((new_a == new_b).float().mean()) > 0.97
    np.testing.assert_allclose(to_np64(out_b), to_np64(out_a), **BF16_TOL)
    ref = oatt.decode_attention(to_np64(q_a), to_np64(kb), to_np64(vb), wl.indices.numpy(),
                                wl.cu_k.numpy(), d ** -0.5)
    np.testing.assert_allclose(to_np64(out_b), ref, **BF16_TOL)
    return p


@pytest.mark.parametrize("case", ["op_test", "cascade", "splits", "long_context_layer",
                                  "h64_g3", "h128_g2", "h64_cascade", "h128_cascade"])
def test_append_decode_rope_matches_separate_ops(case):
    """The q/k norm + rotary embedding taken inside the decode launch, for
    both tile engines (prefix cascade: 32-row tiles; suffix items: 16-row
    tiles) at head sizes 64, 96 and 128."""
    if case == "op_test":
        p = _append_decode_rope_case(OP_TEST, 20260814)
        assert p.prefix_len == 0
    elif case == "cascade":
        p = _append_decode_rope_case(OP_TEST, 3, chunk=32)
        assert p.prefix_len == 24
    elif case == "splits":
        p = _append_decode_rope_case(DecodeShape("sp", 1, 8, 200, 40, 8, 2, 96, 1024), 11,
                                     chunk=64, split=8)
        assert p.num_suffix_splits > 1
    elif case == "long_context_layer":
        shape = DecodeShape("lc1", 1, 24, 4096, 64, 32, 8, 128, 65536)
        p = _append_decode_rope_case(shape, 20260814)
        assert p.num_prefix_chunks > 1
    elif case == "h64_g3":
        _append_decode_rope_case(DecodeShape("h64", 1, 8, 150, 20, 12, 4, 64, 512), 5, shared=0)
    elif case == "h128_g2":
        _append_decode_rope_case(DecodeShape("h128", 1, 8, 140, 24, 16, 8, 128, 512), 6, shared=0)
    elif case == "h64_cascade":
        p = _append_decode_rope_case(DecodeShape("h64c", 1, 8, 150, 20, 12, 4, 64, 512), 5,
                                     chunk=64)
        assert p.prefix_len == 150
    else:
        p = _append_decode_rope_case(DecodeShape("h128c", 1, 8, 140, 24, 16, 8, 128, 512), 6,
                                     chunk=64)
        assert p.prefix_len == 140


@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 64), (8, 8, 128), (48, 8, 96), (64, 8, 128),
                                      (32, 4, 64)])
def test_append_decode_rope_group_sizes(hq, hkv, d):
    """The rotation's pair layout at the group sizes the other cases leave
    out: G = 1 (one query row and the K row), G = 6, and G = 8, whose nine
    rows take two passes of eight lanes per row; suffixes long enough for
    a wavefront's second sub-tile."""
    shape = DecodeShape(f"g{hq // hkv}_{d}", 1, 4, 60, 90, hq, hkv, d, 1024, min_suffix=40)
    _append_decode_rope_case(shape, 31 + hq + d, shared=0)


def test_append_decode_out_of_range_slot_matches_separate_calls():
    _append_decode_case(OP_TEST, 4, chunk=32, oob_row=3)


def test_append_decode_rejects_new_token_inside_shared_prefix():
    shape = DecodeShape("empty_suffix", 1, 8, 40, 0, 8, 2, 96, 256)
    wl = make_decode_workload(shape, seed=5)
    n = shape.num_rows
    p = paged.plan("decode", torch.arange(n + 1, dtype=torch.int32), wl.cu_k, 8, 2, 96,
                   shared_prefix_len=40, prefix_chunk_len=32)
    kv = torch.zeros(n, 2, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="after the shared prefix"):
        paged.append_decode(p, wl.q[0].to(DEV), kv, kv, torch.zeros(n, dtype=torch.int32, device=DEV),
                            wl.k_cache[0].to(DEV), wl.v_cache[0].to(DEV), wl.indices.to(DEV),
                            wl.cu_k.to(DEV), workspace=torch.empty(1 << 20, dtype=torch.uint8,
                                                                   device=DEV))


def test_layer_cache_above_4gib_is_rejected():
    """The kernels address a layer's cache with 32-bit byte offsets: a page
    count that puts the cache at 4 GiB is refused before any launch."""
    from aios_amd import _lib

    wl = make_decode_workload(OP_TEST, seed=3)
    out, p = _run(wl)
    q = wl.q[0].to(DEV)
    kc = wl.k_cache[0].to(DEV)
    ws = torch.empty(max(p.ws_bytes, 1), dtype=torch.uint8, device=DEV)
    pages = (1 << 32) // (p.num_kv_heads * p.head_dim * 2)
    idx, cu_k = wl.indices.to(DEV), wl.cu_k.to(DEV)
    status = _lib.lib().aios_attn_decode(
        p, q.data_ptr(), q.stride(0), kc.data_ptr(), kc.data_ptr(), pages, idx.data_ptr(),
        cu_k.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), p.head_dim ** -0.5, None)
    assert status == _lib.AIOS_ERR_UNSUPPORTED
    assert "4 GiB" in _lib.lib().aios_last_error().decode()


def test_misaligned_output_is_rejected():
    """Kernels store 16-byte vectors: an output view 8 bytes off alignment is
    refused with ValueError before any launch."""
    wl = make_decode_workload(OP_TEST, seed=4)
    out, p = _run(wl)
    ws = torch.empty(max(p.ws_bytes, 1), dtype=torch.uint8, device=DEV)
    flat = torch.empty(out.numel() + 8, dtype=torch.bfloat16, device=DEV)
    bad = flat[4:4 + out.numel()].view(out.shape)
    with pytest.raises(ValueError, match="16-byte aligned"):
        paged.decode(p, wl.q[0].to(DEV), wl.k_cache[0].to(DEV), wl.v_cache[0].to(DEV),
                     wl.indices.to(DEV), wl.cu_k.to(DEV), out=bad, workspace=ws)


def test_empty_batches_are_noops():
    """A batch with no requests: decode and prefill plans carry no work, and
    the calls return empty outputs without touching the caches."""
    cu = torch.zeros(1, dtype=torch.int32)
    kc = torch.randn(16, 2, 96, device=DEV).to(torch.bfloat16)
    vc = torch.randn(16, 2, 96, device=DEV).to(torch.bfloat16)
    k0, v0 = kc.clone(), vc.clone()
    idx = torch.zeros(0, dtype=torch.int32, device=DEV)
    q = torch.zeros(0, 8, 96, dtype=torch.bfloat16, device=DEV)
    pd = paged.plan("decode", cu, cu, 8, 2, 96)
    assert pd.batch_size == 0 and pd.ws_bytes == 0
    out = paged.decode(pd, q, kc, vc, idx, cu.to(DEV))
    pp = paged.plan("prefill", cu, cu, 8, 2, 96)
    assert pp.num_q_tiles == 0
    out2 = paged.prefill(pp, q, kc, vc, idx, cu.to(DEV), cu.to(DEV))
    torch.cuda.synchronize()
    assert out.shape == (0, 8, 96) and out2.shape == (0, 8, 96)
    assert torch.equal(kc, k0) and torch.equal(vc, v0)
