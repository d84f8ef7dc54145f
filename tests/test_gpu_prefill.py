"""Varlen causal paged prefill (HIP kernel (b)) vs the float64 oracle.

Covers a fresh prefix (cached_len 0), the reference test's offset case
(tests/test_attention_backend.py:25-53: seed 17, cached_len in {0, 2},
q_len 3, 4 query / 2 KV heads), the cross-keystroke extension (2 new tokens
against a cached 128-token prefix, Qwen3-0.6B heads), multi-request varlen
batches and a 4096-token prefill checked on sampled query rows.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aios_amd import paged
from oracle import attention as oatt
from tests.util import BF16_TOL, to_np64

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _make(q_lens, kv_lens, hq, hkv, d, pool, seed):
    g = torch.Generator().manual_seed(seed)
    total_kv = sum(kv_lens)
    perm = torch.randperm(pool, generator=g)[:total_kv].to(torch.int32)
    cu_q = torch.zeros(len(q_lens) + 1, dtype=torch.int32)
    cu_q[1:] = torch.tensor(q_lens).cumsum(0)
    cu_k = torch.zeros(len(kv_lens) + 1, dtype=torch.int32)
    cu_k[1:] = torch.tensor(kv_lens).cumsum(0)
    q = (torch.randn(sum(q_lens), hq, d, generator=g) * 0.5).to(torch.bfloat16)
    kc = (torch.randn(pool, hkv, d, generator=g) * 0.5).to(torch.bfloat16)
    vc = (torch.randn(pool, hkv, d, generator=g) * 0.5).to(torch.bfloat16)
    return q, kc, vc, perm, cu_q, cu_k


def _run(q, kc, vc, idx, cu_q, cu_k, hq, hkv, d):
    p = paged.plan("prefill", cu_q, cu_k, hq, hkv, d)
    out = paged.prefill(p, q.to(DEV), kc.to(DEV), vc.to(DEV), idx.to(DEV), cu_q.to(DEV),
                        cu_k.to(DEV))
    torch.cuda.synchronize()
    return out, p


def _oracle(q, kc, vc, idx, cu_q, cu_k, d):
    return oatt.paged_attention(to_np64(q), to_np64(kc), to_np64(vc), idx.numpy(), cu_q.numpy(),
                                cu_k.numpy(), d ** -0.5)


@pytest.mark.parametrize("q_lens,kv_lens,hq,hkv,d", [
    ([32], [32], 8, 2, 96),            # MiniMind-0.1B-shaped prefix prefill
    ([64], [64], 12, 4, 64),           # deployed 0.1B heads (G=3)
    ([128], [128], 16, 8, 128),        # Qwen3-0.6B-shaped prefix
    ([2], [130], 16, 8, 128),          # cross-keystroke extension: 2 tokens vs cached 128
    ([1], [77], 8, 2, 96),             # single-token extension
    ([3, 1, 40, 17], [3, 9, 40, 50], 8, 2, 96),  # ragged batch, mixed cached_len
    ([100, 33], [131, 33], 32, 8, 128),
    ([5], [5], 8, 8, 64),
])
def test_prefill_matches_oracle(q_lens, kv_lens, hq, hkv, d):
    args = _make(q_lens, kv_lens, hq, hkv, d, pool=max(512, 2 * sum(kv_lens)), seed=sum(kv_lens) + d)
    q, kc, vc, idx, cu_q, cu_k = args
    out, _ = _run(q, kc, vc, idx, cu_q, cu_k, hq, hkv, d)
    np.testing.assert_allclose(to_np64(out), _oracle(q, kc, vc, idx, cu_q, cu_k, d), **BF16_TOL)


@pytest.mark.parametrize("cached_len", [0, 2])
def test_reference_offset_case(cached_len):
    # Structure of tests/test_attention_backend.py:25-53 (seed 17, q_len 3,
    # Hq 4, Hkv 2) at the smallest built head_dim.
    d = 64
    g = torch.Generator().manual_seed(17)
    q_len = 3
    kv_len = cached_len + q_len
    q = torch.randn(q_len, 4, d, generator=g).to(torch.bfloat16)
    k = torch.randn(kv_len, 2, d, generator=g).to(torch.bfloat16)
    v = torch.randn(kv_len, 2, d, generator=g).to(torch.bfloat16)
    idx = torch.arange(kv_len, dtype=torch.int32)
    cu_q = torch.tensor([0, q_len], dtype=torch.int32)
    cu_k = torch.tensor([0, kv_len], dtype=torch.int32)
    out, _ = _run(q, k, v, idx, cu_q, cu_k, 4, 2, d)
    expect = oatt.attention_one(to_np64(q), to_np64(k), to_np64(v), cached_len, d ** -0.5)
    np.testing.assert_allclose(to_np64(out), expect, **BF16_TOL)


def test_first_query_row_sees_only_first_key():
    # Causal closed form: with cached_len 0, query row 0 attends to key 0 only.
    q_lens, kv_lens = [50], [50]
    q, kc, vc, idx, cu_q, cu_k = _make(q_lens, kv_lens, 8, 2, 96, 256, seed=4)
    out, _ = _run(q, kc, vc, idx, cu_q, cu_k, 8, 2, 96)
    v0 = vc[idx[0].long()].float().repeat_interleave(4, dim=0)
    torch.testing.assert_close(out[0].float().cpu(), v0, atol=1e-2, rtol=1e-2)


def test_long_prefill_sampled_rows():
    # 4096-token prefill at Qwen3-4B heads; oracle on sampled query rows.
    hq, hkv, d, n = 32, 8, 128, 4096
    q, kc, vc, idx, cu_q, cu_k = _make([n], [n], hq, hkv, d, pool=65536, seed=4096)
    out, p = _run(q, kc, vc, idx, cu_q, cu_k, hq, hkv, d)
    assert p.num_q_tiles * p.prefill_q_tile >= n
    rows = [0, 1, 31, 32, 33, 127, 1000, 2047, 4095]
    qn, kn, vn = to_np64(q), to_np64(kc[idx.long()]), to_np64(vc[idx.long()])
    got = to_np64(out)
    for i in rows:
        ref = oatt.attention_one(qn[i : i + 1], kn[: i + 1], vn[: i + 1], i, d ** -0.5)
        np.testing.assert_allclose(got[i : i + 1], ref, **BF16_TOL)


@pytest.mark.parametrize("q_lens,kv_lens,hq,hkv,d", [([512], [512], 32, 8, 128),
                                                     ([2, 300], [130, 600], 16, 8, 128),
                                                     ([200], [200], 8, 2, 96)])
def test_growing_logits_move_the_softmax_reference(q_lens, kv_lens, hq, hkv, d):
    # K rows scaled up along each request's positions (x1 to x51): a query
    # row's running max keeps growing over its causal range, so the
    # reference moves mid-stream and rescales O and the MFMA row sums.
    q, kc, vc, idx, cu_q, cu_k = _make(q_lens, kv_lens, hq, hkv, d, 4096, seed=29)
    scale = torch.ones(kc.shape[0])
    for r in range(len(kv_lens)):
        lo, hi = int(cu_k[r]), int(cu_k[r + 1])
        scale[idx[lo:hi].long()] = 1.0 + 50.0 * torch.arange(hi - lo, dtype=torch.float32) / (hi - lo)
    kc = (kc.float() * scale.view(-1, 1, 1)).to(torch.bfloat16)
    out, _ = _run(q, kc, vc, idx, cu_q, cu_k, hq, hkv, d)
    np.testing.assert_allclose(to_np64(out), _oracle(q, kc, vc, idx, cu_q, cu_k, d), **BF16_TOL)
