"""Paged KV append (HIP kernel (a)) vs the oracle scatter: bit-exact.

Cases follow the reference's scatter test plan
(resources/lesson-30-triton-kv-store/README.md:433-446): the lesson's known
answer, shuffled indices, non-power-of-two row width 192, a strided v (a view
into the fused qkv projection), multi-layer isolation, plus the config-5
prefill append (4096 tokens x 2 KiB rows) and alignment fallbacks.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_store
from tests.util import bits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _store(k_cache, v_cache, idx, k, v):
    from aios_amd.kernel import store_cache

    store_cache(k_cache, v_cache, idx, k, v)
    torch.cuda.synchronize()


def test_lesson30_known_answer():
    # run_lesson30.py:12-22: indices [17, 4, 9], width 8, rows t*100 + offset.
    width = 8
    idx = torch.tensor([17, 4, 9], dtype=torch.int32, device=DEV)
    vals = torch.tensor([[t * 100 + o for o in range(width)] for t in range(3)], dtype=torch.float32)
    k = vals.to(torch.bfloat16).view(3, 1, width).to(DEV)
    v = (-vals).to(torch.bfloat16).view(3, 1, width).to(DEV)
    kc = torch.full((20, 1, width), -1.0, dtype=torch.bfloat16, device=DEV)
    vc = torch.full((20, 1, width), -1.0, dtype=torch.bfloat16, device=DEV)
    _store(kc, vc, idx, k, v)
    kcf = kc.float().cpu().view(20, width)
    for t, row in enumerate([17, 4, 9]):
        assert kcf[row].tolist() == [t * 100 + o for o in range(width)]
    untouched = [r for r in range(20) if r not in (17, 4, 9)]
    assert (kcf[untouched] == -1).all()
    assert (vc.float().cpu().view(20, width)[[17, 4, 9]] == -vals).all()


@pytest.mark.parametrize("hkv,d,t,pool", [(2, 96, 37, 256), (8, 128, 24, 1024), (2, 64, 1, 16),
                                          (4, 64, 300, 4096)])
def test_random_scatter_bit_exact(hkv, d, t, pool):
    g = torch.Generator().manual_seed(1000 + t)
    idx = torch.randperm(pool, generator=g)[:t].to(torch.int32)
    k = torch.randn(t, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(t, hkv, d, generator=g).to(torch.bfloat16)
    kc = torch.randn(pool, hkv, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(pool, hkv, d, generator=g).to(torch.bfloat16)
    ek, ev = kv_store.store_kv(bits(kc), bits(vc), idx.numpy(), bits(k), bits(v))
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    _store(kc_d, vc_d, idx.to(DEV), k.to(DEV), v.to(DEV))
    np.testing.assert_array_equal(bits(kc_d), ek)
    np.testing.assert_array_equal(bits(vc_d), ev)


def test_strided_v_view_of_qkv():
    # qwen3.py:60-64: v stays a strided view into qkv; k is contiguous after RoPE.
    t, hq, hkv, d, pool = 19, 8, 2, 96, 128
    g = torch.Generator().manual_seed(7)
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(DEV)
    _, k, v = qkv.split([hq * d, hkv * d, hkv * d], dim=-1)
    k = k.reshape(t, hkv, d).contiguous()
    v = v.view(t, hkv, d)
    assert v.stride(0) == (hq + 2 * hkv) * d
    idx = torch.randperm(pool, generator=g)[:t].to(torch.int32)
    kc = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=DEV)
    ek, ev = kv_store.store_kv(bits(kc), bits(vc), idx.numpy(), bits(k), bits(v))
    _store(kc, vc, idx.to(DEV), k, v)
    np.testing.assert_array_equal(bits(kc), ek)
    np.testing.assert_array_equal(bits(vc), ev)


def test_multi_layer_isolation():
    from aios_amd.kvcache import MHAKVCache

    cache = MHAKVCache(num_kv_heads=2, num_layers=3, head_dim=96, num_pages=64, page_size=1,
                       dtype=torch.bfloat16, device=torch.device(DEV))
    cache._kv_buffer.fill_(0.25)
    before = cache._kv_buffer.clone()
    g = torch.Generator().manual_seed(3)
    idx = torch.randperm(64, generator=g)[:10].to(torch.int32).to(DEV)
    k = torch.randn(10, 2, 96, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(10, 2, 96, generator=g).to(torch.bfloat16).to(DEV)
    cache.store_kv(k, v, idx, 1)
    torch.cuda.synchronize()
    for layer in (0, 2):
        assert torch.equal(cache.k_cache(layer), before[0, layer])
        assert torch.equal(cache.v_cache(layer), before[1, layer])
    rows = idx.long().cpu()
    assert torch.equal(cache.k_cache(1)[rows, 0].cpu(), k.cpu())
    assert torch.equal(cache.v_cache(1)[rows, 0].cpu(), v.cpu())
    untouched = torch.ones(64, dtype=torch.bool)
    untouched[rows] = False
    assert torch.equal(cache.k_cache(1)[untouched.to(DEV)], before[0, 1][untouched.to(DEV)])


def test_prefill_sized_append_long_context():
    # 4096 tokens x 8 kv heads x 128 dims: one layer's prefill append of the
    # long-context (4096-token prefix) workload.
    t, hkv, d, pool = 4096, 8, 128, 65536
    g = torch.Generator().manual_seed(11)
    idx = torch.randperm(pool, generator=g)[:t].to(torch.int32)
    k = torch.randn(t, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(t, hkv, d, generator=g).to(torch.bfloat16)
    kc = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=DEV)
    _store(kc, vc, idx.to(DEV), k.to(DEV), v.to(DEV))
    rows = idx.long()
    assert torch.equal(kc.cpu()[rows], k)
    assert torch.equal(vc.cpu()[rows], v)
    mask = torch.ones(pool, dtype=torch.bool)
    mask[rows] = False
    assert int(kc.cpu()[mask].abs().sum()) == 0


def test_out_of_range_indices_are_skipped():
    pool, hkv, d = 32, 2, 64
    idx = torch.tensor([3, -1, 32, 5], dtype=torch.int32, device=DEV)
    k = torch.ones(4, hkv, d, dtype=torch.bfloat16, device=DEV)
    v = torch.ones(4, hkv, d, dtype=torch.bfloat16, device=DEV) * 2
    kc = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=DEV)
    _store(kc, vc, idx, k, v)
    written = kc.abs().sum(dim=(1, 2)).cpu() > 0
    assert written.nonzero().flatten().tolist() == [3, 5]
    assert float(vc[5].float().mean()) == 2.0


@pytest.mark.parametrize("offset_elems,d", [(1, 64), (0, 3), (2, 6)])
def test_unaligned_rows_use_narrow_copies(offset_elems, d):
    t, hkv, pool = 9, 2, 40
    g = torch.Generator().manual_seed(5 + d)
    base = torch.randn(t * hkv * d + offset_elems, generator=g).to(torch.bfloat16).to(DEV)
    k = base[offset_elems:].view(t, hkv, d)
    v = (base[offset_elems:] * 3).view(t, hkv, d)
    idx = torch.randperm(pool, generator=g)[:t].to(torch.int32)
    kc = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=DEV)
    ek, ev = kv_store.store_kv(bits(kc), bits(vc), idx.numpy(), bits(k), bits(v))
    _store(kc, vc, idx.to(DEV), k, v)
    np.testing.assert_array_equal(bits(kc), ek)
    np.testing.assert_array_equal(bits(vc), ev)


def test_empty_batch_is_noop():
    kc = torch.zeros(8, 2, 64, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros(8, 2, 64, dtype=torch.bfloat16, device=DEV)
    e = torch.empty(0, 2, 64, dtype=torch.bfloat16, device=DEV)
    _store(kc, vc, torch.empty(0, dtype=torch.int32, device=DEV), e, e)
    assert int(kc.abs().sum()) == 0


def test_float32_rows_copy_bytes():
    pool, hkv, d, t = 16, 1, 24, 5
    g = torch.Generator().manual_seed(9)
    idx = torch.randperm(pool, generator=g)[:t].to(torch.int32)
    k = torch.randn(t, hkv, d, generator=g)
    v = torch.randn(t, hkv, d, generator=g)
    kc = torch.zeros(pool, hkv, d, device=DEV)
    vc = torch.zeros(pool, hkv, d, device=DEV)
    _store(kc, vc, idx.to(DEV), k.to(DEV), v.to(DEV))
    assert torch.equal(kc.cpu()[idx.long()], k)
    assert torch.equal(vc.cpu()[idx.long()], v)
