"""Decoder-layer kernels (aios_rmsnorm, aios_qk_norm_rope, aios_silu_mul) vs
the torch formulas of the reference layers on the same bf16 inputs."""
from __future__ import annotations

import pytest
import torch

from aios_amd.layers import HipOps
from aios_amd.qwen3 import RotaryEmbedding
from tests.util import TorchOps

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(torch.bfloat16)


def _ulp_close(a, b, ulps=1):
    """bf16 results within `ulps` units in the last place (relative 2^-7 per ulp)."""
    a, b = a.float(), b.float()
    tol = ulps * 2.0 ** -7 * torch.maximum(a.abs(), b.abs()) + 1e-6
    assert bool(((a - b).abs() <= tol).all()), (a - b).abs().max().item()


@pytest.mark.parametrize("rows,hidden", [(1, 768), (8, 768), (37, 1024), (5, 2560), (3, 8192)])
def test_rmsnorm_and_fused_add(rows, hidden):
    x = _bf16((rows, hidden), rows, 2.0)
    r = _bf16((rows, hidden), rows + 1, 3.0)
    w = _bf16((hidden,), 7).abs() + 0.5
    ops, ref = HipOps(), TorchOps()
    _ulp_close(ops.rmsnorm(x, w, 1e-5), ref.rmsnorm(x, w, 1e-5))
    x1, r1 = x.clone(), r.clone()
    x2, r2 = x.clone(), r.clone()
    ops.fused_add_rmsnorm(x1, r1, w, 1e-6)
    ref.fused_add_rmsnorm(x2, r2, w, 1e-6)
    assert torch.equal(r1, r2)  # the residual sum is rounded once, as in the reference
    _ulp_close(x1, x2)


def test_rmsnorm_rejects_unsupported_width():
    with pytest.raises(ValueError, match="multiple of 8"):
        HipOps().rmsnorm(_bf16((2, 100), 1), _bf16((100,), 2), 1e-6)


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 96), (12, 4, 64), (16, 8, 128), (32, 8, 128)])
def test_qk_norm_rope(hq, hkv, d):
    t = 19
    qkv = _bf16((t, (hq + 2 * hkv) * d), d + hq, 1.5)
    qw = _bf16((d,), 3).abs() + 0.5
    kw = _bf16((d,), 4).abs() + 0.5
    rot = RotaryEmbedding(d, 512, 1000000.0, DEV)
    pos = torch.tensor([0, 1, 2, 5, 31, 32, 100, 511] + list(range(200, 211)), dtype=torch.int32,
                       device=DEV)
    q1, k1 = HipOps().qk_norm_rope(qkv, qw, kw, rot.cos, rot.sin, pos, hq, hkv, d, 1e-6)
    q2, k2 = TorchOps().qk_norm_rope(qkv, qw, kw, rot.cos, rot.sin, pos, hq, hkv, d, 1e-6)
    # Same roundings as the torch ops; the norm's fp32 sum may differ in the
    # last bit, which can move an output by one bf16 step.
    _ulp_close(q1, q2, ulps=2)
    _ulp_close(k1, k2, ulps=2)
    # position 0 is the identity rotation: the output is the normalised head
    xn = TorchOps()._norm(qkv[:1, : hq * d].reshape(1, hq, d), qw, 1e-6)
    _ulp_close(q1[:1], xn)


@pytest.mark.parametrize("rows,inter", [(8, 2048), (32, 3072), (3, 9728)])
def test_silu_and_mul(rows, inter):
    x = _bf16((rows, 2 * inter), inter, 2.0)
    _ulp_close(HipOps().silu_and_mul(x), TorchOps().silu_and_mul(x))


@pytest.mark.parametrize("m,n,k", [(1, 1152, 768), (8, 1152, 768), (8, 768, 768), (8, 4096, 768),
                                   (8, 768, 2048), (8, 6400, 768), (24, 1024, 4096),
                                   (17, 2048, 1024), (64, 256, 9728), (33, 16, 128),
                                   # many column tiles: the streaming kernel (even and
                                   # uneven tiles per workgroup)
                                   (8, 16384, 768), (5, 20016, 768), (16, 32768, 1024),
                                   (8, 151936, 1024),
                                   # K 2048 plain (the down projection): 8-column tiles
                                   (1, 16, 2048), (16, 1024, 2048),
                                   # K 3072 plain (fixed step count)
                                   (8, 1024, 3072), (3, 2560, 3072)])
def test_linear_rows_matches_fp32_gemm(m, n, k):
    """Few-row GEMM kernel vs an fp32 matmul of the same bf16 operands: fp32
    accumulation, one bf16 rounding at the end."""
    x = _bf16((m, k), m + k, 1.0)
    w = _bf16((n, k), n, 0.05)
    y = HipOps().linear(x, w)
    ref = (x.float() @ w.float().T)
    err = (y.float() - ref).abs()
    assert bool((err <= 2.0 ** -8 * ref.abs() + 1e-3 * ref.abs().max()).all()), err.max().item()


def test_linear_rows_strided_input_and_fallback():
    x_big = _bf16((8, 2048), 5)
    x = x_big[:, :768]  # row stride 2048
    w = _bf16((1152, 768), 6, 0.05)
    torch.testing.assert_close(HipOps().linear(x, w).float(), (x.float() @ w.float().T),
                               atol=2e-2, rtol=1e-2)
    x65 = _bf16((65, 768), 7)  # more rows than the kernel takes: library GEMM
    torch.testing.assert_close(HipOps().linear(x65, w).float(), (x65.float() @ w.float().T),
                               atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("rows,k,n", [(1, 768, 1152), (8, 768, 1152), (8, 768, 6400),
                                      (24, 1024, 512), (40, 512, 256), (8, 2048, 768),
                                      (24, 768, 1152), (17, 768, 1152),
                                      # the streaming kernel (LM-head shapes)
                                      (8, 768, 16384), (1, 768, 20016), (8, 1024, 151936),
                                      (24, 1024, 151936)])
@pytest.mark.parametrize("with_residual", [True, False])
def test_add_rmsnorm_linear(rows, k, n, with_residual):
    """RMSNorm (with the residual add) folded into the projection: the same
    normalised operand as the separate kernels, the residual sum bit-exact;
    more rows than one launch holds (17, 24 at K 768 / 1024; 40 at K 512)
    run as row chunks."""
    h = _bf16((rows, k), rows + k, 2.0)
    r = _bf16((rows, k), rows + k + 1, 3.0) if with_residual else None
    nw = _bf16((k,), 9).abs() + 0.5
    w = _bf16((n, k), n, 0.05)
    y, new_r = HipOps().add_rmsnorm_linear(h, r, nw, 1e-6, w)
    ref = TorchOps()
    if with_residual:
        x_ref, r_ref = ref.fused_add_rmsnorm(h.clone(), r.clone(), nw, 1e-6)
        assert torch.equal(new_r, r_ref)
    else:
        x_ref = ref.rmsnorm(h, nw, 1e-6)
        assert new_r is h
    y_ref = x_ref.float() @ w.float().T
    err = (y.float() - y_ref).abs()
    assert bool((err <= 2.0 ** -7 * y_ref.abs() + 2e-3 * y_ref.abs().max()).all()), err.max().item()


@pytest.mark.parametrize("rows,k,inter", [(8, 768, 2048), (3, 512, 256), (33, 256, 512),
                                          (1, 1024, 3072), (24, 768, 2048), (24, 1024, 3072)])
@pytest.mark.parametrize("with_residual", [True, False])
def test_add_rmsnorm_linear_silu_pair(rows, k, inter, with_residual):
    """Norm folded in front of the merged gate/up projection and SiLU-and-mul
    behind it: matches norm -> GEMM (bf16 store) -> silu_and_mul."""
    h = _bf16((rows, k), rows + k, 2.0)
    r = _bf16((rows, k), rows + k + 1, 3.0) if with_residual else None
    nw = _bf16((k,), 9).abs() + 0.5
    w = _bf16((2 * inter, k), inter, 0.05)
    y, _ = HipOps().add_rmsnorm_linear(h, r, nw, 1e-6, w, silu=True)
    ref = TorchOps()
    x_ref = (ref.fused_add_rmsnorm(h.clone(), r.clone(), nw, 1e-6)[0] if with_residual
             else ref.rmsnorm(h, nw, 1e-6))
    gu = (x_ref.float() @ w.float().T).to(torch.bfloat16)
    y_ref = ref.silu_and_mul(gu).float()
    err = (y.float() - y_ref).abs()
    assert bool((err <= 2.0 ** -6 * y_ref.abs() + 4e-3 * y_ref.abs().max()).all()), err.max().item()
