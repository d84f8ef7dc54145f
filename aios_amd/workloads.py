"""Seeded synthetic CandidateGroup decode workloads (shared by tests and bench).

A workload is one shared prefix of P pages plus N candidate rows, each with
its own ragged suffix of pages, laid out exactly as the CandidateGroup engine
lays them out: every row of the page table starts with the same P physical
pages (python/aios/ime.py:1155) and the suffix pages follow.  Page ids come
from a seeded permutation of the pool, K/V/Q are N(0, 1) * 0.5 in bf16.

Named shapes:
  op_test       1 layer, N=8, P=24, suffix ~ U{0..16}, 8q/2kv, D=96,
                256-page pool (the single-layer op test)
  long_context  36 layers, N=24, P=4096, suffix ~ U{0..64}, 32q/8kv, D=128,
                65,536-page pool (the Qwen3-4B-shaped long-context stress)
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class DecodeShape:
    name: str
    num_layers: int
    num_rows: int
    prefix_len: int
    max_suffix: int
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    num_pages: int
    min_suffix: int = 0

    @property
    def group(self) -> int:
        return self.num_qo_heads // self.num_kv_heads


OP_TEST = DecodeShape("op_test", 1, 8, 24, 16, 8, 2, 96, 256)
LONG_CONTEXT = DecodeShape("long_context", 36, 24, 4096, 64, 32, 8, 128, 65536)
SHAPES = {s.name: s for s in (OP_TEST, LONG_CONTEXT)}


@dataclass
class DecodeWorkload:
    shape: DecodeShape
    seed: int
    q: torch.Tensor            # [L, N, Hq, D] bf16
    k_cache: torch.Tensor      # [L, num_pages, Hkv, D] bf16
    v_cache: torch.Tensor      # [L, num_pages, Hkv, D] bf16
    page_table: torch.Tensor   # [N, P + max_suffix] int32 (unused tail = -1)
    suffix_lens: list[int]
    kv_lens: list[int]
    cu_k: torch.Tensor         # [N+1] int32 (host)
    indices: torch.Tensor      # [sum kv_lens] int32 (host)

    @property
    def prefix_pages(self) -> torch.Tensor:
        return self.page_table[0, : self.shape.prefix_len]


def make_decode_workload(shape: DecodeShape, seed: int = 20260814, device="cpu",
                         extra_token: bool = False, layers: int | None = None) -> DecodeWorkload:
    """Build a seeded workload.

    With ``extra_token`` every row gets one more page after its drawn suffix:
    the page the current decode step appends to (so kv_len = P + s_i + 1).
    ``layers`` overrides the layer count (e.g. 1 for a single-layer check).
    """
    g = torch.Generator().manual_seed(seed)
    n = shape.num_rows
    nl = shape.num_layers if layers is None else layers
    suffix = torch.randint(shape.min_suffix, shape.max_suffix + 1, (n,), generator=g).tolist()
    if extra_token:
        suffix = [s + 1 for s in suffix]
    need = shape.prefix_len + sum(suffix)
    if need > shape.num_pages:
        raise ValueError("pool too small for the workload")
    perm = torch.randperm(shape.num_pages, generator=g).to(torch.int32)
    width = shape.prefix_len + max(suffix + [0])
    table = torch.full((n, max(width, 1)), -1, dtype=torch.int32)
    prefix = perm[: shape.prefix_len]
    table[:, : shape.prefix_len] = prefix
    off = shape.prefix_len
    for i, s in enumerate(suffix):
        table[i, shape.prefix_len : shape.prefix_len + s] = perm[off : off + s]
        off += s
    kv_lens = [shape.prefix_len + s for s in suffix]
    cu_k = torch.zeros(n + 1, dtype=torch.int32)
    cu_k[1:] = torch.tensor(kv_lens, dtype=torch.int32).cumsum(0)
    indices = torch.cat([table[i, : kv_lens[i]] for i in range(n)])

    dev = torch.device(device)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    hkv, d, hq = shape.num_kv_heads, shape.head_dim, shape.num_qo_heads
    kv_shape = (nl, shape.num_pages, hkv, d)
    k_cache = (torch.randn(kv_shape, generator=gd, device=dev, dtype=torch.float32) * 0.5).to(torch.bfloat16)
    v_cache = (torch.randn(kv_shape, generator=gd, device=dev, dtype=torch.float32) * 0.5).to(torch.bfloat16)
    q = (torch.randn((nl, n, hq, d), generator=gd, device=dev, dtype=torch.float32) * 0.5).to(torch.bfloat16)
    return DecodeWorkload(shape, seed, q, k_cache, v_cache, table, suffix, kv_lens, cu_k, indices)


def decode_bytes_per_layer(shape: DecodeShape, suffix_lens: list[int]) -> int:
    """Algorithmic HBM bytes of one layer's decode attention.

    Prefix K+V once, every row's suffix K+V, Q read + O write, and the int32
    page ids of the prefix and the suffixes:
      P*B_kv + sum(s_i)*B_kv + 2*N*Hq*D*2 + 4*(P + sum(s_i)),  B_kv = 2*Hkv*D*2.
    """
    b_kv = 2 * shape.num_kv_heads * shape.head_dim * 2
    s = sum(suffix_lens)
    n = len(suffix_lens)
    return (shape.prefix_len * b_kv + s * b_kv + 2 * n * shape.num_qo_heads * shape.head_dim * 2
            + 4 * (shape.prefix_len + s))


def kv_append_bytes(n_tokens: int, width: int, elem_bytes: int = 2) -> int:
    """K,V read + write plus the int32 page ids: 4*T*W*e + 4*T."""
    return 4 * n_tokens * width * elem_bytes + 4 * n_tokens
