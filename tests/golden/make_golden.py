"""Writes the golden fixtures under tests/golden/.

Run from the repository root:  python tests/golden/make_golden.py

Every fixture is data: seeded inputs and the float64 oracle's outputs.  No
file of the reference is imported or run; the known answers the reference's
own resources hold are literal data in tests/test_oracle.py.

  op_test_decode.npz   the single-layer shared-prefix decode op test
                       (N=8 candidates, prefix 24, suffixes U{0..16},
                       8q/2kv heads, D=96, 256-page pool, seed 20260814):
                       bf16 inputs as uint16 bit patterns, page ids, cu_k and
                       the float64 attention output [8, 8, 96].
  offset_causal.npz    the seed-17 offset-causal GQA case (q_len 3,
                       cached_len 0 and 2, 4q/2kv heads, D=8) in float32
                       inputs with the float64 oracle output.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from aios_amd.workloads import OP_TEST, make_decode_workload  # noqa: E402
from oracle import attention as oatt  # noqa: E402

SEED = 20260814


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def op_test() -> None:
    wl = make_decode_workload(OP_TEST, seed=SEED)
    q = wl.q[0].to(torch.float64).numpy()
    kc = wl.k_cache[0].to(torch.float64).numpy()
    vc = wl.v_cache[0].to(torch.float64).numpy()
    out = oatt.decode_attention(q, kc, vc, wl.indices.numpy(), wl.cu_k.numpy(),
                                OP_TEST.head_dim ** -0.5)
    np.savez_compressed(os.path.join(HERE, "op_test_decode.npz"),
                        seed=np.int64(SEED), q_bits=_bits(wl.q[0]),
                        k_bits=_bits(wl.k_cache[0]), v_bits=_bits(wl.v_cache[0]),
                        indices=wl.indices.numpy(), cu_k=wl.cu_k.numpy(),
                        suffix_lens=np.asarray(wl.suffix_lens, dtype=np.int32),
                        out=out)


def offset_causal() -> None:
    arrays = {}
    for cached in (0, 2):
        g = torch.Generator().manual_seed(17)
        lq, lk = 3, cached + 3
        q = torch.randn(lq, 4, 8, generator=g)
        k = torch.randn(lk, 2, 8, generator=g)
        v = torch.randn(lk, 2, 8, generator=g)
        out = oatt.attention_one(q.numpy(), k.numpy(), v.numpy(), cached, 8 ** -0.5)
        arrays.update({f"q{cached}": q.numpy(), f"k{cached}": k.numpy(),
                       f"v{cached}": v.numpy(), f"out{cached}": out})
    np.savez_compressed(os.path.join(HERE, "offset_causal.npz"), **arrays)


if __name__ == "__main__":
    op_test()
    offset_causal()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
