"""The C-ABI library loads and exports every symbol include/aios_attn.h declares.

CPU-only: no kernel is launched; aios_attn_plan is host-only and is
exercised for its validation and schedule decisions.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from aios_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "aios_attn.h"


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(aios_\w+)\s*\(", text, re.M))


def test_header_and_binding_agree():
    assert _declared_functions() == set(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_symbol():
    lib = _lib.lib()
    for name in _lib.EXPORTED_SYMBOLS:
        assert hasattr(lib, name), name
    assert lib.aios_version().startswith(b"aios-mi355x")


def test_plan_struct_layout_matches_header():
    text = HEADER.read_text()
    body = text[text.index("typedef struct aios_attn_plan {"):text.index("} aios_attn_plan_t;")]
    fields = re.findall(r"^\s*(int32_t|int64_t)\s+(\w+);", body, re.M)
    ctype = {"int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64}
    assert [(n, ctype[t]) for t, n in fields] == list(_lib.AttnPlan._fields_)
    assert ctypes.sizeof(_lib.AttnPlan) == 24 * 4 + 3 * 8


def _plan(phase, cu_q, cu_k, hq=8, hkv=2, d=96, shared=0, ws=1 << 26, chunk=0, split=0):
    cu_q = np.asarray(cu_q, dtype=np.int32)
    cu_k = np.asarray(cu_k, dtype=np.int32)
    p = _lib.AttnPlan()
    rc = _lib.lib().aios_attn_plan(phase, cu_q.ctypes.data, cu_k.ctypes.data, len(cu_q) - 1, hq,
                                   hkv, d, 1, shared, ws, chunk, split, p)
    return rc, p


def test_plan_decode_short_prefix_reads_per_row():
    # Op-test shape: a 24-token prefix is cheaper to read per row in one launch.
    kv = [24 + s for s in (3, 0, 16, 7, 1, 9, 12, 5)]
    rc, p = _plan(_lib.PHASE_DECODE, np.arange(9), np.cumsum([0] + kv), shared=24)
    assert rc == 0
    assert p.prefix_len == 0 and p.num_parts == 1 and p.ws_bytes == 0
    assert p.num_suffix_splits == 1 and p.suffix_split_len >= max(kv)


def test_plan_decode_forced_cascade():
    kv = [24 + s for s in (3, 0, 16, 7, 1, 9, 12, 5)]
    rc, p = _plan(_lib.PHASE_DECODE, np.arange(9), np.cumsum([0] + kv), shared=24, chunk=32)
    assert rc == 0
    assert p.prefix_len == 24 and p.num_prefix_chunks == 1 and p.cascade_rows == 32
    # with the cascade every suffix wavefront writes its own part
    assert p.suffix_parts_per_item == 4
    assert p.num_parts == p.num_prefix_chunks + 4 * p.num_suffix_splits
    assert p.ws_bytes >= 8 * 2 * p.num_parts * 4 * 96 * 2  # bf16 partial outputs


def test_plan_decode_long_context_schedule():
    kv = [4096 + 1 + s for s in range(0, 65, 3)][:24]
    kv += [4096] * (24 - len(kv))
    rc, p = _plan(_lib.PHASE_DECODE, np.arange(25), np.cumsum([0] + kv), hq=32, hkv=8, d=128,
                  shared=4096)
    assert rc == 0
    assert p.prefix_len == 4096 and p.cascade_rows == 96 and p.cascade_mgroups == 1
    assert p.num_prefix_chunks * p.prefix_chunk_len >= 4096
    assert p.num_parts <= 64


def test_plan_decode_long_rows_without_prefix_split():
    rc, p = _plan(_lib.PHASE_DECODE, np.arange(3), np.cumsum([0, 3000, 17]), shared=0)
    assert rc == 0
    assert p.prefix_len == 0 and p.num_suffix_splits > 1 and p.num_parts <= 64
    # no cascade: the item's wavefronts merge, one part per item
    assert p.suffix_parts_per_item == 1 and p.num_parts == p.num_suffix_splits


def test_plan_rejects_bad_batches():
    lib = _lib.lib()
    rc, _ = _plan(_lib.PHASE_DECODE, [0, 2], [0, 5])  # two query tokens in decode
    assert rc == _lib.AIOS_ERR_INVALID
    assert b"one flat token" in lib.aios_last_error()
    rc, _ = _plan(_lib.PHASE_PREFILL, [0, 5], [0, 3])  # kv shorter than q
    assert rc == _lib.AIOS_ERR_INVALID
    rc, _ = _plan(_lib.PHASE_DECODE, [0, 1, 2], [0, 10, 20], shared=11)  # prefix too long
    assert rc == _lib.AIOS_ERR_INVALID
    rc, _ = _plan(_lib.PHASE_DECODE, [0, 1], [0, 5], hq=6, hkv=4)
    assert rc == _lib.AIOS_ERR_INVALID
    assert b"divisible" in lib.aios_last_error()
    rc, _ = _plan(_lib.PHASE_DECODE, [0, 1], [0, 5], d=80)
    assert rc == _lib.AIOS_ERR_UNSUPPORTED


def test_plan_workspace_too_small():
    kv = [4096 + 10] * 24
    rc, p = _plan(_lib.PHASE_DECODE, np.arange(25), np.cumsum([0] + kv), hq=32, hkv=8, d=128,
                  shared=4096, ws=1024, split=8)
    assert rc == _lib.AIOS_ERR_WORKSPACE


def test_plan_prefill_tiles_cover_queries():
    rc, p = _plan(_lib.PHASE_PREFILL, [0, 4096], [0, 4096], hq=32, hkv=8, d=128)
    assert rc == 0
    assert p.num_q_tiles * p.prefill_q_tile >= 4096
    assert p.prefill_q_tile * 4 <= 128


def test_check_maps_status_to_exceptions():
    rc, _ = _plan(_lib.PHASE_DECODE, [0, 2], [0, 5])
    with pytest.raises(ValueError, match="one flat token"):
        _lib.check(rc, "plan")


def test_noalloc_limit_matches_header():
    text = HEADER.read_text()
    m = re.search(r"#define AIOS_DECODE_NOALLOC_MAX_BYTES \((\d+)ll << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.DECODE_NOALLOC_MAX_BYTES


def test_pool_of_2_24_pages_is_rejected():
    """A page's byte offset is a 24-bit multiply in the kernels: a pool of
    2^24 pages (here a 2 GiB cache, inside the 4 GiB offset range) is refused
    before any launch, as is a 4 GiB cache."""
    lib = _lib.lib()
    rc, p = _plan(_lib.PHASE_DECODE, [0, 1], [0, 5], hq=4, hkv=1, d=64)
    assert rc == 0 and p.ws_bytes == 0
    fake = 1 << 20  # 16-byte aligned, never dereferenced: the call is refused first
    for pages, what in (((1 << 24), b"2^24"), ((1 << 32) // 128 + 1, b"2^24")):
        rc = lib.aios_attn_decode(p, fake, 4 * 64, fake, fake, pages, fake, fake, fake, None, 0,
                                  0.125, None)
        assert rc == _lib.AIOS_ERR_UNSUPPORTED
        assert what in lib.aios_last_error()


def test_cg_step_prepare_rejects_bad_arguments():
    """Argument checks run before any device access (fake pointers)."""
    lib = _lib.lib()
    P = 4096  # a 16-byte-aligned stand-in address, never dereferenced
    args = lambda **kw: [kw.get("step", P), P, 4, 8, P, P, kw.get("pt_stride", 256),
                         kw.get("pt_cols", 256), P, P, P, kw.get("max_kv_len", 128), None, P,
                         kw.get("embed", None), kw.get("vocab", 100), kw.get("hidden", 768),
                         kw.get("h_out", P), None]
    rc = lib.aios_cg_step_prepare(*args(max_kv_len=300))
    assert rc == _lib.AIOS_ERR_INVALID and b"max_kv_len" in lib.aios_last_error()
    rc = lib.aios_cg_step_prepare(*args(pt_stride=100))
    assert rc == _lib.AIOS_ERR_INVALID
    rc = lib.aios_cg_step_prepare(*args(step=None))
    assert rc == _lib.AIOS_ERR_INVALID and b"null pointer" in lib.aios_last_error()
    rc = lib.aios_cg_step_prepare(*args(embed=P, hidden=100))
    assert rc == _lib.AIOS_ERR_INVALID and b"multiple of 8" in lib.aios_last_error()
    rc = lib.aios_cg_step_prepare(*args(embed=P + 8))
    assert rc == _lib.AIOS_ERR_INVALID and b"16-byte" in lib.aios_last_error()
    rc = lib.aios_cg_step_prepare(*args(embed=P, h_out=None))
    assert rc == _lib.AIOS_ERR_INVALID
