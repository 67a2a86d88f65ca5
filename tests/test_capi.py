"""CPU: libtreemoe_amd.so loads, exports every entry point declared in
include/treemoe_amd.h, and rejects bad arguments before touching the GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "treemoe_amd.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(tm_\w+)\s*\(", text, flags=re.M)


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ("tm_version", "tm_status_string", "tm_op1_router_gates", "tm_op1_route_bucket",
              "tm_op1_gemm1", "tm_op1_gemm2", "tm_op1_combine", "tm_op1_prefill_gemm1",
              "tm_op1_prefill_gemm2", "tm_op1_prefill_gemm1_routed", "tm_op4_argmax_walk", "tm_op4_rep_penalty",
              "tm_op4_sample_walk", "tm_op4_kv_commit", "tm_tree_attention",
              "tm_tree_attention_plan", "tm_tree_mask_pack"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from treemoe_spec_amd import _capi

    lib = _capi.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(_capi.SIGNATURES) <= set(declared_functions())
    assert lib.tm_version() == 50000


def test_status_strings():
    from treemoe_spec_amd import _capi

    lib = _capi.lib()
    assert lib.tm_status_string(0) == b"ok"
    for code in (1001, 1002, 1003):
        assert lib.tm_status_string(code) not in (b"ok", b"unknown status")


def _attn_args(**kw):
    """tm_tree_attention arguments at the config-4 shape (null pointers)."""
    a = dict(q=0, q_stride=4096, k_tail=0, v_tail=0, tail_stride=1024, k_cache=0, v_cache=0,
             stride_page=16 * 1024, stride_slot=1024, page_size=16, block_table=0,
             num_table_pages=256, seq_len=4096, scratch_pages=0, num_scratch_pages=4,
             write_tree=1, mask_bits=0, N=64, Hq=32, kvh=8, hd=128, scale=0.088, out=0,
             out_stride=4096, chunk_keys=0, workspace=0, workspace_bytes=0, stream=0)
    a.update(kw)
    return ("tm_tree_attention", *a.values())


@pytest.mark.parametrize("call,expect", [
    (_attn_args(), 1001),                                  # workspace too small
    (_attn_args(hd=64, workspace_bytes=1 << 30), 1001),
    (_attn_args(N=0, workspace_bytes=1 << 30), 1001),
    (_attn_args(N=257, workspace_bytes=1 << 30), 1001),
    (_attn_args(page_size=24, workspace_bytes=1 << 30), 1001),
    (_attn_args(Hq=12, workspace_bytes=1 << 30), 1001),    # Hq % kvh
    (_attn_args(num_table_pages=255, workspace_bytes=1 << 30), 1001),
    (_attn_args(num_scratch_pages=3, workspace_bytes=1 << 30), 1001),
    (_attn_args(q=8, workspace_bytes=1 << 30), 1002),
    (_attn_args(stride_slot=1028, stride_page=16 * 1028, workspace_bytes=1 << 30), 1002),
    (_attn_args(scale=0.0, workspace_bytes=1 << 30), 1003),
    (_attn_args(chunk_keys=-1, workspace_bytes=1 << 30), 1003),
    (("tm_tree_mask_pack", 0, 0, 1, 0, 0), 1001),
    (("tm_tree_mask_pack", 0, 4, 4, 4, 0), 1002),
])
def test_tree_attention_argument_errors(call, expect):
    from treemoe_spec_amd import _capi

    name, *args = call
    assert getattr(_capi.lib(), name)(*args) == expect


def test_tree_attention_plan():
    import ctypes

    from treemoe_spec_amd import _capi

    chunks, ws = ctypes.c_int64(), ctypes.c_int64()
    plan = _capi.lib().tm_tree_attention_plan
    assert plan(64, 32, 8, 128, 0, 16, 0, ctypes.byref(chunks), ctypes.byref(ws)) == 0
    assert chunks.value == 1 and ws.value == 0
    assert plan(64, 32, 8, 128, 4096, 16, 64, ctypes.byref(chunks), ctypes.byref(ws)) == 0
    # 65 chunks x 8 heads x 2 row blocks (128 rows each) x 4 waves x
    # (32 queries x 128 fp16 partials + 32 x (m, l) fp32)
    assert chunks.value == 65 and ws.value == 65 * 8 * 2 * 4 * (32 * 128 * 2 + 32 * 2 * 4)
    assert plan(64, 32, 8, 128, 4096, 16, 0, ctypes.byref(chunks), ctypes.byref(ws)) == 0
    assert 8 * 2 * chunks.value >= 200   # automatic chunks spread over the 256 CUs
    # prefix and tree keys chunk separately: 4096 = 12 x 320 + 256 prefix
    # keys, then the tree keys (64 or 256) in one chunk of their own; a
    # 300-key prefix at 64 keys per chunk takes 5 chunks, the tree one more
    assert plan(64, 32, 8, 128, 4096, 16, 320, ctypes.byref(chunks), ctypes.byref(ws)) == 0
    assert chunks.value == 13 + 1
    assert plan(256, 8, 8, 128, 4096, 16, 320, ctypes.byref(chunks), ctypes.byref(ws)) == 0
    assert chunks.value == 13 + 1
    assert plan(64, 32, 8, 128, 300, 16, 64, ctypes.byref(chunks), ctypes.byref(ws)) == 0
    assert chunks.value == 5 + 1
    # work that fits one chunk stays one chunk (no combine)
    assert plan(64, 32, 8, 128, 100, 16, 256, ctypes.byref(chunks), ctypes.byref(ws)) == 0
    assert chunks.value == 1 and ws.value == 0
    # no prefix: tree keys only, in chunks of 64
    assert plan(130, 8, 2, 128, 0, 16, 64, ctypes.byref(chunks), ctypes.byref(ws)) == 0
    assert chunks.value == 3
    assert plan(64, 32, 8, 64, 4096, 16, 0, ctypes.byref(chunks), ctypes.byref(ws)) == 1001


def _routed_args(**kw):
    """tm_op1_prefill_gemm1_routed arguments at the config-2 shape; every
    pointer is null except where a case sets one, so only the cases that
    fail a check may be called (the first, valid case is not called)."""
    a = dict(x=0, w1=0, w3=0, h=0, gates=0, accept=0, T=64, H=4096, I=14336, E=8, budget=8,
             tau=0.05, objective=0, block_m=16, max_blocks=16, max_tiles=9, topk=0, gflat=0,
             padded=0, blk=0, s2r=0, demand=0, offsets=0, sorted=0, slot_pos=0, tiles=0,
             dtype=1, stream=0)
    a.update(kw)
    return ("tm_op1_prefill_gemm1_routed", *a.values())


@pytest.mark.parametrize("call,expect", [
    (("tm_op1_router_gates", 0, 0, 0, 4096, 8, 0, 1, 0), 1001),          # T = 0
    (("tm_op1_router_gates", 0, 0, 4, 4095, 8, 0, 1, 0), 1001),          # H % 8
    (("tm_op1_router_gates", 0, 0, 4, 4096, 65, 0, 1, 0), 1001),         # E > 64
    (("tm_op1_router_gates", 8, 0, 4, 4096, 8, 0, 1, 0), 1002),          # unaligned x
    (("tm_op1_router_gates", 0, 0, 4, 4096, 8, 0, 0, 0), 1003),          # fp32 is no op1 dtype
    (("tm_op1_combine", 0, 0, 0, 64, 4096, 2, 3, 0), 1003),                # unknown dtype
    (("tm_op1_gemm1", 0, 0, 0, 0, 0, 0, 1, 64, 4000, 14336, 8, 1, 0), 1001),  # H % 256
    (("tm_op1_gemm2", 0, 0, 0, 0, 0, 0, 1, 3, 64, 4096, 14336, 8, 1, 0), 1001),  # split
    (("tm_op1_combine", 0, 0, 0, 64, 4094, 2, 1, 0), 1001),
    (("tm_op1_prefill_gemm1", 0, 0, 0, 0, 0, 0, 0, 9, 2048, 4000, 14336, 8, 1, 0), 1001),  # H % 64
    (("tm_op1_prefill_gemm1", 0, 0, 0, 0, 0, 0, 0, 0, 2048, 4096, 14336, 8, 1, 0), 1001),  # tiles
    (("tm_op1_prefill_gemm1", 8, 0, 0, 0, 0, 0, 0, 9, 2048, 4096, 14336, 8, 1, 0), 1002),  # align
    (("tm_op1_prefill_gemm2", 0, 0, 0, 0, 0, 0, 0, 9, 2, 2048, 4032, 14336, 8, 1, 0), 1001),  # H % 256
    (("tm_op1_prefill_gemm1", 0, 0, 0, 0, 0, 0, 0, 9, 2048, 4096, 14272, 8, 1, 0), 1001),  # I % 128
    (("tm_op1_prefill_gemm2", 0, 0, 0, 0, 0, 0, 0, 9, 3, 2048, 4096, 14336, 8, 1, 0), 1001),  # split
    (_routed_args(), 0),                                                  # all valid
    (_routed_args(T=65), 1001),                                           # T > 64
    (_routed_args(E=17, budget=8), 1001),                                 # E > 16
    (_routed_args(T=0), 1001),
    (_routed_args(max_blocks=257), 1001),
    (_routed_args(max_tiles=0), 1001),
    (_routed_args(budget=1), 1003),
    (_routed_args(budget=9), 1003),
    (_routed_args(block_m=24), 1003),
    (_routed_args(objective=2), 1003),
    (_routed_args(dtype=0), 1003),
    (_routed_args(H=4000), 1001),                                         # H % 64
    (_routed_args(I=14272), 1001),                                        # I % 128
    (_routed_args(x=8), 1002),                                            # unaligned x
    (_routed_args(h=8), 1002),
    (("tm_op4_argmax_walk", 0, 7, 4, 10, 10, 0, 0, 0, 0, 3, 1, 0, 0, 0, 0, 0, 0, 0), 1003),
    (("tm_op4_argmax_walk", 0, 0, 4, 10, 9, 0, 0, 0, 0, 3, 1, 0, 0, 0, 0, 0, 0, 0), 1001),
    (("tm_op4_argmax_walk", 0, 0, 4, 10, 10, 0, 0, 0, 0, -1, 1, 0, 0, 0, 0, 0, 0, 0), 1001),
    (("tm_op4_argmax_walk", 0, 0, 4, 10, 10, 0, 0, 0, 0, 3, 1, 2, 0, 0, 0, 0, 0, 0), 1003),
    (("tm_op4_rep_penalty", 0, 0, 4, 10, 10, 0, 0, 1.5, 0, 16, 0), 1001),     # no tokens
    (("tm_op4_rep_penalty", 0, 0, 4, 10, 10, 0, 4, 1.5, 0, 12, 0), 1001),     # table size
    (("tm_op4_rep_penalty", 0, 0, 4, 10, 10, 0, 4, 1.5, 0, 4, 0), 1001),      # table < 2n
    (("tm_op4_rep_penalty", 0, 0, 4, 10, 10, 0, 4, 0.0, 0, 16, 0), 1003),     # penalty
    (("tm_op4_rep_penalty", 0, 5, 4, 10, 10, 0, 4, 1.5, 0, 16, 0), 1003),     # dtype
    (("tm_op4_rep_penalty", 0, 0, 4, 10, 10, 0, 1, 1.5, 0, 2, 0), 1001),      # table < 4
    (("tm_op4_rep_penalty", 0, 0, 4, 10, 10, 0, 4, 1.5, 8, 16, 0), 1002),     # table align
    (("tm_op4_sample_walk", 0, 0, 4, (1 << 25) + 1, 1 << 26, 0, 1 << 26, 0, 0, 0, 0, 3, 0, 0,
      1.0, 0, 0, 0, 0, 0), 1001),                                               # V > 2^25
    (("tm_op4_sample_walk", 0, 0, 4, 10, 10, 0, 10, 0, 0, 0, 0, 3, 0, 0, 0.0, 0, 0, 0, 0, 0),
     1003),                                                                     # temperature
    (("tm_op4_sample_walk", 0, 0, 4, 10, 10, 0, 9, 0, 0, 0, 0, 3, 0, 0, 1.0, 0, 0, 0, 0, 0),
     1001),                                                                     # q stride
    (("tm_op4_sample_walk", 0, 0, 4, 10, 10, 0, 10, 0, 0, 0, 0, -1, 0, 0, 1.0, 0, 0, 0, 0, 0),
     1001),                                                                     # num_edges
])
def test_argument_errors_return_before_launch(call, expect):
    from treemoe_spec_amd import _capi

    name, *args = call
    assert len(args) == len(_capi.SIGNATURES[name]), "argument count"
    if expect == 0:
        return  # the valid reference case: only its argument count is checked
    fn = getattr(_capi.lib(), name)
    assert fn(*args) == expect


def test_fused_route_argument_errors():
    from treemoe_spec_amd import _capi

    fn = _capi.lib().tm_op1_route
    # x = 8 is misaligned, so every case below fails a check before any launch
    base = [8, 0, 0, 64, 4096, 8, 4, ctypes.c_float(0.05), 0, 16, 16, 11] + [0] * 11 + [1, 0]
    assert fn(*base) == 1002
    args = list(base)
    args[-2] = 0
    assert fn(*args) == 1003                 # fp32 is no op1 dtype
    args = list(base)
    args[4] = 4095
    assert fn(*args) == 1001                 # H % 8
    args = list(base)
    args[6] = 1
    assert fn(*args) == 1003                 # budget < 2


def test_route_bucket_argument_errors():
    from treemoe_spec_amd import _capi

    fn = _capi.lib().tm_op1_route_bucket
    base = [0, 0, 64, 8, 4, ctypes.c_float(0.05), 0, 16, 16, 11] + [0] * 11
    args = list(base)
    args[4] = 9          # budget > E
    assert fn(*args) == 1003
    args = list(base)
    args[6] = 5          # objective
    assert fn(*args) == 1003
    args = list(base)
    args[7] = 8          # block_m
    assert fn(*args) == 1003
    args = list(base)
    args[8] = 4096       # padded rows beyond the workgroup's table
    assert fn(*args) == 1001


def test_cpython_binding_loads_and_checks_arguments():
    """The CPython binding of the per-step op4 calls is built and rejects a
    wrong argument count before calling into the library."""
    import pytest

    from treemoe_spec_amd import _tmfast

    for name in ("argmax_walk", "kv_commit"):
        with pytest.raises(TypeError):
            getattr(_tmfast, name)(1, 2, 3)
