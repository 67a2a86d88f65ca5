"""TEST INFRASTRUCTURE ONLY: numpy front end of the C oracle (c/tm_oracle.c).

Every function takes and returns numpy arrays on the host.  The library is
built by ``python -m treemoe_spec_amd._build`` (``build_oracle``).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "liboracle_c.so"
_lib = None

TILE_M = 64


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"{_LIB_PATH} missing: run `python -m treemoe_spec_amd._build`")
        lib = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        lib.orc_expf.restype = ctypes.c_float
        lib.orc_expf.argtypes = [ctypes.c_float]
        lib.orc_router_gates.restype = None
        lib.orc_router_gates.argtypes = [P, P, I64, I64, I64, P]
        lib.orc_router_logits.restype = None
        lib.orc_router_logits.argtypes = [P, P, I64, I64, I64, P]
        lib.orc_router_gates_dt.restype = None
        lib.orc_router_gates_dt.argtypes = [P, P, I64, I64, I64, ctypes.c_int, P]
        lib.orc_router_logits_dt.restype = None
        lib.orc_router_logits_dt.argtypes = [P, P, I64, I64, I64, ctypes.c_int, P]
        lib.orc_f32_to_f16.restype = None
        lib.orc_f32_to_f16.argtypes = [P, I64, P]
        lib.orc_route_bucket.restype = ctypes.c_int
        lib.orc_route_bucket.argtypes = [P, P, I64, I64, I64, ctypes.c_float, ctypes.c_int,
                                         I64, I64, I64] + [P] * 10
        lib.orc_argmax.restype = None
        lib.orc_argmax.argtypes = [P, ctypes.c_int, I64, I64, I64, P]
        lib.orc_softmax_argmax.restype = None
        lib.orc_softmax_argmax.argtypes = [P, ctypes.c_int, I64, I64, I64, P]
        lib.orc_greedy_walk.restype = None
        lib.orc_greedy_walk.argtypes = [P, P, P, P, P, I64, I64, P, P, P]
        lib.orc_kv_commit.restype = None
        lib.orc_kv_commit.argtypes = [P, P, I64, I64, I64, I64, I64, I64, I64, P, I64, P, P, I64]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def expf(x: float) -> float:
    return float(_load().orc_expf(ctypes.c_float(x)))


def expf_array(x: np.ndarray) -> np.ndarray:
    lib = _load()
    return np.array([lib.orc_expf(ctypes.c_float(float(v))) for v in x.ravel()],
                    dtype=np.float32).reshape(x.shape)


def router_gates(x_bits: np.ndarray, wg_bits: np.ndarray, f16: bool = False) -> np.ndarray:
    """gates [T, E] fp32 from the 16-bit bit patterns (uint16) of x [T, H] and
    W_g [E, H]: bf16, or fp16 when ``f16``."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(wg_bits, dtype=np.uint16)
    t, h = x.shape
    e = w.shape[0]
    assert w.shape[1] == h and h % 8 == 0 and e <= 64
    out = np.empty((t, e), dtype=np.float32)
    _load().orc_router_gates_dt(_ptr(x), _ptr(w), t, h, e, 1 if f16 else 0, _ptr(out))
    return out


def router_logits(x_bits: np.ndarray, wg_bits: np.ndarray, f16: bool = False) -> np.ndarray:
    """Bits (uint16, bf16 or fp16) of the router logits [T, E] behind router_gates."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(wg_bits, dtype=np.uint16)
    t, h = x.shape
    e = w.shape[0]
    assert w.shape[1] == h and h % 8 == 0
    out = np.empty((t, e), dtype=np.uint16)
    _load().orc_router_logits_dt(_ptr(x), _ptr(w), t, h, e, 1 if f16 else 0, _ptr(out))
    return out


def f32_to_f16_bits(values: np.ndarray) -> np.ndarray:
    """IEEE half bits of fp32 values, round to nearest even (the oracle's
    rounding for fp16 logits and outputs)."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(v.size, dtype=np.uint16)
    _load().orc_f32_to_f16(_ptr(v), v.size, _ptr(out))
    return out.reshape(np.shape(values))


def compact_block_limit(num_slots: int, budget: int, block_m: int) -> int:
    """Restates treemoe/kernels/op1_tree_moe.py:66-71."""
    active = min(num_slots, budget)
    return active + (num_slots - active) // block_m


def compact_block_capacity(num_slots: int, budget: int, block_m: int) -> int:
    """Restates treemoe/kernels/op1_tree_moe.py:74-79."""
    logical = compact_block_limit(num_slots, budget, block_m)
    return 1 << max(logical - 1, 0).bit_length()


@dataclass
class RouteResult:
    topk_ids: np.ndarray         # [2T] int64, slot s = 2t + k
    gates_flat: np.ndarray       # [2T] fp32
    padded_slots: np.ndarray     # [max_blocks * BM] int64
    block_expert_ids: np.ndarray # [max_blocks] int64
    slot_to_row: np.ndarray      # [2T] int64
    demand: np.ndarray           # [E] fp32
    expert_offsets: np.ndarray   # [E+1] int32
    sorted_slots: np.ndarray     # [2T] int32
    slot_pos: np.ndarray         # [2T] int32
    tiles: np.ndarray            # [max_tiles, 4] int32
    max_blocks: int
    max_tiles: int


def route_bucket(gates: np.ndarray, accept: np.ndarray, budget: int, tau: float = 0.05,
                 objective: str = "mass", block_m: int = 16) -> RouteResult:
    g = np.ascontiguousarray(gates, dtype=np.float32)
    a = np.ascontiguousarray(accept, dtype=np.float32)
    t, e = g.shape
    max_blocks = compact_block_capacity(2 * t, budget, block_m)
    max_tiles = compact_block_limit(2 * t, budget, TILE_M)
    res = RouteResult(
        topk_ids=np.empty(2 * t, np.int64), gates_flat=np.empty(2 * t, np.float32),
        padded_slots=np.empty(max_blocks * block_m, np.int64),
        block_expert_ids=np.empty(max_blocks, np.int64), slot_to_row=np.empty(2 * t, np.int64),
        demand=np.empty(e, np.float32), expert_offsets=np.empty(e + 1, np.int32),
        sorted_slots=np.empty(2 * t, np.int32), slot_pos=np.empty(2 * t, np.int32),
        tiles=np.empty((max_tiles, 4), np.int32), max_blocks=max_blocks, max_tiles=max_tiles)
    rc = _load().orc_route_bucket(
        _ptr(g), _ptr(a), t, e, budget, ctypes.c_float(tau),
        1 if objective == "critical_path" else 0, block_m, max_blocks, max_tiles,
        _ptr(res.topk_ids), _ptr(res.gates_flat), _ptr(res.padded_slots),
        _ptr(res.block_expert_ids), _ptr(res.slot_to_row), _ptr(res.demand),
        _ptr(res.expert_offsets), _ptr(res.sorted_slots), _ptr(res.slot_pos), _ptr(res.tiles))
    if rc != 0:
        raise RuntimeError("oracle route_bucket: layout bound exceeded")
    return res


def argmax(logits: np.ndarray, bf16_bits: bool = False) -> np.ndarray:
    """First-occurrence argmax per row; NaN ranks first (numpy.argmax order)."""
    x = np.ascontiguousarray(logits, dtype=np.uint16 if bf16_bits else np.float32)
    n, v = x.shape
    out = np.empty(n, np.int32)
    _load().orc_argmax(_ptr(x), 1 if bf16_bits else 0, n, v, v, _ptr(out))
    return out


def softmax_argmax(logits: np.ndarray, bf16_bits: bool = False) -> np.ndarray:
    """Per row, the first index of the maximum of softmax(row) rounded to the
    row's dtype (fp32, or bf16 when ``bf16_bits``)."""
    x = np.ascontiguousarray(logits, dtype=np.uint16 if bf16_bits else np.float32)
    n, v = x.shape
    out = np.empty(n, np.int32)
    _load().orc_softmax_argmax(_ptr(x), 1 if bf16_bits else 0, n, v, v, _ptr(out))
    return out


def children_csr(children: list[list[int]]):
    counts = np.array([len(c) for c in children], dtype=np.int32)
    starts = np.zeros(len(children), dtype=np.int32)
    if len(children) > 1:
        starts[1:] = np.cumsum(counts)[:-1]
    flat = np.array([c for kids in children for c in kids] or [0], dtype=np.int32)
    return starts, counts, flat


def greedy_walk(argmax_ids: np.ndarray, tokens: np.ndarray, children: list[list[int]],
                max_depth: int):
    """Returns (accepted_slots [N], accepted_tokens [N], bonus, num_accepted, next_root)."""
    am = np.ascontiguousarray(argmax_ids, dtype=np.int32)
    tok = np.ascontiguousarray(tokens, dtype=np.int64)
    n = tok.shape[0]
    starts, counts, flat = children_csr(children)
    slots = np.empty(n, np.int64)
    toks = np.empty(n, np.int64)
    result = np.empty(3, np.int64)
    _load().orc_greedy_walk(_ptr(am), _ptr(tok), _ptr(starts), _ptr(counts), _ptr(flat), n,
                            max_depth, _ptr(slots), _ptr(toks), _ptr(result))
    return slots, toks, int(result[0]), int(result[1]), int(result[2])


def kv_commit(k: np.ndarray, v: np.ndarray, accepted_slots: np.ndarray, num_accepted: int,
              scratch_pages: np.ndarray, block_table: np.ndarray, seq_len: int) -> None:
    """In-place commit on host arrays k, v of shape [L, pages, page_size, kvh, hd]."""
    assert k.flags["C_CONTIGUOUS"] and v.flags["C_CONTIGUOUS"] and k.shape == v.shape
    L, _, page, kvh, hd = k.shape
    es = k.dtype.itemsize
    st = [s // es for s in k.strides]
    sl = np.ascontiguousarray(accepted_slots, dtype=np.int64)
    sp = np.ascontiguousarray(scratch_pages, dtype=np.int32)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    _load().orc_kv_commit(_ptr(k), _ptr(v), es, L, kvh * hd, st[0], st[1], st[2], page,
                          _ptr(sl), num_accepted, _ptr(sp), _ptr(bt), seq_len)
