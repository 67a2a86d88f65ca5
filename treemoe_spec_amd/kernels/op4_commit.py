"""op4: fused greedy tree verify + paged KV commit on MI355X.

Same call signature as the reference ``fused_verify_commit``
(treemoe/kernels/op4_commit.py:170-272).  Two launches:

  tm_op4_argmax_walk   first-occurrence argmax of every node's logits (row
                       ranges over many workgroups), then in one workgroup the
                       greedy accept walk and the -1-padded result vectors
                       (int64, on device);
  tm_op4_kv_commit     copy of the K/V rows of [root] + accepted path from the
                       tree scratch pages to positions seq_len, seq_len+1, ...

``kv.seq_len`` advances by num_accepted + 1, which reads num_accepted back to
the host exactly like the reference (:267).

Greedy with rep_penalty != 1 (reference :201-214) first penalises the logits
in place (``tm_op4_rep_penalty``; without prev_tokens token 0 is penalised, as
in the reference), then, as the reference does, takes the first-occurrence
argmax of their softmax rounded to the logits' dtype (equal rounded
probabilities tie and the lower index wins).

Sampling (temperature > 0) follows the reference's routing of that mode to
``tree_verify_ref`` (:187-196): the walk is unbounded (max_depth and
rep_penalty are not used), the accept draws are ``torch.rand(N, generator)``
on the logits' device as in the reference, and the bonus token is the
reference's ``torch.multinomial(residual, 1, generator)`` draw: PyTorch
samples one index as the argmax of residual / e over
e = empty_like(residual).exponential_(1, generator), so the host draws that e
from the same generator and the kernel runs the race.  One launch,
``tm_op4_sample_walk``; no host synchronisation (the reference's multinomial
checks its input on the host twice).
"""

from __future__ import annotations

import ctypes
import threading
import time
from dataclasses import dataclass

import torch

from treemoe_spec_amd import _capi
from treemoe_spec_amd._capi import TM_DTYPE_BF16, TM_DTYPE_F32, call, check, ptr
from treemoe_spec_amd.kv_cache import device_tables_of, scratch_pages_of

# The per-step greedy path calls the C ABI through the CPython binding when it
# is built (one Python-to-C transition per entry point instead of ctypes'
# per-argument conversions); the ctypes binding serves every other call.
try:
    from treemoe_spec_amd import _tmfast as _fast
except ImportError:  # not built: the ctypes binding is used
    _fast = None


@dataclass
class VerifyResult:
    """Reference: treemoe/ref/verify_ref.py:20-25."""

    accepted_slots: torch.Tensor   # [N] tree-node indices, -1 padded
    accepted_tokens: torch.Tensor  # [N] token ids, -1 padded
    bonus_token: torch.Tensor      # [] token after the last accepted node
    num_accepted: torch.Tensor     # [] number of accepted nodes


def argmax_workspace(n: int, device) -> torch.Tensor:
    """Scratch of the row-range argmax: N * TM_OP4_MAX_PARTS (value, index) pairs."""
    return torch.empty(n * _capi.TM_OP4_MAX_PARTS * 8, dtype=torch.uint8, device=device)


class _Scratch:
    """Internal buffers of the greedy path for one (N, device, stream, host
    thread): the argmax row partials, the int32 argmax vector, and the pinned
    host word the KV commit writes num_accepted into (created on first use).
    Calls on one stream reuse them in stream order.  A call on another stream
    gets its own: a call with kv=None returns while its kernels are still
    queued, so a second stream would otherwise overwrite its partials.  A
    call from another host thread gets its own too, so that each thread
    reads the count word of its own commit."""

    __slots__ = ("partials", "argmax", "partials_ptr", "argmax_ptr", "note", "note_np",
                 "note_dev")

    def __init__(self, n: int, device):
        self.partials = argmax_workspace(n, device)
        self.argmax = torch.empty(n, dtype=torch.int32, device=device)
        self.partials_ptr = self.partials.data_ptr()
        self.argmax_ptr = self.argmax.data_ptr()
        self.note = None

    def host_count(self) -> int:
        """Device address of the pinned count word (0 if unavailable)."""
        if self.note is None:
            self.note = torch.full((1,), -1, dtype=torch.int64, pin_memory=True)
            self.note_np = self.note.numpy()
            addr = ctypes.c_void_p()
            rc = _capi.lib().tm_host_device_pointer(ctypes.c_void_p(self.note.data_ptr()),
                                                    ctypes.byref(addr))
            self.note_dev = addr.value if rc == 0 and addr.value else 0
        return self.note_dev


# How long the host spins on the pinned count word before it falls back to a
# stream synchronisation (queued work ahead of op4 can delay the word).
_NOTE_SPIN_S = 2e-3


def _read_count(ws: _Scratch, result: torch.Tensor) -> int:
    """num_accepted as written by the KV commit into the pinned word; after
    _NOTE_SPIN_S, or when no word was passed, a synchronising read of
    result[1] (what the reference does, op4_commit.py:267)."""
    if ws.note_dev:
        note = ws.note_np
        deadline = time.perf_counter() + _NOTE_SPIN_S
        while True:
            for _ in range(256):
                v = int(note[0])
                if v >= 0:
                    return v
            if time.perf_counter() > deadline:
                break
        torch.cuda.current_stream(result.device).synchronize()
        v = int(note[0])
        if v >= 0:
            return v
    return int(result[1])


_scratch_cache: dict[tuple, _Scratch] = {}


def _scratch_key(n: int, device: int, stream: int) -> tuple:
    return (n, device, stream, threading.get_ident())


def _scratch(n: int, device: int, stream: int) -> _Scratch:
    """The buffers of (N, device index, raw stream handle, calling thread),
    allocated on first use while that stream is current, so that torch's
    allocator orders their reuse on it."""
    key = _scratch_key(n, device, stream)
    ws = _scratch_cache.get(key)
    if ws is None:
        if len(_scratch_cache) > 16:
            _scratch_cache.clear()
        ws = _scratch_cache[key] = _Scratch(n, device)
    return ws


def _penalty_table_size(num_prev: int) -> int:
    return 1 << max(4, (2 * num_prev - 1).bit_length())


def _apply_rep_penalty(logits: torch.Tensor, dtype: int, prev_tokens, rep_penalty: float,
                       stream: int) -> None:
    n, v = logits.shape
    dev = logits.device
    if prev_tokens is None:
        prev = torch.zeros(1, dtype=torch.int64, device=dev)  # reference :209
    else:
        prev = prev_tokens.to(device=dev, dtype=torch.int64).reshape(-1).contiguous()
        if prev.numel() == 0:
            return
        # tokens outside [0, vocab) are skipped by the kernel (the reference
        # would index past the row)
    size = _penalty_table_size(prev.numel())
    table = torch.empty(2 * size, dtype=torch.int32, device=dev)
    call("tm_op4_rep_penalty", ptr(logits), dtype, n, v, logits.stride(0), ptr(prev),
         prev.numel(), float(rep_penalty), ptr(table), size, stream)


def _pack_children(children: list[list[int]], n: int) -> tuple[list[int], int]:
    """[starts | counts | flat] as one int32 list, and the number of edges."""
    if len(children) != n:
        raise ValueError(f"children must list {n} nodes, got {len(children)}")
    starts, counts, flat = [], [], []
    for kids in children:
        starts.append(len(flat))
        counts.append(len(kids))
        flat.extend(kids)
    if flat and (min(flat) < 0 or max(flat) >= n):
        raise ValueError("child index out of range")
    return starts + counts + (flat or [0]), len(flat)


def _children_csr(children: list[list[int]], n: int, device) -> tuple[torch.Tensor, int]:
    """[starts | counts | flat] int32 on ``device`` and the edge count (the
    length of ``flat``; trees padded with edge-free slots have fewer than
    N - 1).  One host->device copy from pinned memory, ordered on the current
    stream (no host synchronisation)."""
    packed, num_edges = _pack_children(children, n)
    if torch.device(device).type != "cuda":
        return torch.tensor(packed, dtype=torch.int32), num_edges
    host = torch.tensor(packed, dtype=torch.int32, pin_memory=True)
    return host.to(device, non_blocking=True), num_edges


# The child CSR is static metadata per tree shape (the reference flattens it
# "once per tree shape", op4_commit.py:216): the device copy is kept per
# (children list object, device) and reused while the list's contents are
# unchanged, which one C-level list comparison checks.
_csr_cache: dict[tuple, tuple[list, torch.Tensor, int]] = {}


def _cached_csr(children: list[list[int]], n: int, device) -> tuple[torch.Tensor, int]:
    if len(children) != n:
        raise ValueError(f"children must list {n} nodes, got {len(children)}")
    key = (id(children), n, device)
    hit = _csr_cache.get(key)
    if hit is not None and hit[0] == children:
        return hit[1], hit[2]
    csr, num_edges = _children_csr(children, n, device)
    if len(_csr_cache) > 64:
        _csr_cache.clear()
    _csr_cache[key] = ([list(k) for k in children], csr, num_edges)
    return csr, num_edges


def _commit(kv, p_slots: int, p_result: int, n: int, commit_depth: int, dev, stream: int,
            host_count: int = 0) -> None:
    """Copy the KV rows of [root] + accepted path from the tree scratch to
    positions seq_len, seq_len + 1, ... on the device (accepted slots and
    result at device addresses p_slots, p_result); the caller advances
    seq_len."""
    tree_pages = scratch_pages_of(kv)
    k, v = kv.k, kv.v
    if not (k.is_contiguous() and v.is_contiguous() and v.shape == k.shape and k.dim() == 5):
        raise ValueError("KV tensors must be contiguous [L, pages, page, kvh, hd] of equal shape")
    if len(tree_pages) * kv.block_size < n:
        raise ValueError("tree larger than the KV scratch pages")
    kv._ensure_capacity(kv.seq_len + commit_depth + 1)   # reference :251
    table, scratch = device_tables_of(kv, dev)
    args = (ptr(k), ptr(v), k.element_size(), k.shape[0], k.shape[3] * k.shape[4], k.stride(0),
            k.stride(1), k.stride(2), kv.block_size, p_slots, p_result, ptr(scratch),
            len(tree_pages), ptr(table), len(kv.block_table), kv.seq_len, commit_depth,
            host_count, stream)
    if _fast is not None:
        check(_fast.kv_commit(*args), "tm_op4_kv_commit")
    else:
        call("tm_op4_kv_commit", *args)


def _tree_depth(children: list[list[int]]) -> int:
    """Longest root-to-node path (edges) reachable from node 0, at most N - 1;
    bounds the sampling walk, which the reference leaves unbounded."""
    n = len(children)
    depth, frontier, seen = 0, [0], {0}
    while depth < n - 1:
        nxt = [c for node in frontier for c in children[node] if c not in seen]
        if not nxt:
            break
        seen.update(nxt)
        frontier = nxt
        depth += 1
    return depth


def fused_verify_commit(
    target_logits: torch.Tensor,     # [N, V] fp32 or bf16
    draft_probs: torch.Tensor,       # [N, V] (unused by greedy verification)
    tree_tokens: torch.Tensor,       # [N]
    tree_parent: torch.Tensor,       # [N]
    children: list[list[int]],
    kv=None,                         # PagedKVCache | None
    temperature: float = 0.0,
    rep_penalty: float = 1.0,
    prev_tokens: torch.Tensor | None = None,
    max_depth: int = 6,
    generator: torch.Generator | None = None,
) -> VerifyResult:
    if temperature < 0.0:
        raise ValueError("temperature must be >= 0")
    if rep_penalty <= 0.0:
        raise ValueError("rep_penalty must be > 0")
    if not target_logits.is_cuda:
        raise RuntimeError("treemoe_spec_amd op4 runs on ROCm devices only; got a CPU tensor")
    if target_logits.dim() != 2 or target_logits.stride(1) != 1:
        raise ValueError("target_logits must be [N, V] with unit stride along V")
    if target_logits.dtype == torch.float32:
        dtype = TM_DTYPE_F32
    elif target_logits.dtype == torch.bfloat16:
        dtype = TM_DTYPE_BF16
    else:
        raise TypeError(f"target_logits must be float32 or bfloat16, got {target_logits.dtype}")
    n, v = target_logits.shape
    # the CUDA device index: a plain int keys the per-device caches and
    # selects the device below (cheaper per call than torch.device objects)
    dev = target_logits.get_device()
    tokens = tree_tokens
    if tokens.get_device() != dev or tokens.dtype != torch.int64 or not tokens.is_contiguous():
        tokens = tokens.to(device=dev, dtype=torch.int64).contiguous()
    if tokens.numel() != n:
        raise ValueError("tree_tokens must have one entry per node")
    csr, num_edges = _cached_csr(children, n, dev)
    # fresh outputs every call (the reference returns new tensors): one
    # allocation holding accepted_slots [N], accepted_tokens [N] and
    # (bonus, num_accepted, next_root); the launches take its addresses, and
    # its views are made while the device runs them
    out = torch.empty(2 * n + 3, dtype=torch.int64, device=dev)
    p_slots = out.data_ptr()
    p_toks, p_result = p_slots + 8 * n, p_slots + 16 * n
    stream = _capi.stream_of(dev)
    c_start = csr.data_ptr()
    c_count, c_list = c_start + 4 * n, c_start + 8 * n
    if temperature != 0.0:
        q = draft_probs
        if (q is None or not q.is_cuda or q.dtype != torch.float32 or q.dim() != 2
                or tuple(q.shape) != (n, v) or q.stride(1) != 1):
            raise ValueError("sampling needs draft_probs [N, V] float32 on the logits' device "
                             "with unit stride along V")
        uniforms = torch.rand(n, generator=generator, device=dev)  # reference verify_ref.py:51
        # torch.multinomial(residual, 1, generator) (reference :87) is
        # argmax(residual / e) over these exponentials, drawn next
        bonus_exp = torch.empty(v, dtype=torch.float32, device=dev).exponential_(
            1.0, generator=generator)
        residual = torch.empty(v, dtype=torch.float32, device=dev)
        call("tm_op4_sample_walk", ptr(target_logits), dtype, n, v, target_logits.stride(0),
             ptr(q), q.stride(0), ptr(tokens), c_start, c_count, c_list, num_edges,
             ptr(uniforms), ptr(bonus_exp), float(temperature), ptr(residual), p_slots, p_toks,
             p_result, stream)
        commit_depth = _tree_depth(children)
    else:
        if rep_penalty != 1.0:
            _apply_rep_penalty(target_logits, dtype, prev_tokens, rep_penalty, stream)
        ws = _scratch(n, dev, stream)
        args = (ptr(target_logits), dtype, n, v, target_logits.stride(0), ptr(tokens), c_start,
                c_count, c_list, num_edges, max_depth, 1 if rep_penalty != 1.0 else 0,
                ws.argmax_ptr, p_slots, p_toks, p_result, ws.partials_ptr, stream)
        if _fast is not None:
            check(_fast.argmax_walk(*args), "tm_op4_argmax_walk")
        else:
            call("tm_op4_argmax_walk", *args)
        commit_depth = max_depth
    if kv is not None:
        # commit [root] + accepted path: the root token's KV (tree slot 0) is
        # part of the committed sequence too (reference :242-247), launched
        # right behind the walk.  The count comes back through the pinned
        # word the commit writes (reference :267 reads it with a
        # device-to-host copy).
        ws = _scratch(n, dev, stream)
        note = ws.host_count()
        if note:
            ws.note_np[0] = -1
        _commit(kv, p_slots, p_result, n, commit_depth, dev, stream, note)
    slots, toks, result = out.split((n, n, 3))
    bonus, num, _ = result.unbind()
    res = VerifyResult(accepted_slots=slots, accepted_tokens=toks, bonus_token=bonus,
                       num_accepted=num)
    if kv is not None:
        kv.seq_len += _read_count(ws, result) + 1
    return res
