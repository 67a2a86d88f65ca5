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
the host exactly like the reference (:267).  Sampling mode (temperature > 0)
and the repetition penalty are not implemented and raise.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from treemoe_spec_amd import _capi
from treemoe_spec_amd._capi import TM_DTYPE_BF16, TM_DTYPE_F32, call, ptr


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


def _children_csr(children: list[list[int]], n: int, device) -> torch.Tensor:
    """[starts | counts | flat] int32 in one host->device copy."""
    if len(children) != n:
        raise ValueError(f"children must list {n} nodes, got {len(children)}")
    counts = np.fromiter((len(c) for c in children), dtype=np.int64, count=n)
    flat = [c for kids in children for c in kids]
    if flat and (min(flat) < 0 or max(flat) >= n):
        raise ValueError("child index out of range")
    starts = np.zeros(n, dtype=np.int64)
    if n > 1:
        starts[1:] = np.cumsum(counts)[:-1]
    packed = np.concatenate([starts, counts, np.asarray(flat or [0], dtype=np.int64)])
    return torch.from_numpy(packed.astype(np.int32)).to(device, non_blocking=False)


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
    if temperature != 0.0 or rep_penalty != 1.0:
        raise NotImplementedError(
            "treemoe_spec_amd implements greedy verification (temperature == 0, "
            "rep_penalty == 1) only")
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
    dev = target_logits.device
    tokens = tree_tokens.to(device=dev, dtype=torch.int64).contiguous()
    if tokens.numel() != n:
        raise ValueError("tree_tokens must have one entry per node")
    csr = _children_csr(children, n, dev)
    argmax = torch.empty(n, dtype=torch.int32, device=dev)
    slots = torch.empty(n, dtype=torch.int64, device=dev)
    toks = torch.empty(n, dtype=torch.int64, device=dev)
    result = torch.empty(3, dtype=torch.int64, device=dev)
    stream = _capi.stream_of(dev)
    call("tm_op4_argmax_walk", ptr(target_logits), dtype, n, v, target_logits.stride(0),
         ptr(tokens), ptr(csr), ptr(csr) + 4 * n, ptr(csr) + 8 * n, max_depth, ptr(argmax),
         ptr(slots), ptr(toks), ptr(result), ptr(argmax_workspace(n, dev)), stream)
    res = VerifyResult(accepted_slots=slots, accepted_tokens=toks,
                       bonus_token=result[0], num_accepted=result[1])
    if kv is not None:
        # commit [root] + accepted path: the root token's KV (tree slot 0) is
        # part of the committed sequence too (reference :242-247).
        m_max = max_depth + 1
        kv._ensure_capacity(kv.seq_len + m_max)
        table, scratch = kv.device_tables(dev)
        k = kv.k
        if not (k.is_contiguous() and kv.v.is_contiguous() and kv.v.shape == k.shape):
            raise ValueError("KV tensors must be contiguous and of equal shape")
        if len(kv.tree_pages) * kv.block_size < n:
            raise ValueError("tree larger than the KV scratch pages")
        call("tm_op4_kv_commit", ptr(k), ptr(kv.v), k.element_size(), k.shape[0],
             k.shape[3] * k.shape[4], k.stride(0), k.stride(1), k.stride(2), kv.block_size,
             ptr(slots), ptr(result), ptr(scratch), len(kv.tree_pages), ptr(table),
             len(kv.block_table), kv.seq_len, max_depth, stream)
        kv.seq_len += int(res.num_accepted) + 1
    return res
