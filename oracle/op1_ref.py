"""TEST INFRASTRUCTURE ONLY: torch restatement of the op1/op3 reference.

These functions make the same torch calls, in the same order, as the
reference's pure-PyTorch path, so that they (a) pin the C oracle's routing
decisions against the reference algorithm and (b) serve as the CPU baseline
that the benchmark times.  References:

* ``budget_route``        treemoe/ref/tree_moe_ref.py:14-67
* ``route_and_bucket``    treemoe/ref/tree_moe_ref.py:70-99
* ``padded_layout``       treemoe/kernels/op1_tree_moe.py:81-149
* ``tree_moe_forward``    treemoe/ref/tree_moe_ref.py:102-130
* ``expert_ffn_golden``   the same expert loop in FP64 for given routing (the
                          reference's FP32 golden is this loop on FP32 inputs,
                          tests/test_op1.py:195-197)
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def keep_set(gates: torch.Tensor, accept: torch.Tensor, expert_budget: int,
             top1_threshold: float = 0.05, routing_objective: str = "mass") -> torch.Tensor:
    """The experts op3 keeps (tree_moe_ref.py:34-49), in keep order."""
    e = gates.shape[1]
    demand = (accept.unsqueeze(1) * gates).sum(0)
    by_demand = torch.argsort(demand, descending=True, stable=True)
    if routing_objective == "critical_path":
        full = gates.topk(2, dim=-1).indices
        axis = torch.arange(e, device=gates.device)
        need = (full[:, :1] == axis) | (
            (full[:, 1:2] == axis) & (accept >= top1_threshold).unsqueeze(1))
        crit = torch.where(need, accept.unsqueeze(1), -torch.inf).amax(0)
        return by_demand[torch.argsort(crit[by_demand], descending=True,
                                       stable=True)[:expert_budget]]
    return by_demand[:expert_budget]


def budget_route(gates: torch.Tensor, accept: torch.Tensor, expert_budget: int,
                 top1_threshold: float = 0.05, routing_objective: str = "mass"):
    """op3: acceptance-weighted expert budget, masked top-2, renorm, degrade.

    Returns (topk_ids [N, 2] int64, topk_gates [N, 2] fp32)."""
    n, e = gates.shape
    if not 2 <= expert_budget <= e:
        raise ValueError(f"expert_budget must be in [2, {e}]")
    if routing_objective not in ("mass", "critical_path"):
        raise ValueError("routing_objective must be 'mass' or 'critical_path'")
    keep = keep_set(gates, accept, expert_budget, top1_threshold, routing_objective)
    kept = torch.zeros(e, dtype=torch.bool, device=gates.device)
    kept[keep] = True
    w, ids = gates.masked_fill(~kept, 0.0).topk(2, dim=-1)
    w = w / w.sum(-1, keepdim=True)
    low = (accept < top1_threshold).unsqueeze(1)
    top1 = torch.zeros_like(w)
    top1[:, 0] = 1.0
    return ids, torch.where(low, top1, w)


def router_gates(x: torch.Tensor, router_weight: torch.Tensor) -> torch.Tensor:
    """F.linear in the input dtype, then fp32 softmax (tree_moe_ref.py:83-84)."""
    return torch.softmax(F.linear(x, router_weight).float(), dim=-1)


def route_and_bucket(x, router_weight, accept, expert_budget, routing_objective="mass",
                     gates=None):
    """Returns (topk_ids, topk_gates, sorted_slots, expert_offsets)."""
    if gates is None:
        gates = router_gates(x, router_weight)
    ids, w = budget_route(gates, accept, expert_budget,
                          routing_objective=routing_objective)
    e = gates.shape[1]
    flat = ids.reshape(-1)
    order = torch.argsort(flat, stable=True)
    offsets = torch.zeros(e + 1, dtype=torch.long)
    offsets[1:] = torch.bincount(flat, minlength=e).cumsum(0)
    return ids, w, order, offsets


def padded_layout(topk_ids: torch.Tensor, num_experts: int, max_blocks: int,
                  block_m: int = 16):
    """Reference padded BM-row block layout for flat expert ids of 2T slots.

    Returns (padded_slots, block_expert_ids, slot_to_row)."""
    flat = topk_ids.reshape(-1)
    s = flat.numel()
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=num_experts)
    nblk = (counts + block_m - 1) // block_m
    bstart = torch.zeros(num_experts, dtype=torch.long)
    bstart[1:] = nblk.cumsum(0)[:-1]
    sstart = torch.zeros(num_experts, dtype=torch.long)
    sstart[1:] = counts.cumsum(0)[:-1]
    fe = flat[order]
    dest = bstart[fe] * block_m + (torch.arange(s) - sstart[fe])
    padded = torch.full((max_blocks * block_m,), -1, dtype=torch.long)
    padded[dest] = order
    blk = torch.arange(max_blocks)
    owns = (blk[:, None] >= bstart[None, :]) & (blk[:, None] < (bstart + nblk)[None, :])
    ids = torch.full((max_blocks,), -1, dtype=torch.long)
    used = owns.any(1)
    ids[used] = owns[used].long().argmax(1)
    slot_to_row = torch.empty(s, dtype=torch.long)
    slot_to_row[order] = dest
    return padded, ids, slot_to_row


def tree_moe_forward(x, w1, w2, w3, router_weight, accept, expert_budget,
                     routing_objective="mass", routing=None):
    """Expert-major loop with index_add_ in x.dtype (tree_moe_ref.py:102-130).

    ``routing`` = (topk_ids, topk_gates, sorted_slots, expert_offsets) replaces
    the internal router when given."""
    if routing is None:
        routing = route_and_bucket(x, router_weight, accept, expert_budget,
                                   routing_objective=routing_objective)
    _, w, order, offsets = routing
    out = torch.zeros_like(x)
    for e in range(w1.shape[0]):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if lo == hi:
            continue
        slots = order[lo:hi]
        tok, k = slots // 2, slots % 2
        xe = x[tok]
        h = F.silu(xe @ w1[e].t()) * (xe @ w3[e].t())
        out.index_add_(0, tok, (h @ w2[e].t()) * w[tok, k].unsqueeze(1).to(x.dtype))
    return out


def expert_ffn_golden(x, w1, w2, w3, topk_ids, topk_gates, dtype=torch.float64,
                      experts=None):
    """sum_k g_k * W2 (silu(W1 x) * W3 x) per token, computed in ``dtype``.

    topk_ids / topk_gates: [T, 2].  ``experts`` restricts the sum to a subset of
    expert ids (used to sample the work on the CPU)."""
    t = x.shape[0]
    out = torch.zeros(t, x.shape[1], dtype=dtype)
    xd = x.to(dtype)
    ids = topk_ids.reshape(t, 2)
    gw = topk_gates.reshape(t, 2).to(dtype)
    for e in range(w1.shape[0]):
        if experts is not None and e not in experts:
            continue
        sel = (ids == e)
        rows = sel.any(1).nonzero().flatten()
        if rows.numel() == 0:
            continue
        g = (gw * sel.to(dtype)).sum(1)[rows]
        xe = xd[rows]
        h = F.silu(xe @ w1[e].to(dtype).t()) * (xe @ w3[e].to(dtype).t())
        out[rows] += (h @ w2[e].to(dtype).t()) * g.unsqueeze(1)
    return out


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a64, b64 = a.double(), b.double()
    return float((a64 - b64).norm() / b64.norm().clamp_min(1e-300))
