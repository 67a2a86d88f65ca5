"""CPU: the rule the GPU routing-parity test applies (tests/route_parity.py)
rejects a planted near-tie flip and a wrongly resolved exact tie, and accepts
an exact tie resolved to the lower expert id."""

from __future__ import annotations

import pytest
import torch

from oracle import op1_ref
from tests.route_parity import classify_id_rows, require_bit_exact


def _route(logits: torch.Tensor, budget: int):
    gates = torch.softmax(logits.float(), dim=-1)
    accept = torch.ones(logits.shape[0])
    ids, _ = op1_ref.budget_route(gates, accept, budget)
    keep = set(op1_ref.keep_set(gates, accept, budget).tolist())
    return gates, ids, keep


def _logits(seed: int, t: int = 64, e: int = 8) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(t, e, generator=g) * 1.5).to(torch.bfloat16)


def test_identical_routing_passes():
    logits = _logits(1)
    gates, ids, keep = _route(logits, 8)
    ties, flips = classify_id_rows(ids, ids, gates, keep, keep, torch.zeros_like(logits,
                                                                              dtype=torch.bool))
    assert ties == [] and flips == []
    require_bit_exact(keep, keep, flips)


def test_planted_near_tie_flip_fails():
    """Swap a row's second pick with the nearest unpicked expert in the
    "device" logits: the ids differ because logits differ, which the bar
    rejects."""
    logits_t = _logits(2)
    gates_t, ids_t, keep_t = _route(logits_t, 8)
    r = 5
    second = int(ids_t[r, 1])
    rest = [j for j in range(8) if j not in ids_t[r].tolist()]
    near = max(rest, key=lambda j: float(logits_t[r, j]))
    assert float(logits_t[r, near]) < float(logits_t[r, second])
    logits_d = logits_t.clone()
    logits_d[r, second], logits_d[r, near] = logits_t[r, near], logits_t[r, second]
    gates_d, ids_d, keep_d = _route(logits_d, 8)
    assert int(ids_d[r, 1]) == near
    differ = logits_d != logits_t
    ties, flips = classify_id_rows(ids_d, ids_t, gates_t, keep_d, keep_t, differ)
    assert flips == [r] and ties == []
    with pytest.raises(AssertionError, match="bf16 logit differs"):
        require_bit_exact(keep_d, keep_t, flips)


def test_planted_keep_set_flip_fails():
    """Budget 4: swap the demand of the last kept and the first dropped
    expert by exchanging their logit columns; the keep sets differ."""
    logits_t = _logits(3)
    gates_t, ids_t, keep_t = _route(logits_t, 4)
    demand = gates_t.sum(0)
    order = torch.argsort(demand, descending=True, stable=True).tolist()
    a, b = order[3], order[4]
    logits_d = logits_t.clone()
    logits_d[:, [a, b]] = logits_t[:, [b, a]]
    gates_d, ids_d, keep_d = _route(logits_d, 4)
    assert keep_d != keep_t
    ties, flips = classify_id_rows(ids_d, ids_t, gates_t, keep_d, keep_t,
                                   logits_d != logits_t)
    with pytest.raises(AssertionError, match="keep set"):
        require_bit_exact(keep_d, keep_t, flips)


def test_exact_tie_lower_id_passes_and_higher_id_fails():
    logits = _logits(4)
    r = 7
    first, second = (int(i) for i in _route(logits, 8)[1][r])
    # plant an exact tie of the second pick with a lower-id unpicked expert
    lower = [j for j in range(8) if j < second and j != first]
    if not lower:
        pytest.skip("no lower id to tie with at this seed")
    j = lower[0]
    logits[r, j] = logits[r, second]
    gates, ids_t, keep = _route(logits, 8)
    no_diff = torch.zeros(logits.shape, dtype=torch.bool)
    lo, hi = sorted((j, second))
    ids_lo = ids_t.clone()
    ids_lo[r, 1] = lo
    ids_hi = ids_t.clone()
    ids_hi[r, 1] = hi
    # whichever torch picked, the device's lower-id resolution is accepted
    ties, flips = classify_id_rows(ids_lo, ids_t, gates, keep, keep, no_diff)
    assert flips == [] and ties in ([], [r])
    require_bit_exact(keep, keep, flips)
    # resolving the tie to the higher id is an error
    torch_lo = ids_t.clone()
    torch_lo[r, 1] = lo
    with pytest.raises(AssertionError, match="not the lowest id"):
        classify_id_rows(ids_hi, torch_lo, gates, keep, keep, no_diff)
