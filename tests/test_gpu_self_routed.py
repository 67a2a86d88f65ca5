"""op1 at few tokens on the tiled path: the gate/up launch routes its own
jobs and writes the routing outputs (tm_op1_prefill_gemm1_routed), replacing
the separate bucketing launch.

Bar: every routing output it writes (expert ids, gate weights, demand, the
padded and compact layouts, the tile list) is bit-exact against the C oracle
and equal to what the separate routing launch (route_experts) writes; the
layer output is bitwise that of the two-phase path (route_experts, then
tree_moe_forward with that routing), bitwise repeatable, and within rel-L2
1e-2 of the FP64 golden.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import op1_ref, oracle_c
from tests.conftest import bf16_bits, make_moe_inputs

pytestmark = pytest.mark.gpu

FIELDS = ("topk_ids", "gates_flat", "padded_slots", "block_expert_ids", "slot_to_row",
          "demand", "expert_offsets", "sorted_slots", "slot_pos", "tiles")

# t, e, h, i, budget, objective, accept, block_m
CASES = [
    (64, 8, 512, 1024, 8, "mass", "ones", 16),             # 64-row gate/up tile
    (64, 8, 512, 1024, 4, "mass", "uniform", 16),          # 128-row gate/up tile
    (64, 8, 512, 1024, 2, "critical_path", "uniform", 32),
    (37, 8, 256, 512, 3, "critical_path", "uniform", 16),
    (64, 16, 256, 512, 6, "mass", "uniform", 32),          # the expert limit
    (50, 16, 256, 768, 16, "critical_path", "uniform", 16),
    (1, 8, 256, 512, 2, "mass", "uniform", 16),
    (2, 2, 256, 512, 2, "mass", "uniform", 16),
    (64, 8, 512, 1024, 8, "mass", "zeros", 16),            # every token degraded
    (33, 12, 256, 512, 5, "critical_path", "uniform", 32),  # E not a multiple of 4
]


def _op1():
    from treemoe_spec_amd.kernels import op1_tree_moe

    return op1_tree_moe


def _tiled(monkeypatch, m, block_m):
    monkeypatch.setattr(m, "BM", block_m)
    monkeypatch.setattr(m, "TILED_MIN_ROWS", 1)
    monkeypatch.setattr(m, "TILED_MIN_ROWS_WIDE", 1)


def _inputs(t, e, h, i, accept_kind, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x, w1, w2, w3, router, accept = make_moe_inputs(t, e, h, i, g, dtype=dtype)
    if accept_kind == "ones":
        accept = torch.ones(t)
    elif accept_kind == "zeros":
        accept = torch.zeros(t)
    return x, w1, w2, w3, router, accept


def _snapshot(m, t, e, h, i, budget, dtype, block_m):
    ws = m._ws_cache[(t, e, h, i, torch.cuda.current_device(), dtype, block_m)]
    r = m._routing_of(ws, t, budget)
    return {f: getattr(r, f).clone() for f in FIELDS}


@pytest.mark.parametrize("t,e,h,i,budget,objective,accept_kind,block_m", CASES)
def test_self_routed_matches_oracle_and_two_phase(t, e, h, i, budget, objective, accept_kind,
                                                 block_m, monkeypatch):
    print(f"self-routed t={t} e={e} B={budget} {objective} {accept_kind} BM={block_m}",
          flush=True)
    m = _op1()
    _tiled(monkeypatch, m, block_m)
    assert m.self_routed(t, budget, e, i)
    x, w1, w2, w3, router, accept = _inputs(t, e, h, i, accept_kind, 1000 + t + e + budget)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    out = m.tree_moe_forward(*dev, budget, routing_objective=objective).clone()
    got = _snapshot(m, t, e, h, i, budget, torch.bfloat16, block_m)

    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(router))
    ref = oracle_c.route_bucket(gates, accept.numpy(), budget, objective=objective,
                                block_m=block_m)
    assert np.array_equal(got["topk_ids"].reshape(-1).cpu().numpy(), ref.topk_ids)
    assert np.array_equal(got["gates_flat"].cpu().numpy().view(np.uint32),
                          ref.gates_flat.view(np.uint32))
    assert np.array_equal(got["demand"].cpu().numpy().view(np.uint32), ref.demand.view(np.uint32))
    for f in ("padded_slots", "block_expert_ids", "slot_to_row", "expert_offsets",
              "sorted_slots", "slot_pos"):
        assert np.array_equal(got[f].cpu().numpy(), getattr(ref, f)), f
    assert np.array_equal(got["tiles"].cpu().numpy(), ref.tiles)

    routing = m.route_experts(dev[0], dev[4], dev[5], budget, i, routing_objective=objective)
    for f in FIELDS:
        assert torch.equal(getattr(routing, f), got[f]), f
    two = m.tree_moe_forward(*dev, budget, routing=routing, routing_objective=objective)
    assert torch.equal(two, out)
    again = m.tree_moe_forward(*dev, budget, routing_objective=objective)
    assert torch.equal(again, out)

    ids = torch.from_numpy(ref.topk_ids).view(t, 2)
    wts = torch.from_numpy(ref.gates_flat).view(t, 2)
    golden = op1_ref.expert_ffn_golden(x, w1, w2, w3, ids, wts)
    assert op1_ref.rel_l2(out.cpu().float(), golden) <= 1e-2


def test_self_routed_f16(monkeypatch):
    print("self-routed fp16", flush=True)
    m = _op1()
    _tiled(monkeypatch, m, 16)
    t, e, h, i, budget = 64, 8, 512, 1024, 4
    x, w1, w2, w3, router, accept = _inputs(t, e, h, i, "uniform", 77, dtype=torch.float16)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    out = m.tree_moe_forward(*dev, budget).clone()
    got = _snapshot(m, t, e, h, i, budget, torch.float16, 16)
    routing = m.route_experts(dev[0], dev[4], dev[5], budget, i)
    for f in FIELDS:
        assert torch.equal(getattr(routing, f), got[f]), f
    assert torch.equal(m.tree_moe_forward(*dev, budget, routing=routing), out)
    golden = op1_ref.expert_ffn_golden(x.float(), w1.float(), w2.float(), w3.float(),
                                       routing.topk_ids.cpu(), routing.gates_flat.cpu().view(t, 2))
    assert op1_ref.rel_l2(out.cpu().float(), golden) <= 1e-2


def test_self_routed_then_other_shapes(monkeypatch):
    """Self-routed and separately routed layers of different sizes in turn:
    each call's routing and output match its two-phase counterpart."""
    print("self-routed, shapes in turn", flush=True)
    m = _op1()
    _tiled(monkeypatch, m, 16)
    for t, budget in ((64, 8), (32, 4), (300, 8), (64, 2), (16, 8), (65, 8)):
        x, w1, w2, w3, router, accept = _inputs(t, 8, 256, 512, "uniform", 500 + t)
        dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
        out = m.tree_moe_forward(*dev, budget).clone()
        routing = m.route_experts(dev[0], dev[4], dev[5], budget, 512)
        assert torch.equal(m.tree_moe_forward(*dev, budget, routing=routing), out), (t, budget)
