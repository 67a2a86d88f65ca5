"""CPU: the oracle reproduces the committed golden fixtures bit for bit, and
the fixtures agree with the torch restatement of the reference."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import op1_ref, op4_ref, oracle_c
from tests.golden import make_golden as mg

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def op1g():
    return dict(np.load(GOLDEN / "op1_golden.npz"))


@pytest.fixture(scope="module")
def op4g():
    return dict(np.load(GOLDEN / "op4_golden.npz"))


@pytest.mark.parametrize("seed", mg.SEEDS)
def test_inputs_and_gates(op1g, seed):
    x, router, accept = mg.inputs_for(seed)
    assert np.array_equal(mg.bits(x), op1g[f"s{seed}/x"])
    assert np.array_equal(mg.bits(router), op1g[f"s{seed}/router"])
    gates = oracle_c.router_gates(op1g[f"s{seed}/x"], op1g[f"s{seed}/router"])
    assert np.array_equal(gates.view(np.uint32), op1g[f"s{seed}/gates"].view(np.uint32))
    assert float(op1g[f"s{seed}/weight_checksum"]) == mg.weight_checksum(*mg.weights_for(seed))


@pytest.mark.parametrize("seed,budget,objective,accept_kind", list(mg.op1_cases()))
def test_routing_fixtures(op1g, seed, budget, objective, accept_kind):
    key = f"s{seed}/B{budget}/{objective}/{accept_kind}"
    accept = op1g[f"s{seed}/accept"] if accept_kind == "uniform" else np.ones(mg.T, np.float32)
    gates = op1g[f"s{seed}/gates"]
    r = oracle_c.route_bucket(gates, accept, budget, objective=objective)
    for field in ("topk_ids", "padded_slots", "block_expert_ids", "slot_to_row",
                  "expert_offsets", "sorted_slots", "slot_pos", "tiles"):
        assert np.array_equal(getattr(r, field), op1g[f"{key}/{field}"]), field
    for field in ("gates_flat", "demand"):
        assert np.array_equal(getattr(r, field).view(np.uint32),
                              op1g[f"{key}/{field}"].view(np.uint32)), field
    ids, w = op1_ref.budget_route(torch.from_numpy(gates), torch.from_numpy(accept), budget,
                                  routing_objective=objective)
    got = torch.from_numpy(op1g[f"{key}/topk_ids"]).view(-1, 2)
    for t in (got != ids).any(1).nonzero().flatten().tolist():
        a, b = got[t].tolist()
        assert ids[t].tolist() == [b, a] and gates[t, a] == gates[t, b]


def test_op1_output_fixture(op1g):
    seed = mg.SEEDS[0]
    x, router, accept = mg.inputs_for(seed)
    w1, w2, w3 = mg.weights_for(seed)
    for budget in (2, 4, 8):
        for objective in ("mass", "critical_path"):
            key = f"s{seed}/B{budget}/{objective}/uniform"
            out = op1_ref.expert_ffn_golden(x, w1, w2, w3,
                                            torch.from_numpy(op1g[f"{key}/topk_ids"]),
                                            torch.from_numpy(op1g[f"{key}/gates_flat"]))
            assert np.array_equal(out.float().numpy(), op1g[f"{key}/out_fp64_as_fp32"])


@pytest.mark.parametrize("i", range(20))
def test_op4_fixtures(op4g, i):
    p = f"t{i}"
    parent = op4g[f"{p}/parent"].tolist()
    children = [[] for _ in parent]
    for c in range(1, len(parent)):
        children[parent[c]].append(c)
    tokens = torch.from_numpy(op4g[f"{p}/tokens"])
    logits = torch.from_numpy(op4g[f"{p}/logits"])
    slots, toks, bonus, num = op4_ref.tree_verify(logits, None, tokens, children)
    assert np.array_equal(slots.numpy(), op4g[f"{p}/accepted_slots"])
    assert [bonus, num] == op4g[f"{p}/bonus_num"].tolist()
    c = oracle_c.greedy_walk(oracle_c.argmax(op4g[f"{p}/logits"]), op4g[f"{p}/tokens"],
                             children, 64)
    assert np.array_equal(c[0], op4g[f"{p}/accepted_slots"]) and [c[2], c[3]] == [bonus, num]


def test_kv_commit_fixture(op4g):
    k = op4g["kv/k_before"].copy()
    v = op4g["kv/v_before"].copy()
    acc = op4g["kv/accepted"]
    num = int((acc >= 0).sum())
    oracle_c.kv_commit(k, v, acc, num, op4g["kv/scratch"], op4g["kv/table"],
                       int(op4g["kv/seq_len"]))
    assert np.array_equal(k, op4g["kv/k_after"]) and np.array_equal(v, op4g["kv/v_after"])
