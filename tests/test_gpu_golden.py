"""GPU: the HIP path on the committed golden fixtures (bit-exact routing and
KV bytes, rel-L2 <= 1e-2 outputs, exact greedy results)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import op1_ref
from tests.golden import make_golden as mg

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _t(bits16: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits16.view(np.int16).copy()).view(torch.bfloat16)


@pytest.fixture(scope="module")
def op1g():
    return dict(np.load(GOLDEN / "op1_golden.npz"))


@pytest.fixture(scope="module")
def op4g():
    return dict(np.load(GOLDEN / "op4_golden.npz"))


@pytest.mark.parametrize("seed,budget,objective,accept_kind", list(mg.op1_cases()))
def test_routing_on_fixtures(op1g, seed, budget, objective, accept_kind):
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    print(f"golden routing {seed} {budget} {objective} {accept_kind}", flush=True)
    key = f"s{seed}/B{budget}/{objective}/{accept_kind}"
    x = _t(op1g[f"s{seed}/x"]).cuda()
    router = _t(op1g[f"s{seed}/router"]).cuda()
    accept = op1g[f"s{seed}/accept"] if accept_kind == "uniform" else np.ones(mg.T, np.float32)
    r = m.route_experts(x, router, torch.from_numpy(accept).cuda(), budget, mg.I,
                        routing_objective=objective)
    assert np.array_equal(r.router_gates.cpu().numpy().view(np.uint32),
                          op1g[f"s{seed}/gates"].view(np.uint32))
    for field, got in (("topk_ids", r.topk_ids.reshape(-1)), ("padded_slots", r.padded_slots),
                       ("block_expert_ids", r.block_expert_ids), ("slot_to_row", r.slot_to_row),
                       ("expert_offsets", r.expert_offsets), ("sorted_slots", r.sorted_slots),
                       ("slot_pos", r.slot_pos), ("tiles", r.tiles)):
        assert np.array_equal(got.cpu().numpy(), op1g[f"{key}/{field}"]), field
    for field, got in (("gates_flat", r.gates_flat), ("demand", r.demand)):
        assert np.array_equal(got.cpu().numpy().view(np.uint32),
                              op1g[f"{key}/{field}"].view(np.uint32)), field


@pytest.mark.parametrize("budget", [2, 4, 8])
@pytest.mark.parametrize("objective", ["mass", "critical_path"])
def test_forward_on_fixtures(op1g, budget, objective):
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    seed = mg.SEEDS[0]
    key = f"s{seed}/B{budget}/{objective}/uniform"
    w1, w2, w3 = (w.cuda() for w in mg.weights_for(seed))
    out = m.tree_moe_forward(_t(op1g[f"s{seed}/x"]).cuda(), w1, w2, w3,
                             _t(op1g[f"s{seed}/router"]).cuda(),
                             torch.from_numpy(op1g[f"s{seed}/accept"]).cuda(), budget,
                             routing_objective=objective)
    golden = torch.from_numpy(op1g[f"{key}/out_fp64_as_fp32"])
    assert op1_ref.rel_l2(out.cpu().float(), golden) <= 1e-2


@pytest.mark.parametrize("i", range(20))
def test_greedy_on_fixtures(op4g, i):
    from treemoe_spec_amd.kernels.op4_commit import fused_verify_commit

    p = f"t{i}"
    parent = op4g[f"{p}/parent"].tolist()
    children = [[] for _ in parent]
    for c in range(1, len(parent)):
        children[parent[c]].append(c)
    res = fused_verify_commit(torch.from_numpy(op4g[f"{p}/logits"]).cuda(), None,
                              torch.from_numpy(op4g[f"{p}/tokens"]).cuda(),
                              torch.tensor(parent).cuda(), children, max_depth=16)
    assert np.array_equal(res.accepted_slots.cpu().numpy(), op4g[f"{p}/accepted_slots"])
    assert np.array_equal(res.accepted_tokens.cpu().numpy(), op4g[f"{p}/accepted_tokens"])
    assert [int(res.bonus_token), int(res.num_accepted)] == op4g[f"{p}/bonus_num"].tolist()


def test_kv_commit_on_fixture(op4g):
    from treemoe_spec_amd import _capi

    k = _t(op4g["kv/k_before"]).cuda().contiguous()
    v = _t(op4g["kv/v_before"]).cuda().contiguous()
    acc = torch.from_numpy(op4g["kv/accepted"]).cuda()
    num = int((acc >= 0).sum())
    result = torch.tensor([0, num, 0], dtype=torch.long).cuda()
    scratch = torch.from_numpy(op4g["kv/scratch"]).cuda()
    table = torch.from_numpy(op4g["kv/table"]).cuda()
    _capi.call("tm_op4_kv_commit", k.data_ptr(), v.data_ptr(), 2, k.shape[0],
               k.shape[3] * k.shape[4], k.stride(0), k.stride(1), k.stride(2), k.shape[2],
               acc.data_ptr(), result.data_ptr(), scratch.data_ptr(), scratch.numel(),
               table.data_ptr(), table.numel(), int(op4g["kv/seq_len"]), 8, 0,
               _capi.stream_of(k.device))
    torch.cuda.synchronize()
    assert np.array_equal(k.cpu().view(torch.int16).numpy().view(np.uint16), op4g["kv/k_after"])
    assert np.array_equal(v.cpu().view(torch.int16).numpy().view(np.uint16), op4g["kv/v_after"])
