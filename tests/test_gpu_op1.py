"""op1 parity on the GPU: HIP library vs the CPU oracle.

Bar: routing (expert ids, gate weights, demand, every layout index) is
bit-exact against the C oracle; the MoE output is within rel-L2 <= 1e-2 of an
FP64 (small shapes) or FP32 torch (Mixtral shapes) evaluation of the same
expert FFN with the same routing; outputs are bitwise reproducible.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle_c
from oracle import op1_ref
from tests.conftest import bf16_bits, make_moe_inputs

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-2


def _op1():
    from treemoe_spec_amd.kernels import op1_tree_moe

    return op1_tree_moe


def _say(msg: str) -> None:
    print(msg, flush=True)


def _route_case(seed, t, e, h, budget, objective, accept_kind, block_m=16, router_scale=0.1):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    router = (torch.randn(e, h, generator=g) * router_scale).to(torch.bfloat16)
    if accept_kind == "ones":
        accept = torch.ones(t)
    elif accept_kind == "zeros":
        accept = torch.zeros(t)
    else:
        accept = torch.rand(t, generator=g)
    return x, router, accept


@pytest.mark.parametrize("t,h,e", [(1, 64, 8), (5, 512, 8), (64, 4096, 8), (64, 256, 2),
                                   (33, 1024, 16), (2048, 4096, 8), (64, 512, 64),
                                   # the row router (T >= 1024, W_g in LDS): ragged last
                                   # workgroup, H = 2048 with E = 16; then a W_g too large
                                   # for its LDS copy (one workgroup per token)
                                   (1025, 4096, 8), (1100, 2048, 16), (1024, 4096, 16)])
def test_router_gates_bit_exact(t, h, e):
    _say(f"router t={t} h={h} e={e}")
    m = _op1()
    x, router, _ = _route_case(7, t, e, h, 2, "mass", "ones")
    gates = torch.empty(t, e, dtype=torch.float32, device="cuda")
    m._launch_router(x.cuda(), router.cuda(), gates)
    expect = oracle_c.router_gates(bf16_bits(x), bf16_bits(router))
    got = gates.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


@pytest.mark.parametrize("t,h,e", [(5, 512, 8), (64, 4096, 8), (2048, 4096, 8),
                                   (1100, 2048, 16)])
def test_router_gates_f16_bit_exact(t, h, e):
    """fp16 operands: logits rounded to fp16 (F.linear on fp16 operands), the
    softmax in fp32; bit-exact against the oracle on both router kernels."""
    _say(f"router fp16 t={t} h={h} e={e}")
    m = _op1()
    g = torch.Generator().manual_seed(t + h)
    x = torch.randn(t, h, generator=g).half()
    router = (torch.randn(e, h, generator=g) * 0.1).half()
    gates = torch.empty(t, e, dtype=torch.float32, device="cuda")
    m._launch_router(x.cuda(), router.cuda(), gates)
    expect = oracle_c.router_gates(bf16_bits(x), bf16_bits(router), f16=True)
    assert np.array_equal(gates.cpu().numpy().view(np.uint32), expect.view(np.uint32))


def _forward_f16(t, e, h, i, budget, seed):
    m = _op1()
    g = torch.Generator().manual_seed(seed)
    x, w1, w2, w3, router, accept = make_moe_inputs(t, e, h, i, g)
    x, w1, w2, w3, router = (a.half() for a in (x, w1, w2, w3, router))
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    out = m.tree_moe_forward(*dev, budget)
    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(router), f16=True)
    ref = oracle_c.route_bucket(gates, accept.numpy(), budget)
    r = m.route_experts(dev[0], dev[4], dev[5], budget, i)
    assert np.array_equal(r.topk_ids.reshape(-1).cpu().numpy(), ref.topk_ids)
    golden = op1_ref.expert_ffn_golden(x, w1, w2, w3, torch.from_numpy(ref.topk_ids).view(t, 2),
                                       torch.from_numpy(ref.gates_flat).view(t, 2))
    return out, golden


@pytest.mark.parametrize("path", ["stream", "tiled", "tiled_bucket"])
@pytest.mark.parametrize("budget", [4, 8])
def test_forward_f16_matches_fp64_golden(budget, path, monkeypatch):
    """fp16 I/O (the reference kernels take fp16 too, op1_tree_moe.py:762-766):
    fp16 h and output, fp32 accumulation; routing ids equal the oracle's."""
    _say(f"forward fp16 B={budget} {path}")
    _force_path(monkeypatch, path)
    out, golden = _forward_f16(64, 8, 512, 1024, budget, 41 + budget)
    assert out.dtype == torch.float16
    err = op1_ref.rel_l2(out.cpu().float(), golden)
    assert err <= REL_L2_TOL, err


@pytest.mark.parametrize("t,h,i", [(64, 4096, 14336), (2048, 512, 1024)])
def test_forward_f16_large_shapes(t, h, i):
    """fp16 at the Mixtral layer shape (the tiled GEMMs with the 64-row gate/up
    tile) and at T=2048 (256-row gate/up tiles, the last tile of each expert
    running 1-4 of its 64-row parts)."""
    _say(f"forward fp16 t={t} h={h} i={i}")
    out, golden = _forward_f16(t, 8, h, i, 8, 43)
    err = op1_ref.rel_l2(out.cpu().float(), golden)
    assert out.dtype == torch.float16 and err <= REL_L2_TOL, err


def test_forward_rejects_mixed_dtypes():
    m = _op1()
    g = torch.Generator().manual_seed(3)
    x, w1, w2, w3, router, accept = (a.cuda() for a in make_moe_inputs(8, 4, 256, 256, g))
    with pytest.raises(TypeError, match="dtype"):
        m.tree_moe_forward(x.half(), w1.half(), w2.bfloat16(), w3.half(), router.half(), accept, 2)
    with pytest.raises(TypeError, match="float16"):
        m.tree_moe_forward(x, w1, w2, w3, router, accept, 2)


ROUTE_CASES = [
    (seed, t, budget, objective, accept_kind)
    for seed, t in ((0, 16), (1, 64), (2, 128), (3, 2048), (4, 4096), (5, 7))
    for budget in (2, 4, 8)
    for objective in ("mass", "critical_path")
    for accept_kind in ("ones", "uniform")
]


@pytest.mark.parametrize("seed,t,budget,objective,accept_kind", ROUTE_CASES)
def test_route_bucket_bit_exact(seed, t, budget, objective, accept_kind):
    _say(f"route seed={seed} t={t} B={budget} {objective} {accept_kind}")
    m = _op1()
    e, h = 8, 256
    x, router, accept = _route_case(seed, t, e, h, budget, objective, accept_kind)
    for block_m in (16, 32):
        got = m.route_and_bucket(x.cuda(), router.cuda(), accept.cuda(), budget,
                                 block_m=block_m, return_demand=True,
                                 routing_objective=objective)
        gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(router))
        ref = oracle_c.route_bucket(gates, accept.numpy(), budget, objective=objective,
                                    block_m=block_m)
        ids, w, padded, blk, s2r, max_blocks, demand = got
        assert max_blocks == ref.max_blocks
        assert np.array_equal(ids.reshape(-1).cpu().numpy(), ref.topk_ids)
        assert np.array_equal(w.reshape(-1).cpu().numpy().view(np.uint32),
                              ref.gates_flat.view(np.uint32))
        assert np.array_equal(padded.cpu().numpy(), ref.padded_slots)
        assert np.array_equal(blk.cpu().numpy(), ref.block_expert_ids)
        assert np.array_equal(s2r.cpu().numpy(), ref.slot_to_row)
        assert np.array_equal(demand.cpu().numpy().view(np.uint32), ref.demand.view(np.uint32))


@pytest.mark.parametrize("t,e,budget,objective,block_m", [
    (4097, 8, 4, "mass", 16), (8192, 8, 2, "critical_path", 32), (8192, 8, 8, "mass", 16),
    (20000, 8, 4, "critical_path", 16), (5000, 64, 32, "mass", 32),
    (9001, 64, 5, "critical_path", 16)])
def test_route_many_tokens_bit_exact(t, e, budget, objective, block_m):
    """More tokens than the LDS-resident bucketing holds (4096) go through the
    many-token kernel: every routing output bit-exact against the oracle."""
    _say(f"route many tokens t={t} E={e} B={budget} {objective} BM={block_m}")
    m = _op1()
    g = torch.Generator().manual_seed(t + e)
    gates = torch.softmax(torch.randn(t, e, generator=g) * 2, -1)
    accept = torch.rand(t, generator=g)
    accept[::7] = 0.01  # some tokens below tau
    x = torch.zeros(t, 256, dtype=torch.bfloat16)
    router = torch.zeros(e, 256, dtype=torch.bfloat16)
    ids, w, padded, blk, s2r, max_blocks, demand = m.route_and_bucket(
        x.cuda(), router.cuda(), accept.cuda(), budget, block_m=block_m, return_demand=True,
        router_gates=gates.cuda(), routing_objective=objective)
    ref = oracle_c.route_bucket(gates.numpy(), accept.numpy(), budget, objective=objective,
                                block_m=block_m)
    assert max_blocks == ref.max_blocks
    assert np.array_equal(ids.reshape(-1).cpu().numpy(), ref.topk_ids)
    assert np.array_equal(w.reshape(-1).cpu().numpy().view(np.uint32),
                          ref.gates_flat.view(np.uint32))
    assert np.array_equal(padded.cpu().numpy(), ref.padded_slots)
    assert np.array_equal(blk.cpu().numpy(), ref.block_expert_ids)
    assert np.array_equal(s2r.cpu().numpy(), ref.slot_to_row)
    assert np.array_equal(demand.cpu().numpy().view(np.uint32), ref.demand.view(np.uint32))


def test_route_experts_many_tokens_layout():
    """route_experts at T = 8192 (router + many-token bucketing): the compact
    layout the GEMMs consume equals the oracle's."""
    _say("route_experts t=8192")
    m = _op1()
    t, e, h = 8192, 8, 512
    x, router, accept = _route_case(11, t, e, h, 4, "mass", "uniform")
    r = m.route_experts(x.cuda(), router.cuda(), accept.cuda(), 4, inter=512)
    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(router))
    ref = oracle_c.route_bucket(gates, accept.numpy(), 4)
    assert np.array_equal(r.topk_ids.reshape(-1).cpu().numpy(), ref.topk_ids)
    assert np.array_equal(r.sorted_slots.cpu().numpy(), ref.sorted_slots)
    assert np.array_equal(r.slot_pos.cpu().numpy(), ref.slot_pos)
    assert np.array_equal(r.expert_offsets.cpu().numpy(), ref.expert_offsets)
    assert np.array_equal(r.tiles.cpu().numpy(), ref.tiles)


def test_forward_many_tokens_matches_golden():
    """A layer of 6000 tokens (more than the LDS-resident bucketing holds)
    end to end against the FP64 golden."""
    _say("forward t=6000")
    out, golden, _, _ = _forward_and_golden(6000, 8, 256, 512, 4, 31)
    err = op1_ref.rel_l2(out.cpu().float(), golden)
    assert err <= REL_L2_TOL, err


@pytest.mark.parametrize("t", [7, 64, 2048])
@pytest.mark.parametrize("budget", [2, 4, 8])
def test_bucket_from_given_gates_bit_exact(t, budget):
    """route_and_bucket(router_gates=...) runs the bucketing alone (the
    reference's Kernel A input contract, op1_tree_moe.py:159-190)."""
    _say(f"bucket from gates t={t} B={budget}")
    m = _op1()
    g = torch.Generator().manual_seed(t + budget)
    gates = torch.softmax(torch.randn(t, 8, generator=g) * 2, -1)
    accept = torch.rand(t, generator=g)
    x = torch.zeros(t, 256, dtype=torch.bfloat16)
    router = torch.zeros(8, 256, dtype=torch.bfloat16)
    for objective in ("mass", "critical_path"):
        ids, w, padded, blk, s2r, max_blocks, demand = m.route_and_bucket(
            x.cuda(), router.cuda(), accept.cuda(), budget, return_demand=True,
            router_gates=gates.cuda(), routing_objective=objective)
        ref = oracle_c.route_bucket(gates.numpy(), accept.numpy(), budget, objective=objective)
        assert np.array_equal(ids.reshape(-1).cpu().numpy(), ref.topk_ids)
        assert np.array_equal(w.reshape(-1).cpu().numpy().view(np.uint32),
                              ref.gates_flat.view(np.uint32))
        assert np.array_equal(padded.cpu().numpy(), ref.padded_slots)
        assert np.array_equal(blk.cpu().numpy(), ref.block_expert_ids)
        assert np.array_equal(s2r.cpu().numpy(), ref.slot_to_row)
        assert np.array_equal(demand.cpu().numpy().view(np.uint32), ref.demand.view(np.uint32))


def test_route_repeated_calls_of_different_sizes():
    """Back-to-back routing calls of different sizes reuse nothing stale."""
    _say("fused route repeated")
    m = _op1()
    for t in (64, 5, 64, 300, 1):
        x, router, accept = _route_case(t, t, 8, 512, 4, "mass", "uniform")
        r = m.route_experts(x.cuda(), router.cuda(), accept.cuda(), 4, inter=512)
        gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(router))
        ref = oracle_c.route_bucket(gates, accept.numpy(), 4)
        assert np.array_equal(r.topk_ids.reshape(-1).cpu().numpy(), ref.topk_ids)
        assert np.array_equal(r.tiles.cpu().numpy(), ref.tiles)


@pytest.mark.parametrize("budget", [2, 4, 8])
@pytest.mark.parametrize("objective", ["mass", "critical_path"])
def test_route_experts_compact_layout_bit_exact(budget, objective):
    _say(f"route_experts B={budget} {objective}")
    m = _op1()
    t, e, h = 64, 8, 512
    x, router, accept = _route_case(11, t, e, h, budget, objective, "uniform")
    r = m.route_experts(x.cuda(), router.cuda(), accept.cuda(), budget, inter=1024,
                        routing_objective=objective)
    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(router))
    ref = oracle_c.route_bucket(gates, accept.numpy(), budget, objective=objective,
                                block_m=m.BM)
    assert np.array_equal(r.router_gates.cpu().numpy().view(np.uint32), gates.view(np.uint32))
    assert np.array_equal(r.expert_offsets.cpu().numpy(), ref.expert_offsets)
    assert np.array_equal(r.sorted_slots.cpu().numpy(), ref.sorted_slots)
    assert np.array_equal(r.slot_pos.cpu().numpy(), ref.slot_pos)
    assert np.array_equal(r.tiles.cpu().numpy(), ref.tiles)
    assert r.max_blocks == ref.max_blocks
    assert r.launch_blocks == m.compact_block_limit(2 * t, budget)


@pytest.mark.parametrize("t,budget", [(32, 4), (64, 2), (64, 4), (64, 8), (128, 8), (7, 3)])
def test_routing_ids_match_reference_algorithm(t, budget):
    """The device's routing decisions equal the reference's torch algorithm
    (budget_route_ref) applied to the same gates."""
    _say(f"ids vs torch reference t={t} B={budget}")
    m = _op1()
    e, h = 8, 4096
    g = torch.Generator().manual_seed(3)
    x = torch.randn(t, h, generator=g, dtype=torch.bfloat16)
    router = (torch.randn(e, h, generator=g, dtype=torch.bfloat16) * 0.1)
    accept = torch.rand(t, generator=g)
    for objective in ("mass", "critical_path"):
        ids, w, *_ = m.route_and_bucket(x.cuda(), router.cuda(), accept.cuda(), budget,
                                        routing_objective=objective)
        gates = torch.from_numpy(oracle_c.router_gates(bf16_bits(x), bf16_bits(router)))
        ref_ids, ref_w = op1_ref.budget_route(gates, accept, budget,
                                              routing_objective=objective)
        ids = ids.cpu()
        # torch.topk orders exactly equal gates in an implementation-defined
        # way; the device takes the lower expert id first.  Rows may differ
        # only by such a swap.
        for r in (ids != ref_ids).any(1).nonzero().flatten().tolist():
            a, b = ids[r].tolist()
            assert ref_ids[r].tolist() == [b, a] and gates[r, a] == gates[r, b] and a < b
        torch.testing.assert_close(w.cpu(), ref_w, rtol=1e-6, atol=1e-7)


def _forward_and_golden(t, e, h, i, budget, seed, objective="mass", accept_kind="uniform"):
    m = _op1()
    g = torch.Generator().manual_seed(seed)
    x, w1, w2, w3, router, accept = make_moe_inputs(t, e, h, i, g, dtype=torch.bfloat16)
    if accept_kind == "ones":
        accept = torch.ones(t)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    out = m.tree_moe_forward(*dev, budget, routing_objective=objective)
    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(router))
    ref = oracle_c.route_bucket(gates, accept.numpy(), budget, objective=objective)
    ids = torch.from_numpy(ref.topk_ids).view(t, 2)
    wts = torch.from_numpy(ref.gates_flat).view(t, 2)
    golden = op1_ref.expert_ffn_golden(x, w1, w2, w3, ids, wts)
    return out, golden, (x, w1, w2, w3, router, accept), ref


def _force_path(monkeypatch, path):
    """Route tree_moe_forward through the weight-streaming GEMMs ("stream")
    or the MFMA-tiled ones whatever the rows per expert: "tiled" with the
    gate/up launch routing its own jobs where the token count allows it,
    "tiled_bucket" with the separate routing launch."""
    m = _op1()
    monkeypatch.setattr(m, "TILED_MIN_ROWS", 1 << 30 if path == "stream" else 1)
    monkeypatch.setattr(m, "TILED_MIN_ROWS_WIDE", 1 << 30 if path == "stream" else 1)
    if path == "tiled_bucket":
        monkeypatch.setattr(m, "SELF_ROUTED_MAX_TOKENS", 0)


@pytest.mark.parametrize("path", ["stream", "tiled", "tiled_bucket"])
@pytest.mark.parametrize("budget", [2, 4, 8])
@pytest.mark.parametrize("objective", ["mass", "critical_path"])
def test_forward_matches_fp64_golden_small(budget, objective, path, monkeypatch):
    _say(f"forward small B={budget} {objective} {path}")
    _force_path(monkeypatch, path)
    out, golden, inputs, ref = _forward_and_golden(64, 8, 512, 1024, budget, 5, objective)
    err = op1_ref.rel_l2(out.cpu().float(), golden)
    assert err <= REL_L2_TOL, err
    # the reference's own criterion: kernel error <= 2x the bf16 reference's error
    x, w1, w2, w3, router, accept = inputs
    routing = (torch.from_numpy(ref.topk_ids).view(-1, 2),
               torch.from_numpy(ref.gates_flat).view(-1, 2),
               torch.from_numpy(ref.sorted_slots).long(),
               torch.from_numpy(ref.expert_offsets).long())
    bf = op1_ref.tree_moe_forward(x, w1, w2, w3, router, accept, budget, routing=routing)
    err_out = (out.cpu().double() - golden).abs().max().item()
    err_ref = (bf.double() - golden).abs().max().item()
    assert err_out <= 2 * err_ref + 1e-4, (err_out, err_ref)


@pytest.mark.parametrize("t", [1, 16, 64, 100, 256])
def test_forward_token_counts(t):
    _say(f"forward t={t}")
    out, golden, _, _ = _forward_and_golden(t, 8, 256, 512, 8, 9)
    assert op1_ref.rel_l2(out.cpu().float(), golden) <= REL_L2_TOL


def test_forward_tp8_share_shape():
    """One GPU's share of an 8-way tensor-parallel Mixtral layer: I = 14336 / 8
    = 1792 intermediate columns for all 8 experts at T = 64.  1792 / 2 is not a
    multiple of 256, so the down GEMM runs unsplit (split 1)."""
    _say("forward TP-8 share I=1792")
    from treemoe_spec_amd.kernels.op1_tree_moe import _split_for

    assert _split_for(1792) == 1
    out, golden, _, _ = _forward_and_golden(64, 8, 4096, 1792, 8, 21, accept_kind="ones")
    err = op1_ref.rel_l2(out.cpu().double(), golden)
    _say(f"  rel_l2={err:.3e}")
    assert err <= REL_L2_TOL


def test_forward_degrade_branch():
    _say("forward degrade")
    m = _op1()
    g = torch.Generator().manual_seed(17)
    x, w1, w2, w3, router, _ = make_moe_inputs(64, 8, 256, 512, g, dtype=torch.bfloat16)
    accept = torch.zeros(64)
    out = m.tree_moe_forward(x.cuda(), w1.cuda(), w2.cuda(), w3.cuda(), router.cuda(),
                             accept.cuda(), 8)
    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(router))
    ref = oracle_c.route_bucket(gates, accept.numpy(), 8)
    assert np.all(ref.gates_flat.reshape(-1, 2)[:, 1] == 0)
    golden = op1_ref.expert_ffn_golden(x, w1, w2, w3, torch.from_numpy(ref.topk_ids),
                                       torch.from_numpy(ref.gates_flat))
    assert op1_ref.rel_l2(out.cpu().float(), golden) <= REL_L2_TOL


def test_forward_deterministic_bitwise():
    _say("forward determinism")
    m = _op1()
    g = torch.Generator().manual_seed(11)
    x, w1, w2, w3, router, accept = make_moe_inputs(64, 8, 1024, 2048, g, dtype=torch.bfloat16)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    outs = [m.tree_moe_forward(*dev, 8, deterministic=True).clone() for _ in range(5)]
    outs.append(m.tree_moe_forward(*dev, 8, deterministic=False).clone())
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


@pytest.mark.parametrize("budget", [2, 8])
def test_two_phase_equals_inline(budget):
    _say(f"two-phase B={budget}")
    m = _op1()
    g = torch.Generator().manual_seed(21)
    x, w1, w2, w3, router, accept = make_moe_inputs(64, 8, 512, 1024, g, dtype=torch.bfloat16)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    inline = m.tree_moe_forward(*dev, budget).clone()
    routing = m.route_experts(dev[0], dev[4], dev[5], budget, 1024)
    ids = routing.expert_ids()
    assert ids and all(0 <= i < 8 for i in ids) and len(ids) <= budget
    two = m.tree_moe_forward(*dev, budget, routing=routing)
    assert torch.equal(inline, two)
    out = torch.empty_like(dev[0])
    r = m.tree_moe_forward(*dev, budget, out=out)
    assert r is out and torch.equal(out, inline)


@pytest.mark.parametrize("path", ["stream", "tiled", "tiled_bucket"])
def test_masked_expert_weights_never_read(path, monkeypatch):
    """NaN-poisoned weights of an expert that no token routes to must not leak
    (reference tests/test_op1.py:162-170)."""
    _say(f"nan poison {path}")
    _force_path(monkeypatch, path)
    m = _op1()
    g = torch.Generator().manual_seed(1234)
    x, w1, w2, w3, router, _ = make_moe_inputs(64, 8, 256, 512, g, dtype=torch.float32)
    x[:, 0] = x[:, 0].abs() + 1.0
    router[7].zero_()
    router[7, 0] = -100.0
    w1[7] = float("nan")
    w3[7] = float("nan")
    w2[7] = float("nan")
    args = [a.to(torch.bfloat16).cuda() for a in (x, w1, w2, w3, router)]
    out = m.tree_moe_forward(*args, torch.ones(64, device="cuda"), 7)
    assert not out.isnan().any()


def _check_excluded_gates(routing, ids, gates_before, cold, info):
    """As the reference's exclude_experts does (op1_tree_moe.py:630), the
    excluded slots' gates are zero in gates_flat afterwards, every other gate
    is unchanged, and the returned host gates are the values from before."""
    cold_mask = torch.isin(ids, torch.tensor(cold, device=ids.device))
    after = routing.gates_flat
    assert bool((after[cold_mask] == 0).all())
    assert torch.equal(after[~cold_mask], gates_before[~cold_mask])
    for e, toks, gts in info:
        slots = (ids == e).nonzero().flatten()
        assert torch.equal(gts, gates_before[slots].float().cpu())
        assert torch.equal(toks, (slots // 2).cpu())


def test_exclude_experts_hybrid_matches_full(monkeypatch):
    """Weight-streaming GEMMs (test_exclude_experts_tiled_path covers the tiled
    ones)."""
    _say("exclude experts")
    _force_path(monkeypatch, "stream")
    m = _op1()
    g = torch.Generator().manual_seed(23)
    x, w1, w2, w3, router, accept = make_moe_inputs(64, 8, 512, 1024, g, dtype=torch.bfloat16)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    full = m.tree_moe_forward(*dev, 4).clone()
    routing = m.route_experts(dev[0], dev[4], dev[5], 4, 1024)
    cold = routing.expert_ids()[:2]
    ids = routing.topk_ids.reshape(-1).clone()
    gates_before = routing.gates_flat.clone()
    info = routing.exclude_experts(cold)
    assert [e for e, _, _ in info] == cold
    assert not set(routing.expert_ids()) & set(cold)
    _check_excluded_gates(routing, ids, gates_before, cold, info)
    hybrid = m.tree_moe_forward(*dev, 4, routing=routing).float().cpu()
    for e, toks, gts in info:
        xe = x[toks].double()
        y = (torch.nn.functional.silu(xe @ w1[e].double().t()) * (xe @ w3[e].double().t())) \
            @ w2[e].double().t()
        hybrid.index_add_(0, toks, (gts.double().unsqueeze(1) * y).float())
    torch.testing.assert_close(hybrid, full.float().cpu(), rtol=2e-2, atol=5e-2)


@pytest.mark.parametrize("t,budget,objective", [(512, 8, "mass"), (512, 2, "critical_path"),
                                                (300, 4, "mass"), (1024, 3, "critical_path")])
def test_tiled_gemms_match_fp64_golden(t, budget, objective):
    """At >= 128 rows per routed expert the MFMA-tiled GEMMs run; expert row
    counts that are not multiples of 128 (and unrouted experts) included."""
    _say(f"tiled t={t} B={budget} {objective}")
    m = _op1()
    assert m.uses_tiled_gemms(t, budget, 8)
    out, golden, _, _ = _forward_and_golden(t, 8, 512, 1024, budget, 31 + t, objective)
    err = op1_ref.rel_l2(out.cpu().float(), golden)
    _say(f"  rel_l2={err:.3e}")
    assert err <= REL_L2_TOL


def test_tiled_gemms_skewed_expert():
    """One expert takes every token (several 128-row tiles plus a ragged one)."""
    _say("tiled skewed")
    m = _op1()
    t, e, h, i = 700, 8, 512, 1024
    g = torch.Generator().manual_seed(41)
    x, w1, w2, w3, router, accept = make_moe_inputs(t, e, h, i, g, dtype=torch.float32)
    x[:, 0] = 1.0
    router[:, 0] = 0.0
    router[5, 0] = 40.0
    args = [a.to(torch.bfloat16) for a in (x, w1, w2, w3, router)]
    dev = [a.cuda() for a in args] + [accept.cuda()]
    out = m.tree_moe_forward(*dev, 8)
    gates = oracle_c.router_gates(bf16_bits(args[0]), bf16_bits(args[4]))
    ref = oracle_c.route_bucket(gates, accept.numpy(), 8)
    assert np.sum(ref.topk_ids == 5) == t
    golden = op1_ref.expert_ffn_golden(args[0], args[1], args[2], args[3],
                                       torch.from_numpy(ref.topk_ids).view(t, 2),
                                       torch.from_numpy(ref.gates_flat).view(t, 2))
    assert op1_ref.rel_l2(out.cpu().float(), golden) <= REL_L2_TOL


def test_tiled_and_streaming_gemms_agree(monkeypatch):
    _say("tiled vs streaming")
    m = _op1()
    g = torch.Generator().manual_seed(43)
    x, w1, w2, w3, router, accept = make_moe_inputs(512, 8, 1024, 2048, g, dtype=torch.bfloat16)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    assert m.uses_tiled_gemms(512, 8, 8)
    tiled = m.tree_moe_forward(*dev, 8).clone()
    again = m.tree_moe_forward(*dev, 8)
    assert torch.equal(tiled, again)
    monkeypatch.setattr(m, "TILED_MIN_ROWS", 1 << 30)
    monkeypatch.setattr(m, "TILED_MIN_ROWS_WIDE", 1 << 30)
    assert not m.uses_tiled_gemms(512, 8, 8, 2048)
    streaming = m.tree_moe_forward(*dev, 8)
    assert op1_ref.rel_l2(tiled.float().cpu(), streaming.float().cpu()) <= 5e-3


@pytest.mark.parametrize("t,e,i,budget", [(256, 8, 1792, 8), (100, 16, 1280, 6), (64, 8, 1792, 4)])
def test_tiled_gemms_ragged_column_blocks(t, e, i, budget, monkeypatch):
    """Column blocks that do not divide evenly among the 8 XCDs (I / 128 = 14
    or 10 blocks, so some launch indices map to no job) on the MFMA-tiled
    GEMMs, with 8 and 16 experts: the layer meets the fp64 golden."""
    _say(f"tiled ragged columns t={t} E={e} I={i} B={budget}")
    _force_path(monkeypatch, "tiled")
    out, golden, _, _ = _forward_and_golden(t, e, 512, i, budget, 71 + t)
    err = op1_ref.rel_l2(out.cpu().float(), golden)
    _say(f"  rel_l2={err:.3e}")
    assert err <= REL_L2_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_tiled_gate_up_partial_tiles(dtype):
    """The 256-row gate/up tile on a hand-made layout whose experts end in
    tiles of 1, 100, 150, 250 and 11 rows (1, 2, 3, 4 and 1 of the 64-row
    parts run their MFMAs): every sorted row of h meets a float32 torch
    evaluation of silu(x w1^T) * (x w3^T), and no row past the slots is
    written."""
    from treemoe_spec_amd import _capi

    _say(f"tiled gate/up partial tiles {dtype}")
    t, h, i = 1024, 512, 1024
    counts = [257, 356, 150, 250, 1035]  # 2T slots over E = 5 experts: 2T >= 384 E
    e = len(counts)
    assert sum(counts) == 2 * t and 2 * t >= 384 * e
    g = torch.Generator().manual_seed(97)
    x = torch.randn(t, h, generator=g).to(dtype)
    w1 = (torch.randn(e, i, h, generator=g) * 0.05).to(dtype)
    w3 = (torch.randn(e, i, h, generator=g) * 0.05).to(dtype)
    slots = torch.randperm(2 * t, generator=g).to(torch.int32)
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    tiles = []
    for k, c in enumerate(counts):
        for r0 in range(0, c, 64):
            tiles.append([k, offsets[k] + r0, min(64, c - r0), 0])
    dev = torch.device("cuda")
    xd, w1d, w3d = x.to(dev), w1.to(dev), w3.to(dev)
    slots_d = slots.to(dev)
    offsets_d = torch.tensor(offsets, dtype=torch.int32, device=dev)
    tiles_d = torch.tensor(tiles, dtype=torch.int32, device=dev)
    # one spare row past the 2T slots: it must keep its fill value
    hd = torch.full((2 * t + 1, i), 7.0, dtype=dtype, device=dev)
    code = _capi.TM_DTYPE_F16 if dtype == torch.float16 else _capi.TM_DTYPE_BF16
    _capi.call("tm_op1_prefill_gemm1", xd.data_ptr(), w1d.data_ptr(), w3d.data_ptr(),
               hd.data_ptr(), slots_d.data_ptr(), offsets_d.data_ptr(), tiles_d.data_ptr(),
               len(tiles), t, h, i, e, code, _capi.stream_of(dev))
    torch.cuda.synchronize()
    out = hd.float().cpu()
    assert torch.all(out[2 * t] == 7.0)
    xf, w1f, w3f = x.float(), w1.float(), w3.float()
    for k, c in enumerate(counts):
        rows = slice(offsets[k], offsets[k + 1])
        tok = slots[rows].long() >> 1
        a = xf[tok] @ w1f[k].T
        b = xf[tok] @ w3f[k].T
        ref = (a / (1.0 + torch.exp(-a))) * b
        err = (out[rows] - ref).norm() / ref.norm()
        worst = ((out[rows] - ref).abs().amax(1) / ref.abs().amax(1)).max()
        _say(f"  expert {k} rows {c}: rel_l2={err:.2e} worst row {worst:.2e}")
        assert err <= 1e-2 and worst <= 2e-2


def test_tiled_down_gemm_segment_counts_agree(monkeypatch):
    """The tiled path at a small shape takes 4 K segments for the down GEMM;
    forced back to 2 it must give the same layer up to fp32 summation order,
    and both must meet the fp64 golden."""
    _say("tiled down GEMM, 2 vs 4 K segments")
    m = _op1()
    _force_path(monkeypatch, "tiled")
    out4, golden, inputs, _ = _forward_and_golden(64, 8, 512, 1024, 4, 21)
    ws = next(w for k, w in m._ws_cache.items() if k[:4] == (64, 8, 512, 1024))
    assert m._tiled_split(64, 4, 8, 512, 1024, ws) == 4
    assert op1_ref.rel_l2(out4.cpu().float(), golden) <= REL_L2_TOL
    monkeypatch.setattr(m, "TILED_SPLIT_WIDE", 2)
    dev = [a.cuda() for a in inputs]
    out2 = m.tree_moe_forward(*dev, 4)
    assert op1_ref.rel_l2(out2.cpu().float(), golden) <= REL_L2_TOL
    assert op1_ref.rel_l2(out2.float().cpu(), out4.float().cpu()) <= 2e-3


def test_exclude_experts_tiled_path():
    _say("exclude experts, tiled")
    m = _op1()
    t, budget = 512, 4
    g = torch.Generator().manual_seed(47)
    x, w1, w2, w3, router, accept = make_moe_inputs(t, 8, 512, 1024, g, dtype=torch.bfloat16)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    assert m.uses_tiled_gemms(t, budget, 8)
    full = m.tree_moe_forward(*dev, budget).clone()
    routing = m.route_experts(dev[0], dev[4], dev[5], budget, 1024)
    cold = routing.expert_ids()[:2]
    ids = routing.topk_ids.reshape(-1).clone()
    gates_before = routing.gates_flat.clone()
    info = routing.exclude_experts(cold)
    _check_excluded_gates(routing, ids, gates_before, cold, info)
    hybrid = m.tree_moe_forward(*dev, budget, routing=routing).float().cpu()
    for e, toks, gts in info:
        xe = x[toks].double()
        y = (torch.nn.functional.silu(xe @ w1[e].double().t()) * (xe @ w3[e].double().t())) \
            @ w2[e].double().t()
        hybrid.index_add_(0, toks, (gts.double().unsqueeze(1) * y).float())
    torch.testing.assert_close(hybrid, full.float().cpu(), rtol=2e-2, atol=5e-2)


def _torch_fp32_golden(inp, ids, wts):
    """Same expert FFN in fp32 torch on the GPU (hipBLASLt), for full shapes."""
    x = inp.x.float()
    out = torch.zeros_like(x)
    t = x.shape[0]
    ids = ids.view(t, 2).cuda()
    wts = wts.view(t, 2).cuda()
    for e in range(inp.w1.shape[0]):
        sel = ids == e
        rows = sel.any(1).nonzero().flatten()
        if rows.numel() == 0:
            continue
        gate = (wts * sel.float()).sum(1)[rows]
        xe = x[rows]
        h = torch.nn.functional.silu(xe @ inp.w1[e].float().t()) * (xe @ inp.w3[e].float().t())
        out[rows] += (h @ inp.w2[e].float().t()) * gate.unsqueeze(1)
    return out


@pytest.mark.parametrize("name", ["config2_mixtral_t64_b8", "config3_mixtral_t64_b4_skew",
                                  "config5_mixtral_t2048_zipf"])
def test_mixtral_shape_configs(name):
    _say(f"mixtral {name}")
    from treemoe_spec_amd.workloads import op1_workload

    m = _op1()
    inp = op1_workload(name, device="cuda")
    out = m.tree_moe_forward(inp.x, inp.w1, inp.w2, inp.w3, inp.router, inp.accept,
                             inp.budget)
    routing = m.route_experts(inp.x, inp.router, inp.accept, inp.budget, inp.w1.shape[1])
    gates = oracle_c.router_gates(bf16_bits(inp.x), bf16_bits(inp.router))
    ref = oracle_c.route_bucket(gates, inp.accept.cpu().numpy(), inp.budget)
    assert np.array_equal(routing.topk_ids.reshape(-1).cpu().numpy(), ref.topk_ids)
    assert np.array_equal(routing.gates_flat.cpu().numpy().view(np.uint32),
                          ref.gates_flat.view(np.uint32))
    if inp.budget < 8:
        assert len(routing.expert_ids()) <= inp.budget
    golden = _torch_fp32_golden(inp, torch.from_numpy(ref.topk_ids),
                                torch.from_numpy(ref.gates_flat))
    err = op1_ref.rel_l2(out.float(), golden)
    _say(f"  rel_l2={err:.3e}")
    assert err <= REL_L2_TOL
    again = m.tree_moe_forward(inp.x, inp.w1, inp.w2, inp.w3, inp.router, inp.accept,
                               inp.budget)
    assert torch.equal(out, again)


def test_reference_cpu_config_shape():
    """The reference's CPU-runnable case (T=64, hidden 1024, FFN 3584, E=8,
    top-2, no budget pruning; the configuration its treemoe/ref path is timed
    on) run on the GPU: routing bit-exact against the C oracle, the output
    within rel-L2 1e-2 of the fp64 CPU expert FFN, and deterministic."""
    _say("reference CPU config shape on the GPU")
    from treemoe_spec_amd.workloads import op1_workload

    m = _op1()
    inp = op1_workload("config1_cpu_small", device="cuda")
    out = m.tree_moe_forward(inp.x, inp.w1, inp.w2, inp.w3, inp.router, inp.accept,
                             inp.budget)
    gates = oracle_c.router_gates(bf16_bits(inp.x), bf16_bits(inp.router))
    ref = oracle_c.route_bucket(gates, inp.accept.cpu().numpy(), inp.budget)
    routing = m.route_experts(inp.x, inp.router, inp.accept, inp.budget, inp.w1.shape[1])
    assert np.array_equal(routing.topk_ids.reshape(-1).cpu().numpy(), ref.topk_ids)
    golden = op1_ref.expert_ffn_golden(inp.x.cpu(), inp.w1.cpu(), inp.w2.cpu(), inp.w3.cpu(),
                                       torch.from_numpy(ref.topk_ids),
                                       torch.from_numpy(ref.gates_flat))
    err = op1_ref.rel_l2(out.double().cpu(), golden)
    _say(f"  rel_l2={err:.3e}")
    assert err <= REL_L2_TOL
    assert torch.equal(out, m.tree_moe_forward(inp.x, inp.w1, inp.w2, inp.w3, inp.router,
                                               inp.accept, inp.budget))


def test_rejects_cpu_tensors_and_bad_dtypes():
    m = _op1()
    g = torch.Generator().manual_seed(0)
    x, w1, w2, w3, router, accept = make_moe_inputs(16, 8, 256, 256, g, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm"):
        m.tree_moe_forward(x, w1, w2, w3, router, accept, 8)
    with pytest.raises(TypeError):
        m.tree_moe_forward(x.float().cuda(), w1.cuda(), w2.cuda(), w3.cuda(), router.cuda(),
                           accept.cuda(), 8)
