"""CPU: pin the op1/op3 oracle.

Checks come from the reference's own known-answer tests
(tests/test_op1.py, tests/test_kernel_semantics.py), from invariants of the
layout, from brute force on tiny inputs, and from closed forms (e^x against
libm, bf16 rounding against an FP64 dot product).  Two restatements are
compared against each other: the C oracle (fixed-order fp32, the bits the
device must produce) and the torch restatement of treemoe/ref.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import op1_ref, oracle_c
from tests.conftest import bf16_bits, make_moe_inputs

N, E, H, I = 64, 8, 64, 128


def _gates(rng, n=N, e=E):
    return torch.softmax(torch.randn(n, e, generator=rng), dim=-1)


def _route(gates, accept, budget, tau=0.05, objective="mass", block_m=16):
    return oracle_c.route_bucket(np.asarray(gates, np.float32), np.asarray(accept, np.float32),
                                 budget, tau=tau, objective=objective, block_m=block_m)


# ------------------------------------------------------------- e^x, router --

def test_expf_within_two_ulp_of_libm():
    xs = np.concatenate([np.linspace(-79.9, 0.0, 20001, dtype=np.float32),
                         -np.logspace(-8, 1.9, 2001).astype(np.float32),
                         np.array([0.0, -0.0, -1e-30, -0.34657359, -0.34657360], np.float32)])
    got = oracle_c.expf_array(xs).astype(np.float64)
    exact = np.exp(xs.astype(np.float64))
    ulp = np.spacing(exact.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - exact) / ulp) <= 2.0
    assert oracle_c.expf(0.0) == 1.0
    assert oracle_c.expf(-80.0) == 0.0 and oracle_c.expf(-1000.0) == 0.0


def test_router_logits_are_bf16_rounded_fp64_dot(rng):
    """Each gate row must be the softmax of bf16-rounded dot products: the
    logit recovered from the gates' ratios matches the FP64 dot product to
    one bf16 ulp, and gates match torch's softmax(F.linear) to 1e-6."""
    x = torch.randn(16, 256, generator=rng).to(torch.bfloat16)
    w = (torch.randn(8, 256, generator=rng) * 0.1).to(torch.bfloat16)
    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(w))
    ref = op1_ref.router_gates(x, w).numpy()
    np.testing.assert_allclose(gates, ref, rtol=2e-6, atol=1e-7)
    assert np.allclose(gates.sum(1), 1.0, atol=1e-6)
    exact = (x.double() @ w.double().t()).numpy()
    logit_gap = np.log(gates.astype(np.float64)) - np.log(gates[:, :1].astype(np.float64))
    exact_gap = exact - exact[:, :1]
    bf16_ulp = 2.0 ** (np.floor(np.log2(np.abs(exact) + 1e-30)) - 7)
    tol = bf16_ulp + bf16_ulp[:, :1] + 1e-5
    assert np.all(np.abs(logit_gap - exact_gap) <= tol)


def test_f16_rounding_matches_numpy():
    """The oracle's fp32 -> fp16 rounding (fp16 router logits and outputs) is
    numpy's round-to-nearest-even conversion: random magnitudes over the
    whole range, subnormals, overflow, and exact halfway cases."""
    rng = np.random.default_rng(0)
    mags = 10.0 ** rng.integers(-9, 6, 200000)
    vals = np.concatenate([
        (rng.standard_normal(200000) * mags).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e9, np.inf, -np.inf,
                  2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -25 * 1.0000001,
                  1e-30, 6.1e-5, -6.1e-5], np.float32),
        ((np.arange(1024, 2048, dtype=np.float64) + 0.5) * 2.0 ** -10).astype(np.float32),
        ((np.arange(1, 1024, dtype=np.float64) + 0.5) * 2.0 ** -24).astype(np.float32),
    ])
    got = oracle_c.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert np.isnan(oracle_c.f32_to_f16_bits(np.array([np.nan], np.float32)).view(np.float16)[0])


def test_router_logits_f16_are_rounded_dot(rng):
    """fp16 router: each logit is the fp16 rounding of the dot product (within
    one fp16 ulp of the FP64 value), the gates are the softmax of exactly
    those logits, and they agree with torch's F.linear on fp16 operands up to
    one ulp where the fp32 sums round differently."""
    x = torch.randn(16, 256, generator=rng).to(torch.float16)
    w = (torch.randn(8, 256, generator=rng) * 0.1).to(torch.float16)
    bits = oracle_c.router_logits(bf16_bits(x), bf16_bits(w), f16=True)
    logits = bits.view(np.float16).astype(np.float64)
    exact = (x.double() @ w.double().t()).numpy()
    ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(logits - exact) <= ulp)
    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(w), f16=True)
    ref = torch.softmax(torch.from_numpy(logits).float(), -1).numpy()
    np.testing.assert_allclose(gates, ref, rtol=2e-6, atol=1e-7)
    torch_logits = torch.nn.functional.linear(x, w).double().numpy()
    assert np.all(np.abs(torch_logits - logits) <= ulp)
    # a planted variant that rounds the same sums to bf16 misses the fp16 bound
    bf = oracle_c.router_logits(bf16_bits(x), bf16_bits(w)).astype(np.uint32) << 16
    assert not np.all(np.abs(bf.view(np.float32).astype(np.float64) - exact) <= ulp)


def test_router_order_is_64_lane_fold(rng):
    """A planted variant of the reduction order (plain sequential sum) must
    be distinguishable: the oracle's fold is what the device implements."""
    x = torch.randn(32, 4096, generator=rng).to(torch.bfloat16)
    w = (torch.randn(8, 4096, generator=rng) * 0.1).to(torch.bfloat16)
    xs, ws = x.float().numpy(), w.float().numpy()
    lanes = np.zeros((32, 8, 64), np.float32)
    for c in range(4096 // 8):
        for j in range(8):
            k = 8 * c + j
            lanes[:, :, c % 64] = (lanes[:, :, c % 64]
                                   + (xs[:, None, k] * ws[None, :, k]).astype(np.float32))
    v = lanes
    while v.shape[-1] > 1:
        half = v.shape[-1] // 2
        v = v[..., :half] + v[..., half:]
    logits = torch.from_numpy(v[..., 0]).to(torch.bfloat16).float()
    e = np.exp((logits - logits.max(1, keepdim=True).values).double().numpy())
    expect = (e / e.sum(1, keepdims=True)).astype(np.float32)
    gates = oracle_c.router_gates(bf16_bits(x), bf16_bits(w))
    np.testing.assert_allclose(gates, expect, rtol=1e-6, atol=1e-8)


# ------------------------------------------------------- budget routing KATs --

@pytest.mark.parametrize("budget", [2, 4, 8])
def test_budget_respected(rng, budget):
    r = _route(_gates(rng), torch.rand(N, generator=rng), budget)
    assert len(set(r.topk_ids.tolist())) <= budget
    assert np.allclose(r.gates_flat.reshape(N, 2).sum(1), 1.0, atol=1e-6)


def test_b8_is_plain_top2(rng):
    gates = _gates(rng)
    r = _route(gates, torch.ones(N), 8)
    top_g, top_i = gates.topk(2, dim=-1)
    assert torch.equal(torch.from_numpy(r.topk_ids).view(N, 2).sort(-1).values,
                       top_i.sort(-1).values)
    np.testing.assert_allclose(r.gates_flat.reshape(N, 2),
                               (top_g / top_g.sum(-1, keepdim=True)).numpy(), atol=1e-6)


def test_low_accept_degrades_to_top1(rng):
    r = _route(_gates(rng), torch.zeros(N), 8)
    w = r.gates_flat.reshape(N, 2)
    assert np.all(w[:, 0] == 1.0) and np.all(w[:, 1] == 0.0)


def test_critical_path_protects_root_against_fringe_mass():
    """Reference KAT tests/test_op1.py:45-65."""
    gates = np.array([[0.40, 0.35, 0.15, 0.10],
                      [0.05, 0.05, 0.50, 0.40],
                      [0.05, 0.05, 0.50, 0.40],
                      [0.05, 0.05, 0.50, 0.40]], np.float32)
    accept = np.array([1.0, 0.8, 0.8, 0.8], np.float32)
    mass = _route(gates, accept, 2, tau=0.0, objective="mass")
    crit = _route(gates, accept, 2, tau=0.0, objective="critical_path")
    assert set(mass.topk_ids.tolist()) == {2, 3}
    assert set(crit.topk_ids.tolist()) == {0, 1}
    assert set(crit.topk_ids[:2].tolist()) == {0, 1}
    for objective in ("mass", "critical_path"):
        ids, _ = op1_ref.budget_route(torch.from_numpy(gates), torch.from_numpy(accept), 2,
                                      top1_threshold=0.0, routing_objective=objective)
        expect = {2, 3} if objective == "mass" else {0, 1}
        assert set(ids.unique().tolist()) == expect


def test_critical_path_b8_is_lossless(rng):
    gates = _gates(rng)
    r = _route(gates, torch.rand(N, generator=rng), 8, tau=0.0, objective="critical_path")
    top_g, top_i = gates.topk(2, dim=-1)
    assert torch.equal(torch.from_numpy(r.topk_ids).view(N, 2), top_i)
    np.testing.assert_allclose(r.gates_flat.reshape(N, 2),
                               (top_g / top_g.sum(-1, keepdim=True)).numpy(), rtol=1e-6)


def test_critical_path_ignores_degraded_second_slot():
    """Reference KAT tests/test_op1.py:83-95."""
    gates = np.array([[0.40, 0.35, 0.15, 0.10],
                      [0.05, 0.05, 0.50, 0.40]], np.float32)
    accept = np.array([1.0, 0.01], np.float32)
    r = _route(gates, accept, 2, tau=0.05, objective="critical_path")
    assert set(r.topk_ids[:2].tolist()) == {0, 1}
    assert r.gates_flat[2:].tolist() == [1.0, 0.0]


def test_contract_errors():
    gates = torch.full((2, 4), 0.25)
    with pytest.raises(ValueError, match="expert_budget"):
        op1_ref.budget_route(gates, torch.ones(2), 1)
    with pytest.raises(ValueError, match="routing_objective"):
        op1_ref.budget_route(gates, torch.ones(2), 2, routing_objective="unknown")


def _brute_force(gates, accept, budget, tau, objective):
    """Exhaustive restatement with Python sorting on tiny inputs."""
    n, e = gates.shape
    g = gates.astype(np.float64)
    demand = [sum(float(accept[t]) * g[t, k] for t in range(n)) for k in range(e)]
    if objective == "critical_path":
        crit = [-math.inf] * e
        for t in range(n):
            order = sorted(range(e), key=lambda k: (-g[t, k], k))
            crit[order[0]] = max(crit[order[0]], float(accept[t]))
            if accept[t] >= tau:
                crit[order[1]] = max(crit[order[1]], float(accept[t]))
        order = sorted(range(e), key=lambda k: (-crit[k], -demand[k], k))
    else:
        order = sorted(range(e), key=lambda k: (-demand[k], k))
    keep = set(order[:budget])
    ids = []
    for t in range(n):
        masked = [(g[t, k] if k in keep else 0.0) for k in range(e)]
        o = sorted(range(e), key=lambda k: (-masked[k], k))
        ids.extend(o[:2])
    return ids


@pytest.mark.parametrize("seed", range(40))
def test_brute_force_tiny(seed):
    g = torch.Generator().manual_seed(seed)
    n, e = int(torch.randint(1, 9, (1,), generator=g)), int(torch.randint(2, 7, (1,), generator=g))
    budget = int(torch.randint(2, e + 1, (1,), generator=g))
    gates = torch.softmax(torch.randn(n, e, generator=g) * 2, -1).numpy()
    accept = torch.rand(n, generator=g).numpy()
    for objective in ("mass", "critical_path"):
        r = _route(gates, accept, budget, objective=objective)
        assert r.topk_ids.tolist() == _brute_force(gates, accept, budget, 0.05, objective)


@pytest.mark.parametrize("seed", range(10))
@pytest.mark.parametrize("budget", [2, 4, 8])
def test_oracle_matches_torch_restatement(seed, budget):
    """C oracle vs the reference's torch algorithm on identical gates: same
    expert ids except an order swap at exactly tied gates."""
    g = torch.Generator().manual_seed(100 + seed)
    gates = _gates(g)
    accept = torch.rand(N, generator=g)
    for objective in ("mass", "critical_path"):
        r = _route(gates, accept, budget, objective=objective)
        ids, w = op1_ref.budget_route(gates, accept, budget, routing_objective=objective)
        got = torch.from_numpy(r.topk_ids).view(N, 2)
        for t in (got != ids).any(1).nonzero().flatten().tolist():
            a, b = got[t].tolist()
            assert ids[t].tolist() == [b, a] and gates[t, a] == gates[t, b]
        np.testing.assert_allclose(r.gates_flat.reshape(N, 2), w.numpy(), rtol=1e-6)
        demand = (accept.unsqueeze(1) * gates).sum(0).numpy()
        np.testing.assert_allclose(r.demand, demand, rtol=1e-5)


# ---------------------------------------------------------------- bucketing --

def test_offsets_and_dfs_stability(rng):
    r = _route(_gates(rng), torch.rand(N, generator=rng), 8)
    assert r.expert_offsets[-1] == 2 * N
    for e in range(E):
        seg = r.sorted_slots[r.expert_offsets[e]:r.expert_offsets[e + 1]]
        assert np.all(r.topk_ids[seg] == e)
        assert np.all(np.diff(seg // 2) >= 0)
    assert np.array_equal(r.sorted_slots[r.slot_pos], np.arange(2 * N))


def test_all_tokens_on_two_experts(rng):
    """Reference tests/test_op1.py:121-134: router forcing experts {0, 1}."""
    x, _, _, _, router, _ = make_moe_inputs(N, E, H, I, rng)
    x[:, 0] = x[:, 0].abs() + 1.0
    router.zero_()
    router[0, 0] = 2.0
    router[1, 0] = 1.0
    xb, rb = x.to(torch.bfloat16), router.to(torch.bfloat16)
    gates = oracle_c.router_gates(bf16_bits(xb), bf16_bits(rb))
    r = _route(gates, np.ones(N), 8)
    off = r.expert_offsets
    assert off[1] - off[0] == N and off[2] - off[1] == N and off[2] == off[-1]
    assert r.tiles[0].tolist() == [0, 0, N, 0] and r.tiles[1].tolist() == [1, N, N, 0]


@pytest.mark.parametrize("budget", [2, 4, 8])
@pytest.mark.parametrize("block_m", [16, 32])
def test_padded_layout_matches_reference_composition(rng, budget, block_m):
    r = _route(_gates(rng), torch.rand(N, generator=rng), budget, block_m=block_m)
    padded, blk, s2r = op1_ref.padded_layout(torch.from_numpy(r.topk_ids), E, r.max_blocks,
                                              block_m)
    assert np.array_equal(r.padded_slots, padded.numpy())
    assert np.array_equal(r.block_expert_ids, blk.numpy())
    assert np.array_equal(r.slot_to_row, s2r.numpy())
    assert np.array_equal(r.padded_slots[r.slot_to_row], np.arange(2 * N))


def test_block_expert_ids_monotone_with_masked_suffix(rng):
    r = _route(_gates(rng), torch.rand(N, generator=rng), 4)
    prev = -1
    for b in range(r.max_blocks):
        rows = r.padded_slots[b * 16:(b + 1) * 16]
        if r.block_expert_ids[b] < 0:
            assert np.all(rows == -1)
        else:
            assert r.block_expert_ids[b] >= prev and np.any(rows >= 0)
            prev = r.block_expert_ids[b]


@pytest.mark.parametrize("budget,cap16,cap32,lim16,lim32",
                         [(2, 16, 8, 9, 5), (4, 16, 8, 11, 7), (8, 16, 16, 15, 11)])
def test_compact_capacity_and_limit_kats(budget, cap16, cap32, lim16, lim32):
    """Reference KATs tests/test_kernel_semantics.py:72-87."""
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    assert m.compact_block_capacity(128, budget, 16) == cap16
    assert m.compact_block_capacity(128, budget, 32) == cap32
    assert m.compact_block_limit(128, budget, 16) == lim16
    assert m.compact_block_limit(128, budget, 32) == lim32
    assert oracle_c.compact_block_capacity(128, budget, 16) == cap16
    assert oracle_c.compact_block_limit(128, budget, 16) == lim16


@pytest.mark.parametrize("seed", range(20))
def test_tile_list_covers_every_row_once(seed):
    g = torch.Generator().manual_seed(seed)
    n = int(torch.randint(1, 300, (1,), generator=g))
    budget = int(torch.randint(2, 9, (1,), generator=g))
    gates = torch.softmax(torch.randn(n, E, generator=g) * 3, -1)
    r = _route(gates, torch.rand(n, generator=g), budget)
    assert r.max_tiles == oracle_c.compact_block_limit(2 * n, budget, 64)
    covered = np.zeros(2 * n, np.int64)
    for e, row0, rows, _ in r.tiles.tolist():
        if e < 0:
            assert rows == 0
            continue
        assert 1 <= rows <= 64
        assert r.expert_offsets[e] <= row0 and row0 + rows <= r.expert_offsets[e + 1]
        covered[row0:row0 + rows] += 1
    assert np.all(covered == 1)


# ----------------------------------------------------- expert FFN (golden) --

def test_reference_forward_equals_naive_hf_loop_at_b8(rng):
    """Reference KAT tests/test_op1.py:139-159 (fp32)."""
    x, w1, w2, w3, router, _ = make_moe_inputs(N, E, H, I, rng)
    accept = torch.ones(N)
    out = op1_ref.tree_moe_forward(x, w1, w2, w3, router, accept, 8)
    gates = torch.softmax(torch.nn.functional.linear(x, router), -1)
    top_g, top_i = gates.topk(2, -1)
    top_g = top_g / top_g.sum(-1, keepdim=True)
    naive = torch.zeros_like(x)
    for e in range(E):
        for k in range(2):
            sel = top_i[:, k] == e
            if sel.any():
                xe = x[sel]
                h = torch.nn.functional.silu(xe @ w1[e].t()) * (xe @ w3[e].t())
                naive[sel] += (h @ w2[e].t()) * top_g[sel, k:k + 1]
    torch.testing.assert_close(out, naive, rtol=1e-4, atol=1e-5)
    golden = op1_ref.expert_ffn_golden(x, w1, w2, w3, top_i, top_g)
    torch.testing.assert_close(golden.float(), naive, rtol=1e-4, atol=1e-5)


def test_golden_detects_dropped_gate_term(rng):
    """Planted mistake in the golden (second slot's gate ignored) must fail
    the 1e-2 rel-L2 bar used by the GPU parity tests."""
    x, w1, w2, w3, router, accept = make_moe_inputs(N, E, H, I, rng)
    ids, w, _, _ = op1_ref.route_and_bucket(x, router, torch.ones(N), 8)
    good = op1_ref.expert_ffn_golden(x, w1, w2, w3, ids, w)
    bad_w = w.clone()
    bad_w[:, 1] = 0.0
    bad = op1_ref.expert_ffn_golden(x, w1, w2, w3, ids, bad_w)
    assert op1_ref.rel_l2(bad, good) > 1e-2


def test_empty_expert_contributes_nothing(rng):
    x, w1, w2, w3, router, _ = make_moe_inputs(N, E, H, I, rng)
    x[:, 0] = x[:, 0].abs() + 1.0
    router[7].zero_()
    router[7, 0] = -100.0
    w1[7] = float("nan")
    w3[7] = float("nan")
    out = op1_ref.tree_moe_forward(x, w1, w2, w3, router, torch.ones(N), 7)
    assert not out.isnan().any()


def test_combine_order_is_k0_then_k1():
    """Fixed-order fp32 combine: ((0 + a0 + a1) + b0) + b1 differs from other
    orders for adversarial partials — the device and this oracle use the
    reference order (op1_tree_moe.py:517-528)."""
    a0, a1, b0, b1 = (np.float32(v) for v in (1e8, 1.0, -1e8, 1.0))
    ref = np.float32(np.float32(np.float32(np.float32(0) + a0) + a1) + b0) + b1
    other = np.float32(np.float32(np.float32(np.float32(0) + a0) + b0) + a1) + b1
    assert ref != other
    assert ref == np.float32(1.0)


def test_exhaustive_tiny_layouts():
    """Every assignment of 2 distinct experts per token for T=2, E=3."""
    pairs = [(a, b) for a in range(3) for b in range(3) if a != b]
    for combo in itertools.product(pairs, repeat=2):
        ids = torch.tensor([c for p in combo for c in p])
        padded, blk, s2r = op1_ref.padded_layout(ids, 3, 4, 16)
        assert torch.equal(padded[s2r], torch.arange(4))
