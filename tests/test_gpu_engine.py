"""End to end on the GPU: greedy speculative decoding through this build's
tree attention, op1 MoE (via the engine hook) and op4 verify + KV commit
equals greedy AR decoding token for token (the reference's lossless red line,
tests/test_spec_lossless.py:58-84, 312-372, at B = 8).

The reference runs that gate in float32 with a torch MoE.  Here attention and
the MoE are bf16 kernels, and a 15-node verification forward sums its keys in
a different order than a one-node AR forward, so the two could differ in the
last bits of a logit; only an AR step whose top-2 logit margin is that small
could then decode differently.  Every kernel is bitwise deterministic and the
inputs are seeded, so each case below has one outcome: the test requires the
token sequences to be identical and reports the smallest AR margin it met.
"""

from __future__ import annotations

import pytest
import torch

from tests.engine_harness import (TinyConfig, TinyEngine, ar_generate, random_model,
                                  spec_generate)

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)


@pytest.mark.parametrize("seed", [1, 7, 42, 3, 11, 2024])
def test_spec_decode_matches_ar(seed):
    _say(f"engine spec vs AR seed={seed}")
    cfg = TinyConfig()
    model = random_model(cfg, 21)
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, cfg.vocab_size, (5,), generator=g).tolist()
    ar, margins = ar_generate(TinyEngine(cfg, model), prompt, 40)
    eng = TinyEngine(cfg, model)
    spec, steps, accepted = spec_generate(eng, prompt, 40, ar, seed)
    _say(f"  steps={steps} accepted={accepted} smallest AR top-2 margin={min(margins):.4f}")
    assert spec == ar, (next(i for i, (a, b) in enumerate(zip(ar, spec)) if a != b), ar, spec)
    # the planted paths were accepted: fewer steps than tokens; the cache holds
    # the prompt but its last token, then [root] + accepted path per step (the
    # last bonus token is the next root, not yet committed)
    assert accepted > 0 and steps < 40
    assert eng.kv.seq_len == len(prompt) - 1 + steps + accepted


def test_moe_hook_contract():
    """Accept probabilities, per-layer budgets and the demand observer reach the
    op1 path exactly as the engine sets them (loop.py:60-69, 166-168)."""
    _say("engine moe hook contract")
    from treemoe_spec_amd.kernels.op1_tree_moe import route_experts, tree_moe_forward
    from treemoe_spec_amd.moe_adapter import make_moe_fn

    cfg = TinyConfig()
    layers, _, _ = random_model(cfg, 3)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(12, cfg.hidden_dim, generator=g).to(torch.bfloat16).cuda()
    accept = torch.rand(12, generator=g).cuda()
    fn = make_moe_fn(expert_budget=8, tree_size=12)
    seen = []
    fn.demand_observer = lambda li, d: seen.append((li, d.clone()))
    fn.current_accept_prob = accept
    fn.current_layer_budgets = torch.tensor([8, 3])
    for li, lw in enumerate(layers):
        got = fn(x, lw, li)
        budget = [8, 3][li]
        r = route_experts(x, lw.router, accept, budget, inter=cfg.intermediate_dim)
        want = tree_moe_forward(x, lw.w1, lw.w2, lw.w3, lw.router, accept, budget)
        assert torch.equal(got, want)
        assert seen[-1][0] == li and torch.equal(seen[-1][1], r.demand)
        assert len(set(r.topk_ids.flatten().tolist())) <= budget
    # a caller whose row count differs from the tree gets acceptance 1
    x5 = x[:5].contiguous()
    fn.current_layer_budgets = None
    got = fn(x5, layers[0], 0)
    want = tree_moe_forward(x5, layers[0].w1, layers[0].w2, layers[0].w3, layers[0].router,
                            torch.ones(5, device="cuda"), 8)
    assert torch.equal(got, want)
