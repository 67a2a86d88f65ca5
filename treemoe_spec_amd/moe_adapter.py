"""The engine's MoE hook backed by the MI355X op1 path.

The reference engine calls ``moe_fn(x, lw, layer_idx)`` for every layer of
every forward (``MoEFn``, treemoe/model/mixtral.py:24) and talks to it through
three attributes: ``current_accept_prob`` (the tree's acceptance
probabilities, set per verification step, treemoe/engine/loop.py:166-168),
``current_layer_budgets`` and ``demand_observer`` (``_configure_moe``,
loop.py:60-69).  ``make_moe_fn`` builds that hook with the semantics of the
resident-weight branch of the reference adapter (benchmarks/bench_e2e.py:
482-501, 654-658): phase-1 routing with the layer's budget, the demand
handed to the observer, then the grouped GEMMs reusing that routing.  The
reference's offload, CPU-expert and tracing branches are not part of this
path (all experts are resident in HBM).
"""

from __future__ import annotations

import torch

from treemoe_spec_amd.kernels.op1_tree_moe import route_experts, tree_moe_forward


def make_moe_fn(expert_budget: int = 8, top1_threshold: float = 0.05,
                routing_objective: str = "mass", deterministic: bool = True,
                tree_size: int = 64, device="cuda"):
    """Returns ``moe_fn(x, lw, layer_idx) -> Tensor`` for ``MixtralForward``.

    ``lw`` needs ``router`` [E, H], ``w1``/``w3`` [E, I, H] and ``w2`` [E, H, I]
    (the reference's ``LayerWeights``).  Per call:
      * accept = ``moe_fn.current_accept_prob`` when it has one entry per row
        of ``x``, else ones (prefill and any other caller, bench_e2e.py:485-487);
      * budget = ``current_layer_budgets[layer_idx]`` when set, else
        ``expert_budget`` (:488-491);
      * ``demand_observer(layer_idx, routing.demand)`` when set (:502-504).
    """

    def moe_fn(x: torch.Tensor, lw, layer_idx: int) -> torch.Tensor:
        accept = moe_fn.current_accept_prob
        if accept is None or accept.shape[0] != x.shape[0]:
            accept = torch.ones(x.shape[0], device=x.device)
        budgets = moe_fn.current_layer_budgets
        budget = int(budgets[layer_idx]) if budgets is not None else expert_budget
        routing = route_experts(x, lw.router, accept, budget, inter=lw.w1.shape[1],
                                top1_threshold=top1_threshold,
                                routing_objective=routing_objective)
        observer = moe_fn.demand_observer
        if observer is not None:
            observer(layer_idx, routing.demand)
        return tree_moe_forward(x, lw.w1, lw.w2, lw.w3, lw.router, accept, budget,
                                routing=routing, deterministic=deterministic)

    moe_fn.current_accept_prob = torch.ones(tree_size, device=device)
    moe_fn.current_layer_budgets = None
    moe_fn.demand_observer = None
    return moe_fn
