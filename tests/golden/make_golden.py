"""Write the committed golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

op1 (``op1_golden.npz``): T=64, E=8, H=256, I=256; seeds {1234, 7, 3};
budget {2, 4, 8} x objective {mass, critical_path} x accept {ones, U(0,1)}.
Inputs x, W_g (bf16 bits) and accept are stored; expert weights are re-drawn
from ``torch.Generator().manual_seed(seed)`` (recipe in ``weights_for``) and
pinned by a float64 checksum.  Stored outputs: router gates, expert ids, gate
weights, demand, the reference padded layout (BM16), the compact layout and
tile list, and for seed 1234 the FP64 expert-FFN output (as fp32).

op4 (``op4_golden.npz``): 20 random trees (n=16, V=64) with every third tree
given a planted full-accept path, their greedy results; one page-16 KV commit
(before/after bytes).

The fixtures were cross-checked against the reference's known-answer tests
by tests/test_oracle_op1.py and tests/test_oracle_op4.py before being written.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import op1_ref, op4_ref, oracle_c  # noqa: E402

OUT = Path(__file__).resolve().parent
T, E, H, I = 64, 8, 256, 256
SEEDS = (1234, 7, 3)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def inputs_for(seed: int):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    router = (torch.randn(E, H, generator=g) * 0.1).to(torch.bfloat16)
    accept = torch.rand(T, generator=g)
    return x, router, accept


def weights_for(seed: int):
    g = torch.Generator().manual_seed(seed + 77)
    w1 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    w3 = (torch.randn(E, I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    return w1, w2, w3


def weight_checksum(w1, w2, w3) -> float:
    return float(sum(w.double().abs().sum() for w in (w1, w2, w3)))


def op1_cases():
    for seed in SEEDS:
        for budget in (2, 4, 8):
            for objective in ("mass", "critical_path"):
                for accept_kind in ("ones", "uniform"):
                    yield seed, budget, objective, accept_kind


def make_op1() -> dict:
    data = {}
    for seed in SEEDS:
        x, router, accept = inputs_for(seed)
        data[f"s{seed}/x"] = bits(x)
        data[f"s{seed}/router"] = bits(router)
        data[f"s{seed}/accept"] = accept.numpy()
        gates = oracle_c.router_gates(bits(x), bits(router))
        data[f"s{seed}/gates"] = gates
        w = weights_for(seed)
        data[f"s{seed}/weight_checksum"] = np.array(weight_checksum(*w))
    for seed, budget, objective, accept_kind in op1_cases():
        key = f"s{seed}/B{budget}/{objective}/{accept_kind}"
        accept = data[f"s{seed}/accept"] if accept_kind == "uniform" else np.ones(T, np.float32)
        r = oracle_c.route_bucket(data[f"s{seed}/gates"], accept, budget, objective=objective)
        for field in ("topk_ids", "gates_flat", "padded_slots", "block_expert_ids",
                      "slot_to_row", "demand", "expert_offsets", "sorted_slots", "slot_pos",
                      "tiles"):
            data[f"{key}/{field}"] = getattr(r, field)
        if seed == SEEDS[0] and accept_kind == "uniform":
            x, _, _ = inputs_for(seed)
            w1, w2, w3 = weights_for(seed)
            out = op1_ref.expert_ffn_golden(x, w1, w2, w3, torch.from_numpy(r.topk_ids),
                                            torch.from_numpy(r.gates_flat))
            data[f"{key}/out_fp64_as_fp32"] = out.float().numpy()
    return data


def make_op4() -> dict:
    from treemoe_spec_amd.workloads import random_tree

    data = {}
    for seed in range(20):
        g = torch.Generator().manual_seed(500 + seed)
        parent, children, tokens, _ = random_tree(g, 16, None, 64)
        logits = torch.randn(16, 64, generator=g)
        if seed % 3 == 0:
            for node in range(16):
                if children[node]:
                    logits[node, tokens[children[node][0]]] += 100.0
        slots, toks, bonus, num = op4_ref.tree_verify(logits, None, tokens, children)
        p = f"t{seed}"
        data[f"{p}/parent"] = np.array(parent, np.int64)
        data[f"{p}/tokens"] = tokens.numpy()
        data[f"{p}/logits"] = logits.numpy()
        data[f"{p}/accepted_slots"] = slots.numpy()
        data[f"{p}/accepted_tokens"] = toks.numpy()
        data[f"{p}/bonus_num"] = np.array([bonus, num], np.int64)
    # page-16 KV commit on a small cache
    g = torch.Generator().manual_seed(99)
    L, pages, page, kvh, hd = 2, 12, 16, 2, 8
    k = torch.randn(L, pages, page, kvh, hd, generator=g).to(torch.bfloat16)
    v = torch.randn(L, pages, page, kvh, hd, generator=g).to(torch.bfloat16)
    scratch = [0, 1, 2, 3]
    table = [9, 4, 11, 6, 5]
    seq_len = 29
    accepted = torch.full((64,), -1, dtype=torch.long)
    accepted[:4] = torch.tensor([5, 33, 34, 60])
    data["kv/k_before"] = bits(k)
    data["kv/v_before"] = bits(v)
    kt, vt = k.clone(), v.clone()
    op4_ref.commit_tree(kt, vt, torch.cat([torch.zeros(1, dtype=torch.long), accepted]),
                        scratch, table, seq_len)
    data["kv/k_after"] = bits(kt)
    data["kv/v_after"] = bits(vt)
    data["kv/accepted"] = accepted.numpy()
    data["kv/scratch"] = np.array(scratch, np.int32)
    data["kv/table"] = np.array(table, np.int32)
    data["kv/seq_len"] = np.array(seq_len)
    return data


if __name__ == "__main__":
    np.savez_compressed(OUT / "op1_golden.npz", **make_op1())
    np.savez_compressed(OUT / "op4_golden.npz", **make_op4())
    for f in ("op1_golden.npz", "op4_golden.npz"):
        print(f, (OUT / f).stat().st_size, "bytes")
