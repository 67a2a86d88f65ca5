"""CPU: pin the op4 oracle (argmax, greedy walk, KV commit).

Known answers from the reference's tests (tests/test_op4.py:24-67,
tests/test_kernel_semantics.py:135-172, tests/test_interpret.py:152-185),
numpy.argmax as the closed-form argmax, brute-force byte comparison of the
commit, and the C walk against the torch restatement of verify_ref.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import op4_ref, oracle_c
from tests.conftest import bf16_bits


def chain_tree(tokens):
    n = len(tokens)
    parent = torch.tensor([-1] + list(range(n - 1)))
    children = [[i + 1] for i in range(n - 1)] + [[]]
    return torch.tensor(tokens), parent, children


def make_logits(n, v, winners):
    lg = torch.zeros(n, v)
    for i, w in enumerate(winners):
        lg[i, w] = 10.0
    return lg


def _both(logits, tokens, children, max_depth=64):
    ref = op4_ref.tree_verify(logits, torch.zeros_like(logits), tokens, children)
    am = oracle_c.argmax(logits.float().numpy())
    c = oracle_c.greedy_walk(am, tokens.numpy(), children, max_depth)
    assert c[3] == ref[3] and c[2] == ref[2]
    assert np.array_equal(c[0], ref[0].numpy()) and np.array_equal(c[1], ref[1].numpy())
    return ref


def test_greedy_accepts_matching_chain():
    tokens, _, children = chain_tree([5, 7, 9, 11])
    slots, toks, bonus, num = _both(make_logits(4, 32, [7, 9, 11, 13]), tokens, children)
    assert num == 3 and toks[:3].tolist() == [7, 9, 11] and bonus == 13


def test_greedy_stops_at_first_mismatch():
    tokens, _, children = chain_tree([5, 7, 999, 11])
    slots, toks, bonus, num = _both(make_logits(4, 32000, [7, 9, 11, 13]), tokens, children)
    assert num == 1 and bonus == 9


def test_greedy_picks_matching_branch():
    tokens = torch.tensor([5, 8, 7])
    children = [[1, 2], [], []]
    slots, _, bonus, num = _both(make_logits(3, 32, [7, 0, 4]), tokens, children)
    assert num == 1 and int(slots[0]) == 2 and bonus == 4


def test_sampling_mode_with_injected_uniforms():
    """Reference tests/test_op4.py:54-67 (torch restatement only)."""
    tokens, _, children = chain_tree([5, 7, 9])
    logits = make_logits(3, 32, [7, 9, 11])
    q = torch.full((3, 32), 1.0 / 32)
    res = op4_ref.tree_verify(logits, q, tokens, children, temperature=1.0,
                              uniforms=torch.zeros(3), generator=torch.Generator().manual_seed(0))
    assert res[3] == 2
    res = op4_ref.tree_verify(logits, q, tokens, children, temperature=1.0,
                              uniforms=torch.ones(3), generator=torch.Generator().manual_seed(0))
    assert res[3] == 0


def test_all_negative_logits():
    """Regression KAT tests/test_kernel_semantics.py:157-172 (-inf init)."""
    tokens = torch.tensor([0, 5, 2])
    children = [[1], [2], []]
    logits = torch.full((3, 8), -10.0)
    logits[0, 5] = -1.5
    logits[1, 2] = -2.0
    logits[2, 7] = -3.0
    _, _, bonus, num = _both(logits, tokens, children, 6)
    assert num == 2 and bonus == 7


@pytest.mark.parametrize("seed", range(20))
def test_walk_random_trees(seed):
    """tests/test_kernel_semantics.py:135-154 pattern, full-accept every 3rd."""
    from treemoe_spec_amd.workloads import random_tree

    g = torch.Generator().manual_seed(seed)
    n, v = 16, 64
    _, children, tokens, _ = random_tree(g, n, None, v)
    logits = torch.randn(n, v, generator=g)
    if seed % 3 == 0:
        for node in range(n):
            if children[node]:
                logits[node, tokens[children[node][0]]] += 100.0
    _both(logits, tokens, children)


def test_walk_depth_bound():
    tokens, _, children = chain_tree(list(range(3, 13)))
    logits = make_logits(10, 64, list(range(4, 14)))
    am = oracle_c.argmax(logits.numpy())
    for md in (0, 1, 5, 9, 12):
        _, _, bonus, num, root = oracle_c.greedy_walk(am, tokens.numpy(), children, md)
        assert num == min(md, 9) and root == num and bonus == int(am[root])


def test_argmax_matches_numpy_with_ties_nan_inf():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(12, 777, generator=g) * 4)
    x[0, 10] = x[0, 500] = x[0].max() + 1       # tie: first wins
    x[1] = -float("inf")                        # all -inf -> 0
    x[2, 300] = float("nan")                    # NaN ranks first
    x[2, 100] = float("nan")
    x[3] = -x[3].abs() - 1                      # all negative
    x[4, 5] = float("inf")
    x[4, 6] = float("inf")
    for dtype in (torch.float32, torch.bfloat16):
        xd = x.to(dtype)
        if dtype == torch.float32:
            got = oracle_c.argmax(xd.numpy())
        else:
            got = oracle_c.argmax(bf16_bits(xd), bf16_bits=True)
        assert np.array_equal(got, np.argmax(xd.float().numpy(), axis=1))
        assert np.array_equal(got, xd.float().argmax(1).numpy())


@pytest.mark.parametrize("page", [16, 64, 8])
def test_kv_commit_c_equals_torch_restatement(page):
    g = torch.Generator().manual_seed(page)
    L, kvh, hd, n = 3, 2, 8, 64
    n_scratch = (n + page - 1) // page
    pages = n_scratch + 40
    k = torch.randn(L, pages, page, kvh, hd, generator=g).to(torch.bfloat16)
    v = torch.randn(L, pages, page, kvh, hd, generator=g).to(torch.bfloat16)
    scratch = list(range(n_scratch))
    table = (torch.randperm(pages - n_scratch, generator=g) + n_scratch).tolist()
    seq_len = 37
    accepted = torch.full((n,), -1, dtype=torch.long)
    path = [3, 17, 40, 63, 22]
    accepted[: len(path)] = torch.tensor(path)
    kt, vt = k.clone(), v.clone()
    m = op4_ref.commit_tree(kt, vt, torch.cat([torch.zeros(1, dtype=torch.long), accepted]),
                            scratch, table, seq_len)
    assert m == len(path) + 1
    kc = k.contiguous().view(torch.int16).numpy().copy()
    vc = v.contiguous().view(torch.int16).numpy().copy()
    oracle_c.kv_commit(kc, vc, accepted.numpy(), len(path), np.array(scratch),
                       np.array(table), seq_len)
    assert np.array_equal(kc, kt.view(torch.int16).numpy())
    assert np.array_equal(vc, vt.view(torch.int16).numpy())
    # brute force: every committed row equals its source row, nothing else moved
    src = [0] + path
    for j, s in enumerate(src):
        q = seq_len + j
        dst = kt[:, table[q // page], q % page]
        assert torch.equal(dst, k[:, scratch[s // page], s % page])
    changed = (kt != k).any(-1).any(-1).any(0)
    rows = {(table[(seq_len + j) // page], (seq_len + j) % page) for j in range(len(src))}
    for p, o in changed.nonzero().tolist():
        assert (p, o) in rows
