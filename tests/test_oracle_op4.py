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


# ---------------- sampling: exponential race, rep penalty, distribution ----------------

@pytest.mark.parametrize("seed", range(0, 240, 8))
def test_exp_race_is_torch_multinomial(seed):
    """exp_race over empty(V).exponential_(1, g) picks torch.multinomial(p, 1, g)'s
    index from the same generator state and leaves the generator where
    multinomial leaves it (so later draws stay aligned): sizes from 1 to 70000,
    planted zeros, unnormalised rows, one-hot rows."""
    meta = torch.Generator().manual_seed(seed)
    for k in range(8):
        v = int(torch.randint(1, 70000 if k % 4 == 0 else 300, (1,), generator=meta))
        p = torch.rand(v, generator=meta) ** 3 * float(torch.rand(1, generator=meta) * 7 + 0.1)
        p[torch.rand(v, generator=meta) < 0.4] = 0.0
        if k == 5:
            p.zero_()
            p[int(torch.randint(0, v, (1,), generator=meta))] = 0.25
        if float(p.sum()) == 0.0:
            p[v // 2] = 1.0
        state = seed * 100 + k
        g1 = torch.Generator().manual_seed(state)
        want = int(torch.multinomial(p, 1, generator=g1))
        g2 = torch.Generator().manual_seed(state)
        e = torch.empty(v).exponential_(1.0, generator=g2)
        got = op4_ref.exp_race(p, e)
        assert got == want, (seed, k, v)
        assert p[got] > 0  # a zero-probability token is never drawn
        assert torch.equal(g1.get_state(), g2.get_state())


def test_exp_race_special_cases():
    e = torch.ones(6)
    # equal ratios: the lower index wins (torch.argmax's first occurrence)
    assert op4_ref.exp_race(torch.tensor([0.1, 0.0, 0.3, 0.0, 0.0, 0.3]), e) == 2
    # the ratio, not the probability, decides
    assert op4_ref.exp_race(torch.tensor([0.6, 0.4]), torch.tensor([3.0, 1.0])) == 1
    # zero probabilities lose to any positive one however small e is
    assert op4_ref.exp_race(torch.tensor([0.0, 1e-30, 0.0]), torch.tensor([1e-30, 50.0, 1e-30])) == 1
    # an all-zero row (multinomial refuses it) gives index 0
    assert op4_ref.exp_race(torch.zeros(4), torch.rand(4) + 0.5) == 0
    # NaN ratios rank above every number, the first one wins (torch.argmax)
    nan = float("nan")
    assert op4_ref.exp_race(torch.tensor([0.1, nan, 0.3, nan]), torch.ones(4)) == 1
    assert op4_ref.exp_race(torch.tensor([nan, nan]), torch.ones(2)) == 0


def test_exp_race_distribution():
    """Empirical frequencies of exp_race(p, Exp(1)) match p (6-sigma binomial)."""
    g = torch.Generator().manual_seed(5)
    p = torch.tensor([0.05, 0.0, 0.4, 0.15, 0.3, 0.1])
    trials = 20000
    e = torch.empty(trials, 6).exponential_(1.0, generator=g)
    counts = np.bincount([op4_ref.exp_race(p, e[t]) for t in range(trials)], minlength=6)
    expect = p.double().numpy() * trials
    sigma = np.sqrt(trials * p.double().numpy() * (1 - p.double().numpy())) + 1e-9
    assert counts[1] == 0
    assert np.all(np.abs(counts - expect) <= 6 * sigma)


def test_tree_verify_sampling_uses_the_reference_draws():
    """Without injected draws the oracle takes rand(N) then multinomial's
    exponentials from the generator: injecting exactly those draws gives the
    same result, and the bonus is torch.multinomial's (verify_ref.py:51, :87)."""
    v, n = 500, 9
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(n, v, generator=g) * 2
    q = torch.softmax(torch.randn(n, v, generator=g) * 2, -1)
    tokens = torch.randint(0, v, (n,), generator=g)
    children = [[1, 2], [3], [4, 5], [], [6], [7], [8], [], []]
    for seed in range(40):
        a = op4_ref.tree_verify(logits, q, tokens, children, temperature=0.9,
                                generator=torch.Generator().manual_seed(seed))
        g2 = torch.Generator().manual_seed(seed)
        u = torch.rand(n, generator=g2)
        e = torch.empty(v).exponential_(1.0, generator=g2)
        b = op4_ref.tree_verify(logits, q, tokens, children, temperature=0.9, uniforms=u,
                                bonus_exp=e)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and a[2:] == b[2:]


def test_rep_penalty_closed_form_power_of_two():
    """penalty 2 is exact in fp32: a token listed k times is x / 2**k when
    x > 0 and x * 2**k otherwise; unlisted and out-of-range tokens untouched."""
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(4, 50, generator=g) * 5
    logits[:, 7] = 0.0
    prev = torch.tensor([3, 9, 3, 3, 7, 49, -1, 50, 9])
    out = logits.clone()
    op4_ref.rep_penalty_inplace(out, prev, 2.0)
    k = np.bincount([t for t in prev.tolist() if 0 <= t < 50], minlength=50)
    scale = torch.tensor(2.0 ** k, dtype=torch.float32)
    expect = torch.where(logits > 0, logits / scale, logits * scale)
    assert torch.equal(out, expect)
    assert torch.equal(out[:, k == 0], logits[:, k == 0])


def test_rep_penalty_order_independent():
    g = torch.Generator().manual_seed(4)
    logits = (torch.randn(3, 40, generator=g) * 4).to(torch.bfloat16)
    prev = torch.randint(0, 40, (30,), generator=g)
    a, b = logits.clone(), logits.clone()
    op4_ref.rep_penalty_inplace(a, prev, 1.3)
    op4_ref.rep_penalty_inplace(b, prev.flip(0), 1.3)
    assert torch.equal(a, b)


def test_rep_penalty_bf16_rounds_every_application():
    """The reference stores each application to the bf16 tensor, so a token
    listed k times rounds k times; rounding once at the end differs."""
    g = torch.Generator().manual_seed(8)
    logits = (torch.randn(1, 4000, generator=g) * 7).to(torch.bfloat16)
    prev = torch.arange(4000).repeat(3)
    stepwise = logits.clone()
    op4_ref.rep_penalty_inplace(stepwise, prev, 1.3)
    x = logits.float()
    for _ in range(3):  # torch's own bf16 store after every step
        x = torch.where(x > 0, x / 1.3, x * 1.3).to(torch.bfloat16).float()
    assert torch.equal(stepwise.float(), x)
    once = logits.float()
    once = torch.where(once > 0, once / 1.3 / 1.3 / 1.3, once * 1.3 * 1.3 * 1.3)
    assert not torch.equal(stepwise, once.to(torch.bfloat16))


def test_tree_sampling_preserves_target_distribution():
    """Recursive rejection sampling over a root with three children whose
    tokens are drawn from their own draft distributions emits its first token
    with exactly p = softmax(logits[root] / T).  A wrong residual update (no
    clamp, no renormalisation, q of the wrong child) or a bonus drawn from p
    instead of the residual breaks the match (6-sigma binomial bound)."""
    v, temperature, trials = 6, 0.8, 6000
    g = torch.Generator().manual_seed(21)
    logits = torch.randn(4, v, generator=g) * 1.5
    q = torch.softmax(torch.randn(4, v, generator=g) * 1.5, -1)
    children = [[1, 2, 3], [], [], []]
    p = torch.softmax(logits[0] / temperature, -1).double().numpy()
    counts = np.zeros(v)
    for _ in range(trials):
        tokens = torch.zeros(4, dtype=torch.long)
        for c in (1, 2, 3):
            tokens[c] = int(torch.multinomial(q[c], 1, generator=g))
        u = torch.rand(4, generator=g)
        e = torch.empty(v).exponential_(1.0, generator=g)
        _, toks, bonus, num = op4_ref.tree_verify(logits, q, tokens, children,
                                                  temperature=temperature, uniforms=u,
                                                  bonus_exp=e)
        counts[int(toks[0]) if num else bonus] += 1
    sigma = np.sqrt(trials * p * (1 - p))
    assert np.all(np.abs(counts - trials * p) <= 6 * sigma)


def _torch_softmax_argmax(x: torch.Tensor) -> int:
    """The reference's pick: first-occurrence argmax of softmax in the row's
    dtype (probs = empty_like(logits), op4_commit.py:211)."""
    p = torch.softmax(x.float(), dim=-1).to(x.dtype).float().numpy()
    return int(np.argmax(p))


def test_softmax_argmax_planted_ties():
    """Probabilities that round equal tie, and the first index wins although
    its logit is smaller: fp32 (a 1e-9 gap at the maximum: e = 1 - 1e-9
    rounds to 1) and bf16 (a one-ulp gap at 2^-8: the bf16 probabilities
    round equal).  torch's softmax makes the same pick; the plain logit
    argmax does not."""
    from oracle import oracle_c

    x = torch.full((1, 100), -10.0)
    x[0, 5], x[0, 7] = 0.0, 1e-9
    assert int(x.argmax()) == 7
    assert oracle_c.softmax_argmax(x.numpy())[0] == 5 == _torch_softmax_argmax(x[0])
    xb = torch.full((1, 64), -3.0, dtype=torch.bfloat16)
    xb[0, 3] = 2.0 ** -8
    xb[0, 9] = 2.0 ** -8 + 2.0 ** -15
    assert float(xb[0, 9]) > float(xb[0, 3]) and int(xb.float().argmax()) == 9
    got = oracle_c.softmax_argmax(bf16_bits(xb), bf16_bits=True)[0]
    assert got == 3 == _torch_softmax_argmax(xb[0])
    # without the bf16 rounding of the probabilities the pick would be 9
    assert oracle_c.softmax_argmax(xb.float().numpy())[0] == 9
    # a row of -inf: index 0
    assert oracle_c.softmax_argmax(np.full((1, 8), -np.inf, np.float32))[0] == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_softmax_argmax_random_rows_agree_with_torch(dtype):
    """On N(0, 3) rows (config-4 logits) the oracle's pick equals torch's
    softmax pick (and here the logit argmax: no rounded ties at the top)."""
    from oracle import oracle_c

    g = torch.Generator().manual_seed(17)
    x = (torch.randn(32, 32000, generator=g) * 3).to(dtype)
    if dtype == torch.bfloat16:
        got = oracle_c.softmax_argmax(bf16_bits(x), bf16_bits=True)
    else:
        got = oracle_c.softmax_argmax(x.numpy())
    want = [_torch_softmax_argmax(x[r]) for r in range(32)]
    assert got.tolist() == want
    assert want == x.float().argmax(1).tolist()
