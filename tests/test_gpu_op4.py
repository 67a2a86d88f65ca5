"""op4 parity on the GPU: argmax, greedy walk and KV commit are bit-exact
against the oracle (C restatement and the torch restatement of
treemoe/ref/verify_ref.py / PagedKVCache.commit_tree)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle_c
from oracle import op4_ref
from tests.conftest import bf16_bits

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)


def _op4():
    from treemoe_spec_amd.kernels import op4_commit

    return op4_commit


def _tree(seed, n, vocab, max_depth=None):
    from treemoe_spec_amd.workloads import random_tree

    g = torch.Generator().manual_seed(seed)
    parent, children, tokens, depth = random_tree(g, n, max_depth, vocab)
    return g, torch.tensor(parent), children, tokens, depth


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,v", [(16, 512), (64, 32000), (3, 7), (5, 1000), (64, 32001),
                                 (6, 300001)])
def test_argmax_first_occurrence(dtype, n, v):
    _say(f"argmax {dtype} n={n} v={v}")
    op4 = _op4()
    g = torch.Generator().manual_seed(n * 7 + v)
    logits = (torch.randn(n, v, generator=g) * 3).to(dtype)
    # exact ties at an earlier index, all-negative rows, -inf rows, NaN rows
    for r in range(0, n, 3):
        j = int(logits[r].float().argmax())
        if j > 0:
            logits[r, j // 2] = logits[r, j]
    if n > 1:
        logits[1] = -(logits[1].abs() + 1)
    if n > 2:
        logits[2] = -float("inf")
    if n > 4:
        logits[4, v // 3] = float("nan")
        logits[4, v // 2] = float("nan")
    tokens = torch.zeros(n, dtype=torch.long)
    children = [[] for _ in range(n)]
    res = op4.fused_verify_commit(logits.cuda(), None, tokens.cuda(), None, children)
    got_bonus = int(res.bonus_token)
    # argmax of row 0 is the bonus of a walk that accepts nothing
    if dtype == torch.float32:
        expect = oracle_c.argmax(logits.numpy())
    else:
        expect = oracle_c.argmax(bf16_bits(logits), bf16_bits=True)
    assert got_bonus == int(expect[0])
    assert np.array_equal(expect, logits.float().argmax(-1).numpy())
    # full vector through the workspace of a direct call
    argmax = torch.empty(n, dtype=torch.int32, device="cuda")
    _direct_argmax(logits.cuda(), argmax)
    assert np.array_equal(argmax.cpu().numpy(), expect)


def _direct_argmax(logits, argmax):
    from treemoe_spec_amd import _capi
    from treemoe_spec_amd.kernels.op4_commit import _children_csr, argmax_workspace

    n, v = logits.shape
    dtype = _capi.TM_DTYPE_F32 if logits.dtype == torch.float32 else _capi.TM_DTYPE_BF16
    tokens = torch.zeros(n, dtype=torch.long, device="cuda")
    csr, edges = _children_csr([[] for _ in range(n)], n, "cuda")
    out = [torch.empty(n, dtype=torch.long, device="cuda") for _ in range(2)]
    result = torch.empty(3, dtype=torch.long, device="cuda")
    _capi.call("tm_op4_argmax_walk", logits.data_ptr(), dtype, n, v, logits.stride(0),
               tokens.data_ptr(), csr.data_ptr(), csr.data_ptr() + 4 * n,
               csr.data_ptr() + 8 * n, edges, 0, 0, argmax.data_ptr(), out[0].data_ptr(),
               out[1].data_ptr(), result.data_ptr(),
               argmax_workspace(n, logits.device).data_ptr(), _capi.stream_of(logits.device))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_unaligned_rows(dtype):
    """Rows that start off a 16-byte boundary take the scalar loads."""
    n, v = 7, 5003
    g = torch.Generator().manual_seed(11)
    full = (torch.randn(n, v + 1, generator=g) * 3).to(dtype)
    full[3, 4000] = full[3, 1:].max() + 1
    full[3, 17] = full[3, 4000]
    logits = full.cuda()[:, 1:]
    assert logits.data_ptr() % 16 != 0 and logits.stride(0) == v + 1
    argmax = torch.empty(n, dtype=torch.int32, device="cuda")
    _direct_argmax(logits, argmax)
    expect = full[:, 1:].float().argmax(-1).numpy()
    assert np.array_equal(argmax.cpu().numpy(), expect)
    assert int(argmax[3]) == 16


def test_greedy_walk_large_tree_from_global_memory():
    """A 2100-node chain (more nodes than the walk stages in LDS) is accepted
    to the end."""
    _say("walk n=2100 chain")
    op4 = _op4()
    n, v = 2100, 64
    g = torch.Generator().manual_seed(5)
    tokens = torch.randint(0, v, (n,), generator=g)
    children = [[i + 1] for i in range(n - 1)] + [[]]
    logits = torch.randn(n, v, generator=g)
    for i in range(n - 1):
        logits[i, int(tokens[i + 1])] = 50.0
    res = op4.fused_verify_commit(logits.cuda(), None, tokens.cuda(), None, children,
                                  max_depth=n)
    c_slots, c_toks, c_bonus, c_num, _ = oracle_c.greedy_walk(
        oracle_c.argmax(logits.numpy()), tokens.numpy(), children, n)
    assert int(res.num_accepted) == c_num == n - 1
    assert np.array_equal(res.accepted_slots.cpu().numpy(), c_slots)
    assert np.array_equal(res.accepted_tokens.cpu().numpy(), c_toks)
    assert int(res.bonus_token) == c_bonus


@pytest.mark.parametrize("seed", range(50))
def test_greedy_walk_random_trees(seed):
    """Reference tests/test_op4.py:70-91, plus planted full-accept chains."""
    op4 = _op4()
    n, v = 16, 512
    g, parent, children, tokens, _ = _tree(seed, n, v)
    logits = torch.randn(n, v, generator=g) * 3
    if seed % 3 == 0:
        for node in range(n):
            if children[node]:
                logits[node, tokens[children[node][0]]] += 100.0
    ref_slots, ref_toks, ref_bonus, ref_num = op4_ref.tree_verify(
        logits, torch.zeros(n, v), tokens, children)
    res = op4.fused_verify_commit(logits.cuda(), torch.zeros(n, v).cuda(), tokens.cuda(),
                                  parent.cuda(), children, max_depth=n)
    assert int(res.num_accepted) == ref_num
    assert torch.equal(res.accepted_slots.cpu(), ref_slots)
    assert torch.equal(res.accepted_tokens.cpu(), ref_toks)
    assert int(res.bonus_token) == ref_bonus
    am = oracle_c.argmax(logits.numpy())
    c_slots, c_toks, c_bonus, c_num, c_root = oracle_c.greedy_walk(am, tokens.numpy(),
                                                                   children, n)
    assert c_num == ref_num and c_bonus == ref_bonus
    assert np.array_equal(c_slots, ref_slots.numpy())


def test_greedy_max_depth_truncates_like_reference_kernel():
    """The device walk stops after max_depth levels (op4_commit.py:107)."""
    op4 = _op4()
    n, v = 10, 64
    tokens = torch.arange(n) + 3
    parent = torch.tensor([-1] + list(range(n - 1)))
    children = [[i + 1] for i in range(n - 1)] + [[]]
    logits = torch.zeros(n, v)
    for i in range(n - 1):
        logits[i, int(tokens[i + 1])] = 10.0
    for md in (0, 1, 4, 9, 20):
        res = op4.fused_verify_commit(logits.cuda(), None, tokens.cuda(), parent.cuda(),
                                      children, max_depth=md)
        c_slots, _, c_bonus, c_num, _ = oracle_c.greedy_walk(
            oracle_c.argmax(logits.numpy()), tokens.numpy(), children, md)
        assert int(res.num_accepted) == c_num == min(md, n - 1)
        assert int(res.bonus_token) == c_bonus


def _kv_setup(layers, kvh, hd, page, num_pages, seq_len, tree_size, seed, dtype):
    from treemoe_spec_amd.kv_cache import MixtralConfig, PagedKVCache

    cfg = MixtralConfig(num_layers=layers, num_kv_heads=kvh, head_dim=hd)
    kv = PagedKVCache(cfg, num_pages, device="cuda", dtype=dtype, page_size=page,
                      tree_size=tree_size)
    g = torch.Generator(device="cuda").manual_seed(seed)
    kv.k.normal_(generator=g)
    kv.v.normal_(generator=g)
    # non-trivial page order: shuffle the free list
    perm = torch.randperm(len(kv._free), generator=torch.Generator().manual_seed(seed)).tolist()
    kv._free = [kv._free[i] for i in perm]
    kv._ensure_capacity(seq_len)
    kv.seq_len = seq_len
    return kv


@pytest.mark.parametrize("page,layers,kvh,hd,seq_len,dtype", [
    (16, 32, 8, 128, 4096, torch.bfloat16),   # config 4
    (64, 2, 2, 16, 10, torch.float32),        # reference page size, tiny model
    (16, 4, 2, 8, 37, torch.bfloat16),        # 16-byte rows (vector path)
    (8, 3, 1, 3, 5, torch.bfloat16),          # 6-byte rows (byte path)
])
def test_kv_commit_bytes(page, layers, kvh, hd, seq_len, dtype):
    _say(f"kv commit page={page} L={layers} seq={seq_len} {dtype}")
    op4 = _op4()
    from treemoe_spec_amd.workloads import op4_workload

    n = 64
    w = op4_workload(n=n, vocab=4096, max_depth=8, seed=seq_len)
    num_pages = (seq_len + 64) // page + (n + page - 1) // page + 8
    kv = _kv_setup(layers, kvh, hd, page, num_pages, seq_len, n, seq_len + 1, dtype)
    k0, v0 = kv.k.clone(), kv.v.clone()
    table_before = list(kv.block_table)
    res = op4.fused_verify_commit(w.logits.cuda(), None, w.tokens.cuda(), w.parent.cuda(),
                                  w.children, kv=kv, max_depth=w.max_depth)
    torch.cuda.synchronize()
    num = int(res.num_accepted)
    assert kv.seq_len == seq_len + num + 1
    # oracle: same commit on the pre-call cache with the table after capacity growth
    commit = torch.cat([torch.zeros(1, dtype=torch.long), res.accepted_slots.cpu()])
    assert kv.block_table[: len(table_before)] == table_before
    committed = op4_ref.commit_tree(k0, v0, commit, kv.tree_pages, kv.block_table, seq_len)
    assert committed == num + 1
    assert torch.equal(kv.k, k0) and torch.equal(kv.v, v0)
    # and the walk itself against the reference restatement
    ref_slots, _, ref_bonus, ref_num = op4_ref.tree_verify(w.logits.float(), None, w.tokens,
                                                           w.children)
    assert ref_num == num and int(res.bonus_token) == ref_bonus
    assert torch.equal(res.accepted_slots.cpu(), ref_slots)


@pytest.mark.parametrize("binding", ["cpython", "ctypes"])
def test_commit_count_word_across_calls(monkeypatch, binding):
    """num_accepted reaches the host through the pinned word the KV commit
    writes: back-to-back calls with different accepted paths each read their
    own count, and the synchronising fallback (no spin) reads the same.  Both
    bindings of the C ABI (the CPython module and ctypes) are exercised."""
    _say(f"kv commit count word, 6 calls, {binding} binding")
    op4 = _op4()
    if binding == "ctypes":
        monkeypatch.setattr(op4, "_fast", None)
    else:
        assert op4._fast is not None, "the CPython binding is not built"
    from treemoe_spec_amd.workloads import op4_workload

    n, seq0 = 64, 100
    kv = _kv_setup(2, 2, 16, 16, 80, seq0, n, 5, torch.bfloat16)
    from treemoe_spec_amd import _capi

    dev = torch.cuda.current_device()
    key = op4._scratch_key(n, dev, _capi.stream_of(dev))
    nums = []
    for call, seed in enumerate((11, 12, 13, 14, 15, 16)):
        if call == 3:
            monkeypatch.setattr(op4, "_NOTE_SPIN_S", 0.0)
        w = op4_workload(n=n, vocab=4096, max_depth=8, seed=seed)
        _, _, _, ref_num = op4_ref.tree_verify(w.logits.float(), None, w.tokens, w.children)
        before = kv.seq_len
        res = op4.fused_verify_commit(w.logits.cuda(), None, w.tokens.cuda(), w.parent.cuda(),
                                      w.children, kv=kv, max_depth=8)
        assert kv.seq_len == before + ref_num + 1, (call, seed)
        torch.cuda.synchronize()
        assert int(res.num_accepted) == ref_num
        ws = op4._scratch_cache[key]
        assert ws.note_dev != 0 and int(ws.note_np[0]) == ref_num
        nums.append(ref_num)
    assert len(set(nums)) > 1, "the seeds should give different path lengths"


def test_two_streams_do_not_share_partials():
    """Two kv=None calls with the same N on two streams, the first queued
    behind a GPU spin so that the second is issued while the first's kernels
    still wait: each returns its own tree's accepted path (the row partials
    and argmax vector are per stream)."""
    _say("two streams, kv=None, same N")
    op4 = _op4()
    from treemoe_spec_amd.workloads import op4_workload

    n = 64
    ws = [op4_workload(n=n, vocab=4096, max_depth=8, seed=s) for s in (21, 22)]
    refs = [op4_ref.tree_verify(w.logits.float(), None, w.tokens, w.children) for w in ws]
    assert refs[0][3] != refs[1][3] or not torch.equal(refs[0][0], refs[1][0])
    ins = [(w.logits.cuda(), w.tokens.cuda(), w.parent.cuda()) for w in ws]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    res = [None, None]
    with torch.cuda.stream(streams[0]):
        torch.cuda._sleep(2_000_000)
        res[0] = op4.fused_verify_commit(ins[0][0], None, ins[0][1], ins[0][2], ws[0].children)
    with torch.cuda.stream(streams[1]):
        res[1] = op4.fused_verify_commit(ins[1][0], None, ins[1][1], ins[1][2], ws[1].children)
    torch.cuda.synchronize()
    for r, (slots, toks, bonus, num) in zip(res, refs):
        assert torch.equal(r.accepted_slots.cpu(), slots)
        assert torch.equal(r.accepted_tokens.cpu(), toks)
        assert int(r.bonus_token) == bonus and int(r.num_accepted) == num


def test_config4_planted_path_accepted():
    _say("config4 planted path")
    op4 = _op4()
    from treemoe_spec_amd.workloads import op4_workload

    for seed in range(3, 13):
        w = op4_workload(n=64, vocab=32000, max_depth=8, seed=seed, tie_rows=0)
        res = op4.fused_verify_commit(w.logits.cuda(), None, w.tokens.cuda(), w.parent.cuda(),
                                      w.children, max_depth=8)
        num = int(res.num_accepted)
        assert num >= len(w.planted_path)
        assert res.accepted_slots[: len(w.planted_path)].tolist() == w.planted_path


def test_rejects_cpu_and_bad_sampling_inputs():
    op4 = _op4()
    logits = torch.zeros(2, 8)
    with pytest.raises(RuntimeError, match="ROCm"):
        op4.fused_verify_commit(logits, None, torch.zeros(2, dtype=torch.long), None,
                                [[1], []])
    with pytest.raises(ValueError, match="draft_probs"):
        op4.fused_verify_commit(logits.cuda(), None, torch.zeros(2, dtype=torch.long), None,
                                [[1], []], temperature=1.0)
    with pytest.raises(ValueError, match="draft_probs"):
        op4.fused_verify_commit(logits.cuda(), torch.zeros(2, 7, device="cuda"),
                                torch.zeros(2, dtype=torch.long), None, [[1], []],
                                temperature=1.0)


# ------------------------------------------------------------- sampling --

def _dt(t):
    from treemoe_spec_amd import _capi

    return _capi.TM_DTYPE_F32 if t.dtype == torch.float32 else _capi.TM_DTYPE_BF16


def _direct_sample(logits, q, tokens, children, uniforms, bonus_exp, temperature):
    """tm_op4_sample_walk on device tensors; returns (slots, toks, result, residual)."""
    from treemoe_spec_amd import _capi
    from treemoe_spec_amd.kernels.op4_commit import _children_csr

    n, v = logits.shape
    assert q.shape == (n, v) and tokens.numel() == n and uniforms.numel() >= n
    csr, edges = _children_csr(children, n, "cuda")
    slots = torch.empty(n, dtype=torch.int64, device="cuda")
    toks = torch.empty(n, dtype=torch.int64, device="cuda")
    result = torch.empty(3, dtype=torch.int64, device="cuda")
    residual = torch.empty(v, dtype=torch.float32, device="cuda")
    p = _capi.ptr
    _capi.call("tm_op4_sample_walk", p(logits), _dt(logits), n, v, logits.stride(0), p(q),
               q.stride(0), p(tokens), p(csr), p(csr) + 4 * n, p(csr) + 8 * n, edges, p(uniforms),
               p(bonus_exp), float(temperature), p(residual), p(slots), p(toks), p(result),
               _capi.stream_of(logits.device))
    torch.cuda.synchronize()
    return slots.cpu(), toks.cpu(), result.cpu(), residual.cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sampling_injected_uniforms_kat(dtype):
    """Reference tests/test_op4.py:54-67: u = 0 accepts the whole chain,
    u = 1 rejects the first child."""
    _say(f"sampling KAT {dtype}")
    tokens = torch.tensor([5, 7, 9]).cuda()
    children = [[1], [2], []]
    logits = torch.zeros(3, 32)
    for i, w in enumerate([7, 9, 11]):
        logits[i, w] = 10.0
    logits = logits.to(dtype).cuda()
    q = torch.full((3, 32), 1.0 / 32, device="cuda")
    bu = torch.ones(32, device="cuda")
    slots, toks, result, _ = _direct_sample(logits, q, tokens, children,
                                            torch.zeros(3, device="cuda"), bu, 1.0)
    assert int(result[1]) == 2 and slots.tolist() == [1, 2, -1] and toks.tolist() == [7, 9, -1]
    assert int(result[2]) == 2
    slots, toks, result, _ = _direct_sample(logits, q, tokens, children,
                                            torch.ones(3, device="cuda"), bu, 1.0)
    assert int(result[1]) == 0 and slots.tolist() == [-1, -1, -1]
    assert int(result[2]) == 0


def _sampling_case(seed, n, v, follow):
    """Random tree whose child tokens follow the parent's most likely token
    with probability `follow`, and per-node draft distributions."""
    g, parent, children, tokens, _ = _tree(seed, n, v)
    logits = torch.randn(n, v, generator=g) * 3
    q = torch.softmax(torch.randn(n, v, generator=g) * 2, -1)
    for node, kids in enumerate(children):
        if kids and float(torch.rand(1, generator=g)) < follow:
            tokens[kids[int(torch.randint(0, len(kids), (1,), generator=g))]] = \
                int(logits[node].argmax())
    return g, children, tokens, logits, q


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seed,n,v,temperature", [
    (1, 16, 64, 1.0), (2, 64, 32000, 0.7), (3, 33, 1000, 1.5), (4, 64, 32001, 1.0),
    (5, 8, 5, 0.3), (6, 64, 4096, 2.0), (7, 12, 32768, 1.0), (8, 12, 32769, 0.9),
    (9, 16, 100000, 1.0), (10, 6, 9000, 1.2), (11, 2100, 300, 1.0), (12, 2100, 40000, 0.8)])
def test_sampling_matches_oracle(dtype, seed, n, v, temperature):
    """Accept path, next root and bonus bit-exact against the oracle with the
    same uniforms and exponentials; the final residual within rtol 1e-4 /
    atol 1e-6 (fp32 softmax and residual updates with a different exp and
    summation order).  The bonus is exactly the first index of the largest
    residual / e over the kernel's own residual (IEEE fp32 division), and the
    oracle's index unless the oracle's two largest ratios lie closer than that
    residual tolerance.
    bf16 logits: the oracle gets them widened to fp32, as the kernel reads them.
    V up to 32768 runs the register-resident walk (8, 16 or 32 entries per
    thread), larger V the tiled walk over a global residual (32769: a one-entry
    second tile; 100000: four tiles).  Trees of more than 2048 nodes are walked
    from global memory instead of LDS (n = 2100, both walks)."""
    _say(f"sampling seed={seed} n={n} v={v} T={temperature} {dtype}")
    for rep in range(4):
        g, children, tokens, logits, q = _sampling_case(seed * 10 + rep, n, v, 0.8)
        logits = logits.to(dtype)
        u = torch.rand(n, generator=g)
        e = torch.empty(v).exponential_(1.0, generator=g)
        slots, toks, result, residual = _direct_sample(
            logits.cuda(), q.cuda(), tokens.cuda(), children, u.cuda(), e.cuda(), temperature)
        r_slots, r_toks, r_bonus, r_num, r_res = op4_ref.tree_verify(
            logits.float(), q, tokens, children, temperature=temperature, uniforms=u,
            bonus_exp=e, return_residual=True)
        assert int(result[1]) == r_num
        assert torch.equal(slots, r_slots) and torch.equal(toks, r_toks)
        assert int(result[2]) == (int(r_slots[r_num - 1]) if r_num else 0)
        torch.testing.assert_close(residual, r_res.float(), rtol=1e-4, atol=1e-6)
        bonus = int(result[0])
        assert bonus == int(torch.argmax(residual / e))
        if bonus != r_bonus:
            ratio = r_res.float() / e
            assert float(ratio[bonus]) >= float(ratio.max()) * (1 - 3e-4), (bonus, r_bonus)


def test_sampling_first_token_distribution():
    """The emitted first token (accepted child or bonus) is distributed as
    p = softmax(logits[root] / T) when child tokens are drawn from their draft
    distributions: 4000 launches, 6-sigma binomial bound per token."""
    _say("sampling distribution")
    v, temperature, trials = 6, 0.8, 4000
    g = torch.Generator().manual_seed(21)
    logits = (torch.randn(4, v, generator=g) * 1.5).cuda()
    q = torch.softmax(torch.randn(4, v, generator=g) * 1.5, -1)
    children = [[1, 2, 3], [], [], []]
    p = torch.softmax(logits[0].cpu() / temperature, -1).double().numpy()
    tokens = torch.zeros(trials, 4, dtype=torch.long)
    for c in (1, 2, 3):
        tokens[:, c] = torch.multinomial(q[c], trials, replacement=True, generator=g)
    tokens = tokens.cuda()
    u = torch.rand(trials, 4, generator=g).cuda()
    e = torch.empty(trials, v).exponential_(1.0, generator=g).cuda()
    q = q.cuda()
    from treemoe_spec_amd import _capi
    from treemoe_spec_amd.kernels.op4_commit import _children_csr

    csr, edges = _children_csr(children, 4, "cuda")
    slots = torch.empty(trials, 4, dtype=torch.int64, device="cuda")
    toks = torch.empty(trials, 4, dtype=torch.int64, device="cuda")
    result = torch.empty(trials, 3, dtype=torch.int64, device="cuda")
    residual = torch.empty(v, dtype=torch.float32, device="cuda")
    P = _capi.ptr
    stream = _capi.stream_of(logits.device)
    for t in range(trials):
        _capi.call("tm_op4_sample_walk", P(logits), _dt(logits), 4, v, v, P(q), v,
                   P(tokens[t]), P(csr), P(csr) + 16, P(csr) + 32, edges, P(u[t]), P(e[t]),
                   temperature, P(residual), P(slots[t]), P(toks[t]), P(result[t]), stream)
    torch.cuda.synchronize()
    num = result[:, 1].cpu()
    first = torch.where(num > 0, toks[:, 0].cpu(), result[:, 0].cpu())
    counts = np.bincount(first.numpy(), minlength=v)
    sigma = np.sqrt(trials * p * (1 - p))
    assert np.all(np.abs(counts - trials * p) <= 6 * sigma), (counts, trials * p)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_sampling_draws_from_the_generator_and_commits(dtype):
    """fused_verify_commit(temperature > 0) takes its draws from the caller's
    generator as the reference does (rand(N), then torch.multinomial): the
    oracle run on the GPU with a generator in the same state, calling
    torch.multinomial itself, gives the same path and bonus; the commit moves
    [root] + accepted path, bytes equal to the oracle."""
    _say(f"fused sampling + commit {dtype}")
    op4 = _op4()
    n, v, seq_len, page = 64, 4096, 37, 16
    g, children, tokens, logits, q = _sampling_case(77, n, v, 0.9)
    logits = logits.to(dtype).cuda()
    kv = _kv_setup(4, 2, 8, page, 40, seq_len, n, 9, torch.bfloat16)
    k0, v0 = kv.k.cpu(), kv.v.cpu()
    gen = torch.Generator(device="cuda").manual_seed(1234)
    res = op4.fused_verify_commit(logits, q.cuda(), tokens.cuda(), None, children, kv=kv,
                                  temperature=0.9, generator=gen)
    torch.cuda.synchronize()
    gen2 = torch.Generator(device="cuda").manual_seed(1234)
    r_slots, r_toks, r_bonus, r_num = op4_ref.tree_verify(
        logits.float(), q.cuda(), tokens, children, temperature=0.9, generator=gen2)
    assert int(res.num_accepted) == r_num and int(res.bonus_token) == r_bonus
    assert torch.equal(res.accepted_slots.cpu(), r_slots)
    assert torch.equal(res.accepted_tokens.cpu(), r_toks)
    assert torch.equal(gen.get_state(), gen2.get_state())
    assert kv.seq_len == seq_len + r_num + 1
    commit = torch.cat([torch.zeros(1, dtype=torch.long), r_slots])
    assert op4_ref.commit_tree(k0, v0, commit, kv.tree_pages, kv.block_table, seq_len) == r_num + 1
    assert torch.equal(kv.k.cpu(), k0) and torch.equal(kv.v.cpu(), v0)


@pytest.mark.parametrize("n,v,follow", [(64, 32000, 0.9), (16, 100000, 0.6), (2100, 1000, 0.5),
                                        (8, 7, 0.0)])
def test_sampling_seed_exact_with_reference_draws(n, v, follow):
    """Same generator seed, same tokens: fused_verify_commit against the
    reference's algorithm (the oracle on the GPU drawing torch.rand(N) and
    calling torch.multinomial(residual, 1, generator)) over 12 seeds each,
    register walk (V <= 32768), tiled walk (V = 100000) and a tree walked from
    global memory (N = 2100).  Equal unless two of the race's ratios lie within
    the residual's fp32 rounding difference, which these seeds do not hit."""
    _say(f"seed-exact sampling n={n} v={v}")
    op4 = _op4()
    for seed in range(12):
        g, children, tokens, logits, q = _sampling_case(500 + seed, n, v, follow)
        logits, q = logits.cuda(), q.cuda()
        res = op4.fused_verify_commit(logits, q, tokens.cuda(), None, children, temperature=0.8,
                                      generator=torch.Generator(device="cuda").manual_seed(seed))
        r_slots, r_toks, r_bonus, r_num = op4_ref.tree_verify(
            logits, q, tokens, children, temperature=0.8,
            generator=torch.Generator(device="cuda").manual_seed(seed))
        assert int(res.num_accepted) == r_num, seed
        assert int(res.bonus_token) == r_bonus, seed
        assert torch.equal(res.accepted_slots.cpu(), r_slots)
        assert torch.equal(res.accepted_tokens.cpu(), r_toks)


# ---------------------------------------------------------- rep penalty --

def _direct_penalty(logits, prev, penalty):
    from treemoe_spec_amd import _capi
    from treemoe_spec_amd.kernels.op4_commit import _penalty_table_size

    n, v = logits.shape
    size = _penalty_table_size(prev.numel())
    table = torch.empty(2 * size, dtype=torch.int32, device="cuda")
    p = _capi.ptr
    _capi.call("tm_op4_rep_penalty", p(logits), _dt(logits), n, v, logits.stride(0), p(prev),
               prev.numel(), float(penalty), p(table), size, _capi.stream_of(logits.device))
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,v,num_prev,penalty", [
    (16, 32000, 40, 1.3), (64, 32000, 5000, 1.1), (3, 7, 12, 0.7), (5, 1000, 1, 2.5)])
def test_rep_penalty_matches_oracle(dtype, n, v, num_prev, penalty):
    """Bit-exact against the oracle: duplicates applied once per listing,
    out-of-range entries skipped, bf16 rounded after every application,
    rows addressed through a row stride wider than V."""
    _say(f"rep penalty {dtype} n={n} v={v} prev={num_prev} p={penalty}")
    g = torch.Generator().manual_seed(n + v + num_prev)
    base = (torch.randn(n, v + 3, generator=g) * 4).to(dtype)
    base[:, ::5] = -base[:, ::5].abs()
    base[:, 1] = 0.0
    prev = torch.randint(0, v, (num_prev,), generator=g)
    if num_prev > 4:
        prev[:4] = torch.tensor([-1, v, int(prev[5]), int(prev[5])])
    got = base.cuda()
    _direct_penalty(got[:, :v], prev.cuda(), penalty)
    want = base.clone()
    op4_ref.rep_penalty_inplace(want[:, :v], prev, penalty)
    assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_greedy_with_rep_penalty(dtype):
    """fused_verify_commit(rep_penalty != 1): logits penalised in place like the
    reference, then the greedy walk over them; a penalised argmax flips the
    accept decision; no prev_tokens penalises token 0 once."""
    _say(f"greedy + rep penalty {dtype}")
    op4 = _op4()
    n, v = 8, 512
    tokens = torch.tensor([3, 10, 11, 12, 13, 14, 15, 16])
    children = [[1, 2], [3], [], [4], [], [], [], []]
    logits = torch.randn(n, v, generator=torch.Generator().manual_seed(9))
    logits[0, 10], logits[0, 11] = 9.0, 8.0     # 10 wins unless penalised
    logits[1, 12] = 9.0
    logits[3, 13] = 9.0
    logits[4, 0] = 20.0                         # still row 4's argmax once penalised
    logits = logits.to(dtype)
    prev = torch.tensor([10, 10, 7])
    for prev_arg, penalty in ((prev, 1.5), (None, 1.5), (prev, 1.0)):
        lg = logits.clone().cuda()
        res = op4.fused_verify_commit(lg, None, tokens.cuda(), None, children,
                                      rep_penalty=penalty, prev_tokens=prev_arg)
        want = logits.clone()
        if penalty != 1.0:
            op4_ref.rep_penalty_inplace(want, prev_arg if prev_arg is not None
                                        else torch.zeros(1, dtype=torch.long), penalty)
        assert torch.equal(lg.cpu(), want)
        if penalty != 1.0:
            # the reference's pick after a penalty: argmax of the rounded softmax
            am = (oracle_c.softmax_argmax(bf16_bits(want), bf16_bits=True)
                  if dtype == torch.bfloat16 else oracle_c.softmax_argmax(want.numpy()))
        else:
            am = oracle_c.argmax(want.float().numpy())
        r_slots, _, r_bonus, r_num, _ = oracle_c.greedy_walk(am, tokens.numpy(), children, 6)
        assert int(res.num_accepted) == r_num and int(res.bonus_token) == r_bonus
        assert np.array_equal(res.accepted_slots.cpu().numpy(), r_slots)
    # with the penalty on token 10 the walk takes node 2 (token 11) instead
    lg = logits.clone().cuda()
    res = op4.fused_verify_commit(lg, None, tokens.cuda(), None, children, rep_penalty=1.5,
                                  prev_tokens=prev.cuda())
    assert res.accepted_slots[:1].tolist() == [2]


# ------------------------------------------- reference cache and padded trees --

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_commit_through_reference_cache_layout(dtype):
    """fused_verify_commit with a cache that has exactly the reference
    PagedKVCache attributes (page 64, scratch block ``tree_block``, no
    tree_pages / device_tables), fp32 logits as the engine passes them
    (loop.py:185): committed bytes equal the oracle's commit_tree."""
    _say(f"commit through reference cache layout {dtype}")
    from tests.ref_layout_cache import RefLayoutKVCache
    from treemoe_spec_amd.workloads import op4_workload

    op4 = _op4()
    n, seq_len = 64, 1000
    for seed in (11, 12, 13):
        w = op4_workload(n=n, vocab=4096, max_depth=8, seed=seed)
        kv = RefLayoutKVCache(4, 2, 64, (seq_len + 80) // 64 + 4, device="cuda", dtype=dtype)
        g = torch.Generator(device="cuda").manual_seed(seed)
        kv.k.normal_(generator=g)
        kv.v.normal_(generator=g)
        perm = torch.randperm(len(kv._free), generator=torch.Generator().manual_seed(seed))
        kv._free = [kv._free[i] for i in perm.tolist()]
        kv._ensure_capacity(seq_len)
        kv.seq_len = seq_len
        k0, v0 = kv.k.clone(), kv.v.clone()
        res = op4.fused_verify_commit(w.logits.float().cuda(), None, w.tokens.cuda(),
                                      w.parent.cuda(), w.children, kv=kv, max_depth=8)
        torch.cuda.synchronize()
        num = int(res.num_accepted)
        assert kv.seq_len == seq_len + num + 1
        commit = torch.cat([torch.zeros(1, dtype=torch.long), res.accepted_slots.cpu()])
        assert op4_ref.commit_tree(k0, v0, commit, [kv.tree_block], kv.block_table,
                                   seq_len) == num + 1
        assert torch.equal(kv.k, k0) and torch.equal(kv.v, v0)
        ref_slots, _, ref_bonus, ref_num = op4_ref.tree_verify(w.logits.float(), None,
                                                               w.tokens, w.children)
        assert ref_num == num and int(res.bonus_token) == ref_bonus
        assert torch.equal(res.accepted_slots.cpu(), ref_slots)


def _padded_tree(seed, n, num_valid, vocab):
    """A num_valid-node random tree in slots 0..num_valid-1 and edge-free
    padding slots after it, as the engine builds trees smaller than
    tree_size (engine/tree.py:175-188)."""
    g, parent, children, tokens, _ = _tree(seed, num_valid, vocab)
    children = [list(c) for c in children] + [[] for _ in range(n - num_valid)]
    tokens = torch.cat([tokens, torch.zeros(n - num_valid, dtype=tokens.dtype)])
    parent = torch.cat([parent, torch.full((n - num_valid,), -1, dtype=parent.dtype)])
    return g, parent, children, tokens


@pytest.mark.parametrize("seed,num_valid", [(0, 40), (1, 1), (2, 63), (3, 17)])
def test_padded_tree_greedy(seed, num_valid):
    _say(f"padded tree greedy seed={seed} valid={num_valid}")
    op4 = _op4()
    n, v = 64, 2048
    g, parent, children, tokens = _padded_tree(seed, n, num_valid, v)
    logits = torch.randn(n, v, generator=g) * 3
    for node in range(num_valid):
        if children[node] and node % 2 == 0:
            logits[node, tokens[children[node][0]]] += 100.0
    ref = op4_ref.tree_verify(logits, None, tokens, children)
    res = op4.fused_verify_commit(logits.cuda(), None, tokens.cuda(), parent.cuda(), children,
                                  max_depth=n)
    assert int(res.num_accepted) == ref[3] and int(res.bonus_token) == ref[2]
    assert torch.equal(res.accepted_slots.cpu(), ref[0])
    assert torch.equal(res.accepted_tokens.cpu(), ref[1])


@pytest.mark.parametrize("v", [1000, 40000])
@pytest.mark.parametrize("where", ["root", "deep", "draft"])
def test_sampling_nan_follows_the_reference(where, v):
    """NaN logits or draft rows: the softmax, the accept test and the
    residual update keep NaN as torch does, so every child at that node is
    rejected (u < NaN is false) exactly as in the oracle, and the bonus of the
    all-NaN residual is torch.argmax's first NaN, index 0, inside the
    vocabulary.  Register walk (V = 1000) and tiled walk (V = 40000)."""
    _say(f"sampling NaN {where} v={v}")
    n = 12
    g = torch.Generator().manual_seed(31)
    children = [[1, 2], [3], [], [4, 5], [6], [], [7], [], [], [], [], []]
    tokens = torch.randint(0, v, (n,), generator=g)
    logits = torch.randn(n, v, generator=g) * 2
    q = torch.softmax(torch.randn(n, v, generator=g), -1)
    # plant acceptance of 1 -> 3 so that a deeper node is reached
    for node, child in ((0, 1), (1, 3)):
        logits[node, tokens[child]] = 30.0
        q[child, tokens[child]] = 1e-6
    if where == "root":
        logits[0, 5] = float("nan")
    elif where == "deep":
        logits[3, 7] = float("nan")
    else:
        q[4] = float("nan")
    u = torch.rand(n, generator=g) * 0.5
    e = torch.empty(v).exponential_(1.0, generator=g)
    slots, toks, result, _ = _direct_sample(logits.cuda(), q.cuda(), tokens.cuda(), children,
                                            u.cuda(), e.cuda(), 1.0)
    r_slots, r_toks, r_bonus, r_num = op4_ref.tree_verify(
        logits, q, tokens, children, temperature=1.0, uniforms=u, bonus_exp=e)
    assert int(result[1]) == r_num and int(result[0]) == r_bonus
    assert torch.equal(slots, r_slots) and torch.equal(toks, r_toks)
    assert 0 <= int(result[0]) < v
    assert r_num == {"root": 0, "deep": 2, "draft": 2}[where]


@pytest.mark.parametrize("seed,num_valid", [(4, 40), (5, 2)])
def test_padded_tree_sampling(seed, num_valid):
    _say(f"padded tree sampling seed={seed} valid={num_valid}")
    n, v = 64, 1000
    g, parent, children, tokens = _padded_tree(seed, n, num_valid, v)
    logits = torch.randn(n, v, generator=g)
    q = torch.softmax(torch.randn(n, v, generator=g), -1)
    uniforms = torch.rand(n, generator=g) * 0.3
    bonus_exp = torch.empty(v).exponential_(1.0, generator=g)
    slots, toks, result, _ = _direct_sample(logits.cuda(), q.cuda(), tokens.cuda(), children,
                                            uniforms.cuda(), bonus_exp.cuda(), 1.0)
    r_slots, r_toks, r_bonus, r_num = op4_ref.tree_verify(
        logits, q, tokens, children, temperature=1.0, uniforms=uniforms, bonus_exp=bonus_exp)
    assert int(result[1]) == r_num and int(result[0]) == r_bonus
    assert torch.equal(slots, r_slots) and torch.equal(toks, r_toks)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_softmax_argmax_matches_oracle(dtype):
    """The argmax of the rounded softmax (greedy + repetition penalty) is
    bit-exact against the oracle: config-4 rows, unaligned rows, planted ties
    whose rounded probabilities are equal (the lower index wins although its
    logit is smaller), a row of -inf."""
    _say(f"softmax argmax {dtype}")
    from treemoe_spec_amd import _capi
    from treemoe_spec_amd.kernels.op4_commit import _children_csr, argmax_workspace

    g = torch.Generator().manual_seed(23)
    for n, v in ((64, 32000), (5, 1001), (3, 7)):
        x = torch.randn(n, v, generator=g) * 3
        if v > 100:
            x[0] = -10.0
            x[0, 5], x[0, 7] = 0.0, 1e-9
            x[1] = -3.0
            x[1, 3], x[1, 9] = 2.0 ** -8, 2.0 ** -8 + 2.0 ** -15
            x[2] = -float("inf")
        x = x.to(dtype)
        if dtype == torch.bfloat16:
            want = oracle_c.softmax_argmax(bf16_bits(x), bf16_bits=True)
        else:
            want = oracle_c.softmax_argmax(x.numpy())
        if v > 100:
            # row 0 ties in both dtypes; row 1 only once rounded to bf16
            assert want[0] == 5 and want[2] == 0
            assert want[1] == (3 if dtype == torch.bfloat16 else 9)
        xd = x.cuda()
        tokens = torch.zeros(n, dtype=torch.long, device="cuda")
        csr, edges = _children_csr([[] for _ in range(n)], n, "cuda")
        argmax = torch.empty(n, dtype=torch.int32, device="cuda")
        out = [torch.empty(n, dtype=torch.long, device="cuda") for _ in range(2)]
        result = torch.empty(3, dtype=torch.long, device="cuda")
        _capi.call("tm_op4_argmax_walk", xd.data_ptr(), _dt(xd), n, v, xd.stride(0),
                   tokens.data_ptr(), csr.data_ptr(), csr.data_ptr() + 4 * n,
                   csr.data_ptr() + 8 * n, edges, 0, 1, argmax.data_ptr(), out[0].data_ptr(),
                   out[1].data_ptr(), result.data_ptr(),
                   argmax_workspace(n, xd.device).data_ptr(), _capi.stream_of(xd.device))
        torch.cuda.synchronize()
        assert np.array_equal(argmax.cpu().numpy(), want), (n, v)
