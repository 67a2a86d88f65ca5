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
    csr = _children_csr([[] for _ in range(n)], n, "cuda")
    out = [torch.empty(n, dtype=torch.long, device="cuda") for _ in range(2)]
    result = torch.empty(3, dtype=torch.long, device="cuda")
    _capi.call("tm_op4_argmax_walk", logits.data_ptr(), dtype, n, v, logits.stride(0),
               tokens.data_ptr(), csr.data_ptr(), csr.data_ptr() + 4 * n,
               csr.data_ptr() + 8 * n, 0, argmax.data_ptr(), out[0].data_ptr(),
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


def test_rejects_sampling_mode_and_cpu():
    op4 = _op4()
    logits = torch.zeros(2, 8)
    with pytest.raises(RuntimeError, match="ROCm"):
        op4.fused_verify_commit(logits, None, torch.zeros(2, dtype=torch.long), None,
                                [[1], []])
    with pytest.raises(NotImplementedError):
        op4.fused_verify_commit(logits.cuda(), None, torch.zeros(2, dtype=torch.long), None,
                                [[1], []], temperature=1.0)
