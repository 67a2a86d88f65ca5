"""Tree attention on the GPU against the CPU oracle (float32 restatement of the
reference's gather + mask + scaled_dot_product_attention).

Tolerance: the kernel reads bf16, accumulates in fp32, rounds the softmax
weights to bf16 for the P.V product (as bf16 attention kernels do) and writes
bf16; the output must be within rel-L2 <= 1e-2 of the fp32 oracle and every
element within 2e-2 * max|oracle| + 1e-3.
"""

from __future__ import annotations

import pytest
import torch

from oracle import attn_ref

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-2


def _say(msg: str) -> None:
    print(msg, flush=True)


def _case(n, hq, kvh, seq_len, page, seed, q_scale=3.0, layers=2):
    from treemoe_spec_amd.kv_cache import MixtralConfig, PagedKVCache

    g = torch.Generator().manual_seed(seed)
    cfg = MixtralConfig(num_layers=layers, num_kv_heads=kvh, head_dim=128, num_heads=hq)
    num_pages = (n + page - 1) // page + (seq_len + page - 1) // page + 6
    kv = PagedKVCache(cfg, num_pages, device="cuda", dtype=torch.bfloat16, page_size=page,
                      tree_size=n)
    kv.k.copy_(torch.randn(kv.k.shape, generator=g).to(torch.bfloat16))
    kv.v.copy_(torch.randn(kv.v.shape, generator=g).to(torch.bfloat16))
    perm = torch.randperm(len(kv._free), generator=g).tolist()
    kv._free = [kv._free[i] for i in perm]
    kv._ensure_capacity(seq_len)
    kv.seq_len = seq_len
    q = (torch.randn(n, hq, 128, generator=g) * q_scale).to(torch.bfloat16)
    k = torch.randn(n, kvh, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(n, kvh, 128, generator=g).to(torch.bfloat16)
    parent = [-1] + [int(torch.randint(0, i, (1,), generator=g)) for i in range(1, n)]
    mask = attn_ref.ancestor_mask(parent)
    return kv, q, k, v, mask


def _oracle(kv, q, k, v, mask, layer):
    return attn_ref.tree_attention(q, k, v, kv.k.cpu(), kv.v.cpu(), layer, kv.block_table,
                                   kv.seq_len, kv.block_size, mask)


def _check(got, want):
    got = got.float().cpu()
    rel = float((got - want).norm() / want.norm())
    assert rel <= REL_L2_TOL, rel
    bound = 2e-2 * float(want.abs().max()) + 1e-3
    assert float((got - want).abs().max()) <= bound


@pytest.mark.parametrize("n,hq,kvh,seq_len,page,chunk_keys", [
    (64, 32, 8, 4096, 16, 0),      # config 4 shape, automatic chunks
    (64, 32, 8, 4096, 16, 64),     # one stage per chunk: 65 chunks to combine
    (64, 32, 8, 300, 16, 0),       # ragged prefix
    (1, 8, 2, 0, 16, 0),           # the root alone
    (7, 8, 2, 37, 16, 0),
    (33, 4, 4, 129, 64, 0),        # group 1, reference page size
    (200, 4, 2, 1000, 16, 0),      # four mask words per row
    (64, 32, 8, 5000, 16, 192),
    (16, 8, 8, 64, 16, 0),         # prefix exactly one stage
])
def test_matches_oracle(n, hq, kvh, seq_len, page, chunk_keys):
    _say(f"tree attention n={n} hq={hq} kvh={kvh} seq={seq_len} page={page} chunk={chunk_keys}")
    from treemoe_spec_amd.kernels.tree_attention import tree_attention

    kv, q, k, v, mask = _case(n, hq, kvh, seq_len, page, n * 131 + seq_len)
    out = tree_attention(q.cuda(), k.cuda(), v.cuda(), kv, 1, mask.cuda(),
                         chunk_keys=chunk_keys)
    torch.cuda.synchronize()
    _check(out, _oracle(kv, q, k, v, mask, 1))


@pytest.mark.parametrize("n,seq_len", [(64, 0), (7, 0), (64, 100), (16, 100)])
def test_structured_masks(n, seq_len):
    """Whole stages of tree keys (seq_len = 0: every key is a tree row), with
    all-visible, self-only, causal, ancestor and root-plus-self masks; with
    no prefix a self-only mask returns exactly the node's own V."""
    _say(f"tree attention structured masks n={n} seq={seq_len}")
    from treemoe_spec_amd.kernels.tree_attention import tree_attention

    kv, q, k, v, anc = _case(n, 8, 2, seq_len, 16, 3)
    eye = torch.eye(n, dtype=torch.bool)
    masks = {"ones": torch.ones(n, n, dtype=torch.bool), "eye": eye,
             "causal": torch.ones(n, n, dtype=torch.bool).tril(), "anc": anc,
             "root": eye | torch.zeros(n, n, dtype=torch.bool).index_fill_(
                 1, torch.tensor([0]), True)}
    for name, m in masks.items():
        out = tree_attention(q.cuda(), k.cuda(), v.cuda(), kv, 0, m.cuda())
        torch.cuda.synchronize()
        _check(out, _oracle(kv, q, k, v, m, 0))
        if name == "eye" and seq_len == 0:
            want = torch.stack([v[:, h // 4] for h in range(8)], 1).reshape(n, -1)
            assert torch.equal(out.cpu(), want), name


@pytest.mark.parametrize("n,seq_len,chunk_keys", [
    (40, 333, 0),
    (200, 333, 64),    # tree rows spread over four chunks, chunk start inside a page
    (130, 0, 64),      # no prefix: every chunk holds tree rows only
])
def test_write_tree_and_nothing_else(n, seq_len, chunk_keys):
    """Each tree row is stored once to its scratch slot by the chunk that
    holds it, whatever the chunking; nothing else in the cache changes."""
    _say(f"tree attention write_tree bytes n={n} seq={seq_len} chunk={chunk_keys}")
    from treemoe_spec_amd.kernels.tree_attention import tree_attention

    page = 16
    kv, q, k, v, mask = _case(n, 16, 4, seq_len, page, 7)
    k0, v0 = kv.k.clone(), kv.v.clone()
    out = tree_attention(q.cuda(), k.cuda(), v.cuda(), kv, 0, mask.cuda(),
                         chunk_keys=chunk_keys)
    torch.cuda.synchronize()
    _check(out, _oracle(kv, q, k, v, mask, 0))
    kk, vv = k0.clone(), v0.clone()
    for j in range(n):
        pg, off = kv.tree_pages[j // page], j % page
        kk[0, pg, off] = k[j].cuda()
        vv[0, pg, off] = v[j].cuda()
    assert torch.equal(kv.k, kk) and torch.equal(kv.v, vv)
    # write_tree=False leaves the cache alone
    kv.k.copy_(k0)
    kv.v.copy_(v0)
    tree_attention(q.cuda(), k.cuda(), v.cuda(), kv, 0, mask.cuda(), write_tree=False,
                   chunk_keys=chunk_keys)
    torch.cuda.synchronize()
    assert torch.equal(kv.k, k0) and torch.equal(kv.v, v0)


def test_deterministic_and_chunking_consistent():
    _say("tree attention determinism")
    from treemoe_spec_amd.kernels.tree_attention import tree_attention

    kv, q, k, v, mask = _case(64, 32, 8, 2000, 16, 11)
    qc, kc, vc, mc = q.cuda(), k.cuda(), v.cuda(), mask.cuda()
    a = tree_attention(qc, kc, vc, kv, 1, mc).clone()
    b = tree_attention(qc, kc, vc, kv, 1, mc).clone()
    assert torch.equal(a, b)
    want = _oracle(kv, q, k, v, mask, 1)
    for ck in (64, 256, 2048 + 64):
        _check(tree_attention(qc, kc, vc, kv, 1, mc, chunk_keys=ck), want)


def test_strided_inputs_and_new_mask_tensor():
    """q/k/v as views of fused projection outputs (node stride > heads * hd),
    and a fresh mask tensor per call (the packed-mask cache must not serve a
    stale mask)."""
    _say("tree attention strided views")
    from treemoe_spec_amd.kernels.tree_attention import tree_attention

    n, hq, kvh = 24, 8, 2
    kv, q, k, v, mask = _case(n, hq, kvh, 77, 16, 5)
    qkv = torch.cat([q.reshape(n, -1), k.reshape(n, -1), v.reshape(n, -1)], 1).cuda()
    qv = qkv[:, : hq * 128].view(n, hq, 128)
    kv_ = qkv[:, hq * 128: (hq + kvh) * 128].view(n, kvh, 128)
    vv = qkv[:, (hq + kvh) * 128:].view(n, kvh, 128)
    out = tree_attention(qv, kv_, vv, kv, 0, mask.cuda())
    _check(out, _oracle(kv, q, k, v, mask, 0))
    for seed in range(3):
        g = torch.Generator().manual_seed(seed)
        parent = [-1] + [int(torch.randint(0, i, (1,), generator=g)) for i in range(1, n)]
        m2 = attn_ref.ancestor_mask(parent)
        out = tree_attention(qv, kv_, vv, kv, 0, m2.cuda())
        _check(out, _oracle(kv, q, k, v, m2, 0))


def test_rejects_bad_inputs():
    from treemoe_spec_amd.kernels.tree_attention import tree_attention

    kv, q, k, v, mask = _case(4, 8, 2, 10, 16, 1)
    with pytest.raises(RuntimeError, match="ROCm"):
        tree_attention(q, k, v, kv, 0, mask)
    with pytest.raises(ValueError, match="bfloat16"):
        tree_attention(q.float().cuda(), k.cuda(), v.cuda(), kv, 0, mask.cuda())
    with pytest.raises(ValueError, match="multiple"):
        tree_attention(q[:, :3].contiguous().cuda(), k.cuda(), v.cuda(), kv, 0, mask.cuda())


def test_reference_cache_layout():
    """A cache with exactly the reference PagedKVCache attributes (page 64,
    scratch block ``tree_block``, no tree_pages / device_tables): the
    attention and its write_tree match the oracle."""
    _say("tree attention through the reference cache layout")
    from tests.ref_layout_cache import RefLayoutKVCache
    from treemoe_spec_amd.kernels.tree_attention import tree_attention

    n, hq, kvh, seq_len = 64, 16, 4, 700
    g = torch.Generator().manual_seed(21)
    kv = RefLayoutKVCache(2, kvh, 128, seq_len // 64 + 5, device="cuda", dtype=torch.bfloat16)
    kv.k.copy_(torch.randn(kv.k.shape, generator=g).to(torch.bfloat16))
    kv.v.copy_(torch.randn(kv.v.shape, generator=g).to(torch.bfloat16))
    perm = torch.randperm(len(kv._free), generator=g).tolist()
    kv._free = [kv._free[i] for i in perm]
    kv._ensure_capacity(seq_len)
    kv.seq_len = seq_len
    q = (torch.randn(n, hq, 128, generator=g) * 3).to(torch.bfloat16)
    k = torch.randn(n, kvh, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(n, kvh, 128, generator=g).to(torch.bfloat16)
    parent = [-1] + [int(torch.randint(0, i, (1,), generator=g)) for i in range(1, n)]
    mask = attn_ref.ancestor_mask(parent)
    want = attn_ref.tree_attention(q, k, v, kv.k.cpu(), kv.v.cpu(), 1, kv.block_table,
                                   seq_len, 64, mask)
    out = tree_attention(q.cuda(), k.cuda(), v.cuda(), kv, 1, mask.cuda())
    torch.cuda.synchronize()
    _check(out, want)
    assert torch.equal(kv.k[1, kv.tree_block, :n].cpu(), k)
    assert torch.equal(kv.v[1, kv.tree_block, :n].cpu(), v)
