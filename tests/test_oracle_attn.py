"""CPU: pin the tree-attention oracle.

torch's own scaled_dot_product_attention (enable_gqa, boolean mask) as the
library routine, a float64 brute-force loop at tiny sizes, closed forms (a
root alone returns its own V; identical keys give the mean of the visible V),
page-order independence of the paged gather, and the ancestor-closure mask
against the reference's properties (tests/test_tree.py:43-64) and its DFS
recurrence (treemoe/engine/tree.py:164-171).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attn_ref


def random_parent(n, g):
    return [-1] + [int(torch.randint(0, i, (1,), generator=g)) for i in range(1, n)]


def make_case(n, hq, kvh, hd, seq_len, page, seed, dtype=torch.float32, layers=2):
    g = torch.Generator().manual_seed(seed)
    n_scratch = (n + page - 1) // page
    pages = n_scratch + (seq_len + page - 1) // page + 3
    kc = torch.randn(layers, pages, page, kvh, hd, generator=g).to(dtype)
    vc = torch.randn(layers, pages, page, kvh, hd, generator=g).to(dtype)
    table = (torch.randperm(pages - n_scratch, generator=g) + n_scratch).tolist()
    q = torch.randn(n, hq, hd, generator=g).to(dtype)
    kt = torch.randn(n, kvh, hd, generator=g).to(dtype)
    vt = torch.randn(n, kvh, hd, generator=g).to(dtype)
    parent = random_parent(n, g)
    return q, kt, vt, kc, vc, table, attn_ref.ancestor_mask(parent), parent


@pytest.mark.parametrize("n,hq,kvh,hd,seq_len,page", [
    (1, 4, 2, 16, 0, 16), (7, 8, 2, 32, 5, 16), (16, 4, 4, 8, 100, 64), (64, 8, 2, 16, 37, 16)])
def test_matches_torch_sdpa(n, hq, kvh, hd, seq_len, page):
    q, kt, vt, kc, vc, table, mask, _ = make_case(n, hq, kvh, hd, seq_len, page, n + seq_len)
    got = attn_ref.tree_attention(q, kt, vt, kc, vc, 1, table, seq_len, page, mask)
    # the reference's own composition: gather, mask, SDPA with GQA
    k = torch.cat([attn_ref.gather_prefix(kc, 1, table, seq_len, page), kt])
    v = torch.cat([attn_ref.gather_prefix(vc, 1, table, seq_len, page), vt])
    full = torch.cat([torch.ones(n, seq_len, dtype=torch.bool), mask], 1)
    want = F.scaled_dot_product_attention(
        q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None],
        attn_mask=full[None, None], scale=hd ** -0.5, enable_gqa=True)
    want = want[0].transpose(0, 1).reshape(n, hq * hd)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_brute_force_float64():
    n, hq, kvh, hd, seq_len, page = 5, 4, 2, 4, 6, 4
    q, kt, vt, kc, vc, table, mask, _ = make_case(n, hq, kvh, hd, seq_len, page, 3)
    got = attn_ref.tree_attention(q, kt, vt, kc, vc, 0, table, seq_len, page, mask)
    group = hq // kvh
    for i in range(n):
        for h in range(hq):
            keys, vals = [], []
            for pos in range(seq_len):
                pg, off = table[pos // page], pos % page
                keys.append(kc[0, pg, off, h // group].double())
                vals.append(vc[0, pg, off, h // group].double())
            for j in range(n):
                if mask[i, j]:
                    keys.append(kt[j, h // group].double())
                    vals.append(vt[j, h // group].double())
            s = [float(q[i, h].double() @ k) / math.sqrt(hd) for k in keys]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            o = sum(wi * vi for wi, vi in zip(w, vals)) / sum(w)
            assert torch.allclose(got[i, h * hd:(h + 1) * hd].double(), o, atol=1e-5)


def test_root_alone_returns_its_value():
    q, kt, vt, kc, vc, table, mask, _ = make_case(1, 8, 2, 16, 0, 16, 9)
    got = attn_ref.tree_attention(q, kt, vt, kc, vc, 0, table, 0, 16, mask)
    want = torch.cat([vt[0, h // 4] for h in range(8)])
    torch.testing.assert_close(got[0], want, rtol=0, atol=1e-6)


def test_identical_keys_average_the_visible_values():
    n, hq, kvh, hd, seq_len, page = 6, 2, 1, 8, 9, 4
    q, kt, vt, kc, vc, table, mask, parent = make_case(n, hq, kvh, hd, seq_len, page, 4)
    kc[:] = kc[0, 0, 0]
    kt[:] = kc[0, 0, 0]
    got = attn_ref.tree_attention(q, kt, vt, kc, vc, 0, table, seq_len, page, mask)
    prefix_v = attn_ref.gather_prefix(vc, 0, table, seq_len, page)[:, 0]
    for i in range(n):
        vis = torch.cat([prefix_v, vt[mask[i], 0]])
        torch.testing.assert_close(got[i, :hd], vis.mean(0), rtol=1e-5, atol=1e-6)


def test_page_order_does_not_matter():
    n, hq, kvh, hd, seq_len, page = 8, 4, 2, 16, 50, 16
    q, kt, vt, kc, vc, table, mask, _ = make_case(n, hq, kvh, hd, seq_len, page, 5)
    a = attn_ref.tree_attention(q, kt, vt, kc, vc, 0, table, seq_len, page, mask)
    # move every prefix page to a different physical page
    perm = list(reversed(table))
    kc2, vc2 = kc.clone(), vc.clone()
    for src, dst in zip(table, perm):
        kc2[:, dst] = kc[:, src]
        vc2[:, dst] = vc[:, src]
    b = attn_ref.tree_attention(q, kt, vt, kc2, vc2, 0, perm, seq_len, page, mask)
    assert torch.equal(a, b)


def test_ancestor_mask_properties():
    """Reference tests/test_tree.py:43-64: self and every ancestor visible,
    nothing else; and row(i) = row(parent(i)) | self (engine/tree.py:164-171)."""
    g = torch.Generator().manual_seed(6)
    for n in (1, 2, 17, 64):
        parent = random_parent(n, g)
        m = attn_ref.ancestor_mask(parent)
        rec = torch.zeros(n, n, dtype=torch.bool)
        for i in range(n):
            if parent[i] >= 0:
                rec[i] = rec[parent[i]]
            rec[i, i] = True
        assert torch.equal(m, rec)
        for i in range(n):
            anc = set()
            j = i
            while j >= 0:
                anc.add(j)
                j = parent[j]
            assert set(m[i].nonzero().flatten().tolist()) == anc
