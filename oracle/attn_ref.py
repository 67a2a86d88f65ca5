"""TEST INFRASTRUCTURE ONLY: restatement of the reference's tree attention.

The verification forward of the reference attends every tree node to the
whole committed prefix plus its own ancestors (and itself) in the tree:

* ``write_tree`` / ``gather_with_tail``  treemoe/model/kv_cache.py:80-86,
  125-145: the prefix K/V of positions 0..seq_len-1 is gathered page by page
  through ``block_table`` and the tree K/V (the rows just computed) is
  appended after it; the tree rows are also stored in the scratch pages.
* the mask  treemoe/model/mixtral.py:208-218: [N, seq_len + N], all prefix
  columns visible, the tree columns given by ``tree_mask`` (ancestor-or-self).
* ``F.scaled_dot_product_attention(q, k, v, attn_mask, scale=hd**-0.5,
  enable_gqa=True)``  mixtral.py:241-250: query head h reads kv head
  h // (Hq / kvh); the context is [N, Hq * hd].

Everything here runs on the CPU in float32 (inputs widened from bf16).
"""

from __future__ import annotations

import torch


def gather_prefix(cache: torch.Tensor, layer: int, block_table: list[int], seq_len: int,
                  page_size: int) -> torch.Tensor:
    """[seq_len, kvh, hd] rows of positions 0..seq_len-1 (kv_cache.py:110-123)."""
    if seq_len == 0:
        return cache.new_zeros((0,) + tuple(cache.shape[3:]))
    nblk = (seq_len + page_size - 1) // page_size
    idx = torch.tensor(block_table[:nblk], dtype=torch.long)
    rows = cache[layer].index_select(0, idx.to(cache.device))
    return rows.reshape(nblk * page_size, *cache.shape[3:])[:seq_len]


def tree_attention(q: torch.Tensor, k_tail: torch.Tensor, v_tail: torch.Tensor,
                   k_cache: torch.Tensor, v_cache: torch.Tensor, layer: int,
                   block_table: list[int], seq_len: int, page_size: int,
                   tree_mask: torch.Tensor, scale: float | None = None) -> torch.Tensor:
    """q [N, Hq, hd]; k_tail, v_tail [N, kvh, hd]; caches [L, pages, page, kvh, hd];
    tree_mask [N, N] bool.  Returns the context [N, Hq * hd] in float32."""
    n, hq, hd = q.shape
    kvh = k_tail.shape[1]
    if scale is None:
        scale = hd ** -0.5
    k = torch.cat([gather_prefix(k_cache, layer, block_table, seq_len, page_size).cpu(),
                   k_tail.cpu()]).float()
    v = torch.cat([gather_prefix(v_cache, layer, block_table, seq_len, page_size).cpu(),
                   v_tail.cpu()]).float()
    mask = torch.zeros(n, seq_len + n, dtype=torch.bool)
    mask[:, :seq_len] = True
    mask[:, seq_len:] = tree_mask.cpu().bool()
    group = hq // kvh
    qf = q.cpu().float()
    out = torch.empty(n, hq, hd)
    for h in range(hq):
        kh = k[:, h // group]                      # [S+N, hd]
        vh = v[:, h // group]
        s = (qf[:, h] @ kh.T) * scale              # [N, S+N]
        s = s.masked_fill(~mask, float("-inf"))
        out[:, h] = torch.softmax(s, dim=-1) @ vh
    return out.reshape(n, hq * hd)


def ancestor_mask(parent: list[int]) -> torch.Tensor:
    """[N, N] bool: mask[i, j] iff j is i or an ancestor of i (parent[0] = -1)."""
    n = len(parent)
    m = torch.zeros(n, n, dtype=torch.bool)
    for i in range(n):
        j = i
        while j >= 0:
            m[i, j] = True
            j = parent[j]
    return m
