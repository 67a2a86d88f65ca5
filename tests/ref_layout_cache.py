"""Test double with exactly the attribute set of the reference's PagedKVCache
(treemoe/model/kv_cache.py:19-58): one scratch block ``tree_block``, page
size 64, ``block_table``, ``seq_len``, ``_ensure_capacity`` and ``slot_of``,
and no ``tree_pages`` / ``device_tables``.  Used to show that op4's commit and
the tree attention accept the reference's cache unchanged."""

from __future__ import annotations

import torch

PAGE = 64


class RefLayoutKVCache:
    def __init__(self, num_layers: int, kv_heads: int, head_dim: int, num_blocks: int,
                 device="cuda", dtype=torch.bfloat16):
        self.block_size = PAGE
        shape = (num_layers, num_blocks, PAGE, kv_heads, head_dim)
        self.k = torch.zeros(shape, device=device, dtype=dtype)
        self.v = torch.zeros(shape, device=device, dtype=dtype)
        self.block_table: list[int] = []
        self.seq_len = 0
        self.tree_block = 0
        # every block except the scratch one is free, popped from the end
        self._free = [b for b in range(num_blocks - 1, 0, -1)]

    def _ensure_capacity(self, new_len: int) -> None:
        while self.block_size * len(self.block_table) < new_len:
            if not self._free:
                raise RuntimeError("KV cache out of blocks")
            self.block_table.append(self._free.pop())

    def slot_of(self, pos: int) -> tuple[int, int]:
        return self.block_table[pos // PAGE], pos % PAGE
