"""Paged KV cache consumed by op4's commit (reference: treemoe/model/kv_cache.py).

Layout per tensor: [layers, pages, page_size, kv_heads, head_dim].  The first
``ceil(tree_size / page_size)`` pages are the tree scratch: tree slot s lives in
page ``tree_pages[s // page_size]`` at offset ``s % page_size`` (with the
reference's page size 64 and a 64-node tree this is the single page 0,
``tree_block``).  Sequence position q lives in ``block_table[q // page_size]``
at offset ``q % page_size`` (reference ``slot_of``, :57-58).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

BLOCK_SIZE = 64


@dataclass(frozen=True)
class MixtralConfig:
    """Mixtral-8x7B dimensions (reference: treemoe/model/config.py:10-29)."""

    num_layers: int = 32
    num_experts: int = 8
    top_k: int = 2
    hidden_dim: int = 4096
    intermediate_dim: int = 14336
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 32000
    rope_theta: float = 1e6
    rms_eps: float = 1e-5
    max_seq_len: int = 8192
    dtype: torch.dtype = torch.bfloat16

    @property
    def expert_bytes_per_layer(self) -> int:
        return 3 * self.intermediate_dim * self.hidden_dim * 2


class PagedKVCache:
    def __init__(self, config, num_blocks: int, device: str = "cuda",
                 dtype: torch.dtype = torch.bfloat16, page_size: int = BLOCK_SIZE,
                 tree_size: int = 64):
        self.config = config
        self.block_size = page_size
        n_scratch = (tree_size + page_size - 1) // page_size
        if num_blocks <= n_scratch:
            raise ValueError("num_blocks must exceed the tree scratch pages")
        shape = (config.num_layers, num_blocks, page_size, config.num_kv_heads,
                 config.head_dim)
        self.k = torch.zeros(shape, device=device, dtype=dtype)
        self.v = torch.zeros(shape, device=device, dtype=dtype)
        self.block_table: list[int] = []
        self.seq_len = 0
        self.tree_pages = list(range(n_scratch))
        self.tree_block = self.tree_pages[0]
        self.tree_size = tree_size
        self._free = list(range(num_blocks - 1, n_scratch - 1, -1))
        self._dev_table: torch.Tensor | None = None
        self._dev_table_len = -1
        self._dev_scratch: torch.Tensor | None = None

    def reset(self) -> None:
        """Start a new sequence without clearing the backing tensors."""
        self._free.extend(reversed(self.block_table))
        self.block_table.clear()
        self.seq_len = 0
        self._dev_table_len = -1

    def _ensure_capacity(self, new_len: int) -> None:
        while len(self.block_table) * self.block_size < new_len:
            if not self._free:
                raise RuntimeError("KV cache out of blocks")
            self.block_table.append(self._free.pop())

    def slot_of(self, pos: int) -> tuple[int, int]:
        return self.block_table[pos // self.block_size], pos % self.block_size

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, start_pos: int) -> None:
        """Write [T, kv_heads, head_dim] at positions start_pos .. start_pos+T-1
        (prefill and autoregressive steps; reference kv_cache.py:62-78).  Page
        and offset indices are computed on the host from block_table."""
        t = k.shape[0]
        self._ensure_capacity(start_pos + t)
        bs = self.block_size
        pos = range(start_pos, start_pos + t)
        blks = torch.tensor([self.block_table[q // bs] for q in pos], device=self.k.device,
                            dtype=torch.long)
        offs = torch.tensor([q % bs for q in pos], device=self.k.device, dtype=torch.long)
        self.k[layer, blks, offs] = k
        self.v[layer, blks, offs] = v
        self.seq_len = max(self.seq_len, start_pos + t)

    def write_tree(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write the KV rows of tree nodes 0..n-1 into the scratch pages."""
        n = k.shape[0]
        if n > len(self.tree_pages) * self.block_size:
            raise ValueError("tree larger than the scratch pages")
        for i, page in enumerate(self.tree_pages):
            lo = i * self.block_size
            hi = min(n, lo + self.block_size)
            if hi <= lo:
                break
            self.k[layer, page, : hi - lo] = k[lo:hi]
            self.v[layer, page, : hi - lo] = v[lo:hi]

    def commit_tree(self, accepted_slots: torch.Tensor) -> None:
        """Host-path commit (reference kv_cache.py:88-106): the valid (>= 0)
        tree slots of ``accepted_slots``, in sequence order, are copied from
        the scratch pages to positions seq_len, seq_len+1, ... of every layer,
        and seq_len advances by their number.  Reads the count back to the
        host, as the reference does; the device path is op4's kv commit."""
        valid = accepted_slots[accepted_slots >= 0]
        m = int(valid.numel())
        if m == 0:
            return
        self._ensure_capacity(self.seq_len + m)
        bs = self.block_size
        dev = self.k.device
        slots = valid.to(device=dev, dtype=torch.long)
        pages = torch.tensor(self.tree_pages, device=dev, dtype=torch.long)
        src_p, src_o = pages[slots // bs], slots % bs
        dest = [self.slot_of(self.seq_len + j) for j in range(m)]
        dst_p = torch.tensor([d[0] for d in dest], device=dev, dtype=torch.long)
        dst_o = torch.tensor([d[1] for d in dest], device=dev, dtype=torch.long)
        self.k[:, dst_p, dst_o] = self.k[:, src_p, src_o]
        self.v[:, dst_p, dst_o] = self.v[:, src_p, src_o]
        self.seq_len += m

    def device_tables(self, device) -> tuple[torch.Tensor, torch.Tensor]:
        """int32 copies of block_table and the scratch page list on ``device``,
        refreshed only when the block table has grown."""
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        if self._dev_table is None or self._dev_table_len != len(self.block_table) \
                or self._dev_table.device != device:
            self._dev_table = torch.tensor(self.block_table or [0], dtype=torch.int32,
                                           device=device)
            self._dev_table_len = len(self.block_table)
        if self._dev_scratch is None or self._dev_scratch.device != device:
            self._dev_scratch = torch.tensor(self.tree_pages, dtype=torch.int32, device=device)
        return self._dev_table, self._dev_scratch

    def gather(self, layer: int, upto: int | None = None):
        """Contiguous [T, kv_heads, head_dim] K and V of positions 0..T-1."""
        t = self.seq_len if upto is None else upto
        nblk = (t + self.block_size - 1) // self.block_size
        idx = torch.tensor(self.block_table[:nblk], device=self.k.device, dtype=torch.long)
        kvh, hd = self.k.shape[3], self.k.shape[4]
        k = self.k[layer, idx].reshape(nblk * self.block_size, kvh, hd)[:t]
        v = self.v[layer, idx].reshape(nblk * self.block_size, kvh, hd)[:t]
        return k, v

    def gather_with_tail(self, layer: int, k_tail: torch.Tensor,
                         v_tail: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous [seq_len + T, kv_heads, head_dim] K and V: the committed
        prefix followed by the tree rows (reference kv_cache.py:125-145, the
        input of the reference's SDPA tree attention; this build's tree
        attention reads the pages in place instead)."""
        s, t = self.seq_len, k_tail.shape[0]
        bs = self.block_size
        nblk = (s + bs - 1) // bs
        idx = torch.tensor(self.block_table[:nblk], device=self.k.device, dtype=torch.long)
        kvh, hd = self.k.shape[3], self.k.shape[4]
        m = max(nblk * bs, s + t)
        out_k = torch.empty(m, kvh, hd, device=self.k.device, dtype=self.k.dtype)
        out_v = torch.empty_like(out_k)
        if nblk:
            torch.index_select(self.k[layer], 0, idx,
                               out=out_k[:nblk * bs].view(nblk, bs, kvh, hd))
            torch.index_select(self.v[layer], 0, idx,
                               out=out_v[:nblk * bs].view(nblk, bs, kvh, hd))
        out_k[s:s + t] = k_tail
        out_v[s:s + t] = v_tail
        return out_k[:s + t], out_v[:s + t]


def scratch_pages_of(kv) -> list[int]:
    """Tree scratch pages of a paged cache: ``tree_pages`` of this module's
    cache, or the single ``tree_block`` of the reference's
    (treemoe/model/kv_cache.py:41)."""
    pages = getattr(kv, "tree_pages", None)
    return list(pages) if pages is not None else [int(kv.tree_block)]


# int32 device copies of the block table and scratch pages for caches without
# ``device_tables`` (the reference's PagedKVCache), per cache object and
# device, rebuilt when the host block table or scratch list changes.
_table_cache: dict[tuple, tuple[list, list, torch.Tensor, torch.Tensor]] = {}


def device_tables_of(kv, device) -> tuple[torch.Tensor, torch.Tensor]:
    """(block_table, scratch_pages) as int32 tensors on ``device`` for any
    cache with the reference's attributes (block_table, tree_block or
    tree_pages)."""
    if hasattr(kv, "device_tables"):
        return kv.device_tables(device)
    pages = scratch_pages_of(kv)
    key = (id(kv), torch.device(device))
    hit = _table_cache.get(key)
    if hit is not None and hit[0] == kv.block_table and hit[1] == pages:
        return hit[2], hit[3]
    table = torch.tensor(kv.block_table or [0], dtype=torch.int32, device=device)
    scratch = torch.tensor(pages, dtype=torch.int32, device=device)
    if len(_table_cache) > 16:
        _table_cache.clear()
    _table_cache[key] = (list(kv.block_table), pages, table, scratch)
    return table, scratch
