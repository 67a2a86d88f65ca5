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

    # Positions map to flat slots of the [pages * page_size] axis:
    # slot = block_table[q // page_size] * page_size + q % page_size.  The
    # host-side paths below (prefill append, the reference's gather for SDPA,
    # the host commit) all go through that map and index_select / index_copy_
    # on the flat view, one op per tensor.

    def reset(self) -> None:
        """Start a new sequence; the backing tensors keep their contents and
        the sequence's pages return to the free list."""
        while self.block_table:
            self._free.append(self.block_table.pop())
        self.seq_len = 0
        self._dev_table_len = -1

    def _ensure_capacity(self, new_len: int) -> None:
        """Map enough pages for positions 0 .. new_len - 1."""
        missing = -(-new_len // self.block_size) - len(self.block_table)
        if missing <= 0:
            return
        if missing > len(self._free):
            raise RuntimeError("KV cache out of blocks")
        for _ in range(missing):
            self.block_table.append(self._free.pop())

    def slot_of(self, pos: int) -> tuple[int, int]:
        page, off = divmod(pos, self.block_size)
        return self.block_table[page], off

    def _flat_slots(self, start: int, count: int) -> torch.Tensor:
        """Flat slots of positions start .. start + count - 1 (mapped pages)."""
        dev = self.k.device
        pos = torch.arange(start, start + count, device=dev, dtype=torch.long)
        table = torch.tensor(self.block_table, device=dev, dtype=torch.long)
        return table[pos // self.block_size] * self.block_size + pos % self.block_size

    def _flat(self, t: torch.Tensor, layer: int) -> torch.Tensor:
        """[pages * page_size, kv_heads, head_dim] view of one layer."""
        return t[layer].flatten(0, 1)

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, start_pos: int) -> None:
        """Write [T, kv_heads, head_dim] at positions start_pos .. start_pos+T-1
        (prefill and autoregressive steps; the contract of the reference's
        append, kv_cache.py:62-78)."""
        t = k.shape[0]
        self._ensure_capacity(start_pos + t)
        slots = self._flat_slots(start_pos, t)
        self._flat(self.k, layer).index_copy_(0, slots, k.to(self.k.dtype))
        self._flat(self.v, layer).index_copy_(0, slots, v.to(self.v.dtype))
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
        src = pages[slots // bs] * bs + slots % bs
        dst = self._flat_slots(self.seq_len, m)
        for cache in (self.k, self.v):
            flat = cache.flatten(1, 2)  # [layers, pages * page_size, kv_heads, head_dim]
            flat[:, dst] = flat[:, src]
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
        """Contiguous [T, kv_heads, head_dim] K and V of positions 0..T-1
        (the reference's gather, kv_cache.py:110-123)."""
        t = self.seq_len if upto is None else upto
        slots = self._flat_slots(0, t)
        return (self._flat(self.k, layer).index_select(0, slots),
                self._flat(self.v, layer).index_select(0, slots))

    def gather_with_tail(self, layer: int, k_tail: torch.Tensor,
                         v_tail: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous [seq_len + T, kv_heads, head_dim] K and V: the committed
        prefix followed by the tree rows, each written once into the result
        (the contract of the reference's gather_with_tail, kv_cache.py:125-145,
        the input of its SDPA tree attention; this build's tree attention
        reads the pages in place instead)."""
        s, t = self.seq_len, k_tail.shape[0]
        slots = self._flat_slots(0, s)
        out = []
        for cache, tail in ((self.k, k_tail), (self.v, v_tail)):
            buf = torch.empty((s + t,) + tuple(cache.shape[3:]), device=cache.device,
                              dtype=cache.dtype)
            torch.index_select(self._flat(cache, layer), 0, slots, out=buf[:s])
            buf[s:] = tail
            out.append(buf)
        return out[0], out[1]


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
