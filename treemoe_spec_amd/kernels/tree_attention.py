"""Tree attention of the verification forward on the paged KV cache.

Drop-in for the tree branch of the reference's ``MixtralForward._attention``
(treemoe/model/mixtral.py:208-250), which runs

    kv.write_tree(layer, k, v)                         # kv_cache.py:80-86
    full_k, full_v = kv.gather_with_tail(layer, k, v)  # kv_cache.py:125-145
    mask = [ones(N, seq_len) | tree_mask]              # mixtral.py:211-218
    o = F.scaled_dot_product_attention(q, full_k, full_v, mask,
                                       scale=hd**-0.5, enable_gqa=True)

as one HIP launch (plus a chunk combine at long contexts): the prefix is read
in place through the block table, the tree rows come from ``k``/``v`` and are
stored into the scratch pages by the same kernel.  The context comes back as
[N, Hq * hd], the layout ``o_proj`` takes (mixtral.py:251-254).
"""

from __future__ import annotations

import ctypes
import weakref

import torch

from treemoe_spec_amd import _capi
from treemoe_spec_amd._capi import call, ptr
from treemoe_spec_amd.kv_cache import device_tables_of, scratch_pages_of

_mask_cache: dict = {}


def pack_tree_mask(tree_mask: torch.Tensor) -> torch.Tensor:
    """[N, N] bool device mask -> [N, ceil(N/64)] int64 bit words (bit j of row
    i = tree_mask[i, j]); cached per live mask tensor and its version counter,
    since the engine reuses one mask for every layer of a step."""
    hit = _mask_cache.get(id(tree_mask))
    if hit is not None and hit[0]() is tree_mask and hit[1] == tree_mask._version:
        return hit[2]
    n = tree_mask.shape[0]
    if tree_mask.dim() != 2 or tree_mask.shape[1] != n or tree_mask.stride(1) != 1:
        raise ValueError("tree_mask must be [N, N] with unit stride along columns")
    m = tree_mask if tree_mask.dtype in (torch.bool, torch.uint8) else tree_mask.bool()
    bits = torch.empty(n, (n + 63) // 64, dtype=torch.int64, device=tree_mask.device)
    call("tm_tree_mask_pack", ptr(m), n, m.stride(0), ptr(bits),
         _capi.stream_of(tree_mask.device))
    if len(_mask_cache) > 16:
        _mask_cache.clear()
    _mask_cache[id(tree_mask)] = (weakref.ref(tree_mask), tree_mask._version, bits)
    return bits


def tree_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv, layer: int,
                   tree_mask: torch.Tensor, scale: float | None = None,
                   out: torch.Tensor | None = None, write_tree: bool = True,
                   chunk_keys: int = 0) -> torch.Tensor:
    """q [N, Hq, hd] (after RoPE), k/v [N, kvh, hd] (k after RoPE) for the tree
    nodes; ``kv`` a paged cache with ``seq_len`` committed positions.  Returns
    the attention context [N, Hq * hd] bf16.  ``write_tree`` also stores k/v
    in the scratch pages, as the reference's write_tree does."""
    if not q.is_cuda:
        raise RuntimeError("treemoe_spec_amd tree attention runs on ROCm devices only; "
                           "got a CPU tensor")
    n, hq, hd = q.shape
    if k.shape[0] != n or v.shape != k.shape or k.dim() != 3:
        raise ValueError("k and v must be [N, kv_heads, head_dim] like q's N")
    kvh = k.shape[1]
    if hq % kvh != 0:
        raise ValueError("num_heads must be a multiple of num_kv_heads")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16")
        if t.stride(2) != 1 or t.stride(1) != hd:
            raise ValueError(f"{name} must have contiguous heads")
    if k.stride(0) != v.stride(0):
        raise ValueError("k and v must share the node stride")
    if kv.k.dtype != torch.bfloat16 or kv.k.shape[3] != kvh or kv.k.shape[4] != hd:
        raise ValueError("cache layout must be [L, pages, page, kv_heads, head_dim] bf16")
    if tuple(tree_mask.shape) != (n, n):
        raise ValueError("tree_mask must be [N, N]")
    dev = q.device
    if scale is None:
        scale = hd ** -0.5
    bits = pack_tree_mask(tree_mask)
    pages = scratch_pages_of(kv)
    if write_tree and len(pages) * kv.block_size < n:
        raise ValueError("tree larger than the KV scratch pages")
    table, scratch = device_tables_of(kv, dev)
    seq_len = kv.seq_len
    chunks = ctypes.c_int64()
    wbytes = ctypes.c_int64()
    call("tm_tree_attention_plan", n, hq, kvh, hd, seq_len, kv.block_size, chunk_keys,
         ctypes.byref(chunks), ctypes.byref(wbytes))
    ws = _workspace(wbytes.value, dev)
    if out is None:
        out = torch.empty(n, hq * hd, dtype=torch.bfloat16, device=dev)
    elif out.shape != (n, hq * hd) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous [N, Hq * hd] bf16 tensor")
    kc = kv.k[layer]
    vc = kv.v[layer]
    call("tm_tree_attention", ptr(q), q.stride(0), ptr(k), ptr(v), k.stride(0), ptr(kc),
         ptr(vc), kc.stride(0), kc.stride(1), kv.block_size, ptr(table),
         max(1, len(kv.block_table)), seq_len, ptr(scratch), len(pages),
         1 if write_tree else 0, ptr(bits), n, hq, kvh, hd, float(scale), ptr(out), hq * hd,
         chunk_keys, ptr(ws), wbytes.value, _capi.stream_of(dev))
    return out


_ws_cache: dict = {}


def _workspace(nbytes: int, device) -> torch.Tensor | None:
    """Chunk partials; one buffer per device, grown on demand (stream-ordered
    reuse, like the reference's per-shape workspaces)."""
    if nbytes == 0:
        return None
    key = torch.device(device)
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _ws_cache[key] = buf
    return buf
