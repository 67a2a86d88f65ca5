"""op1: tree-aware grouped MoE layer (with op3 budget routing) on MI355X.

Same Python surface as the reference module treemoe/kernels/op1_tree_moe.py
(``compact_block_limit`` :66, ``compact_block_capacity`` :74, ``route_and_bucket``
:81, ``Routing`` :568, ``route_experts`` :641, ``tree_moe_forward`` :711); the
work runs in libtreemoe_amd.so:

  routing      tm_op1_route          router (bf16 logits, fp32 softmax), then
                                     budget routing + bucketing (two launches);
                                     at few tokens on the tiled path the
                                     bucketing runs inside the gate/up launch
                                     (tm_op1_prefill_gemm1_routed)
  gate/up      tm_op1_gemm1          MFMA, SwiGLU fused, h kept in bf16
  down         tm_op1_gemm2          MFMA, deterministic K split, gate applied
  combine      tm_op1_combine        fixed order, bf16 output

At many rows per expert (uses_tiled_gemms) gate/up and down run as
tm_op1_prefill_gemm1 / tm_op1_prefill_gemm2, MFMA-tiled over rows and weights.

There is no CPU path: CPU tensors, other dtypes, or a missing library raise.
"""

from __future__ import annotations

import os

import torch

from treemoe_spec_amd import _capi
from treemoe_spec_amd._capi import TM_GEMM_TILE_M, TM_OBJECTIVE, call, ptr

BM = int(os.getenv("TREEMOE_BLOCK_M", "16"))
if BM not in {16, 32}:
    raise ValueError("TREEMOE_BLOCK_M must be 16 or 32")

# K segments of the down projection.  Each segment is one deterministic
# partial; more segments = more, shorter workgroups and more partial traffic.
# Measured at the Mixtral shape on MI355X (T=64, B=8): 1 and 2 segments are
# within 2 us per layer (478.5 and 476.8 us); 4 makes the down GEMM ~9 %
# slower.
SPLIT_K = 2
TILE_M = TM_GEMM_TILE_M


def compact_block_limit(num_slots: int, expert_budget: int, block_m: int = BM) -> int:
    """Tight upper bound on the compact blocks of S slots over <= B experts."""
    active_upper = min(num_slots, expert_budget)
    return active_upper + (num_slots - active_upper) // block_m


def compact_block_capacity(num_slots: int, expert_budget: int, block_m: int = BM) -> int:
    """Power-of-two storage capacity for a compact expert-major bucket."""
    logical = compact_block_limit(num_slots, expert_budget, block_m)
    return 1 << max(logical - 1, 0).bit_length()


# Rows per active expert from which the MFMA-tiled GEMMs (tiles that reuse
# each weight tile across rows) replace the weight-streaming GEMMs (one pass
# over an expert's weights per 64-row tile).  The tiled pair streams a
# single-tile expert's weights with the non-temporal policy, so it also wins
# at few rows per expert when the FFN is wide enough to fill the chip with
# column jobs.  Measured at the Mixtral shape (H=4096, E=8, B=8, forward us,
# streaming / tiled): I=14336 at 8 rows per expert (T=32) 459 / 453, 16 rows
# (T=64, config 2) 476 / 457, 32 rows (T=128) 609 / 477; at 4 rows (T=16)
# 436 / 448.  With the 64-row gate/up tile for few rows per expert, 16 rows
# per expert: I=7168 262 / 242, I=3584 148 / 132 (8 rows 135 / 129; B=4 104 /
# 100), I=1792 89 / 101 (8 rows 83 / 95).
TILED_MIN_ROWS = 32           # tiled from this many rows per routed expert ..
TILED_MIN_ROWS_WIDE = 8       # .. or from this many when inter >= TILED_WIDE_INTER
TILED_WIDE_INTER = 3584


def uses_tiled_gemms(num_tokens: int, expert_budget: int, num_experts: int,
                     inter: int = 0) -> bool:
    """True when the average rows per routed expert reach TILED_MIN_ROWS, or
    TILED_MIN_ROWS_WIDE for an intermediate size of TILED_WIDE_INTER or more."""
    active = min(expert_budget, num_experts)
    if 2 * num_tokens >= TILED_MIN_ROWS * active:
        return True
    return inter >= TILED_WIDE_INTER and 2 * num_tokens >= TILED_MIN_ROWS_WIDE * active


def tiled_gate_up_tile(num_tokens: int, num_experts: int, max_tiles: int) -> str:
    """The tile tm_op1_prefill_gemm1 picks (the rule in op1_prefill.hip):
    256-row tiles when the experts average 384 rows or more, the 64-row
    decode tile when the tile list leaves at most 16 rows per entry, else
    128-row tiles.  For naming kernels in measurements."""
    if 2 * num_tokens >= 384 * num_experts:
        return "Tile<256, 32, 4>"
    if 2 * num_tokens <= 16 * max_tiles:
        return "Tile<64, 64, 3, 128, 256>"
    return "Tile<128, 64, 3>"


def _split_for(inter: int) -> int:
    for s in (SPLIT_K, 2, 1):
        if s >= 1 and inter % s == 0 and (inter // s) % 256 == 0:
            return s
    raise ValueError("intermediate size must be a multiple of 256")


# The tiled down GEMM launches (real M-tiles) x (hidden / 256) x split jobs.
# With few rows per layer (config 3: 4 experts, 128 rows) split 2 fills only
# half the 256 CUs; 4 K segments fill one round: measured 120 -> 96 us at
# T=64, B=4 (7 or 8 segments: 105-107 us).  Partials of 4 segments are kept
# only where they are small.
TILED_SPLIT_WIDE = 4
_TILED_WIDE_MAX_BYTES = 64 << 20
_CUS = 256


def _tiled_split(n: int, expert_budget: int, num_experts: int, hidden: int, inter: int,
                 ws: "_Workspace") -> int:
    """K segments for the tiled down GEMM: TILED_SPLIT_WIDE when split 2 would
    leave CUs idle and the workspace holds that many partials, else ws.split."""
    s = TILED_SPLIT_WIDE
    mtiles = -(-2 * n // 128) + min(expert_budget, num_experts)  # bound on real 128-row M-tiles
    if (ws.partial.shape[0] >= s and inter % s == 0 and (inter // s) % 64 == 0
            and mtiles * (hidden // 256) * ws.split < _CUS):
        return s
    return ws.split


def _check_budget(expert_budget: int, num_experts: int, routing_objective: str) -> None:
    if not 2 <= expert_budget <= num_experts:
        raise ValueError(f"expert_budget must be in [2, {num_experts}]")
    if routing_objective not in TM_OBJECTIVE:
        raise ValueError("routing_objective must be 'mass' or 'critical_path'")


def _require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "treemoe_spec_amd op1 runs on ROCm devices only; got a CPU tensor "
                "(no CPU fallback is provided)")


_DTYPE_CODE = {torch.bfloat16: _capi.TM_DTYPE_BF16, torch.float16: _capi.TM_DTYPE_F16}


def _require_half(name: str, t: torch.Tensor, like: torch.Tensor | None = None) -> int:
    """The C-ABI dtype code of a contiguous bf16 or fp16 tensor (the
    reference kernels take either, op1_tree_moe.py:762-766); ``like`` fixes
    the dtype all operands must share."""
    if t.dtype not in _DTYPE_CODE:
        raise TypeError(f"{name} must be torch.bfloat16 or torch.float16, got {t.dtype}")
    if like is not None and t.dtype != like.dtype:
        raise TypeError(f"{name} must have x's dtype {like.dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return _DTYPE_CODE[t.dtype]


class _Workspace:
    """Static per-shape device buffers, rewritten by every call."""

    def __init__(self, n: int, e: int, hidden: int, inter: int, device, dtype):
        self.max_blocks = compact_block_capacity(2 * n, e, BM)
        self.max_tiles = compact_block_limit(2 * n, e, TILE_M)
        self.num_experts = e
        self.rows = self.max_blocks * BM
        self.split = _split_for(inter)
        # the tiled down GEMM may use more K segments at small shapes
        wide = TILED_SPLIT_WIDE * 2 * n * hidden * 4 <= _TILED_WIDE_MAX_BYTES
        nsplit = max(self.split, TILED_SPLIT_WIDE) if wide else self.split
        i32, i64, f32 = torch.int32, torch.int64, torch.float32
        self.router_gates = torch.empty(n, e, dtype=f32, device=device)
        # gate/up output, tile-swizzled: max_tiles x 64 rows x inter (A-fragment order)
        self.h = torch.empty(self.max_tiles * TILE_M, inter, dtype=dtype, device=device)
        self.partial = torch.zeros(nsplit, 2 * n, hidden, dtype=f32, device=device)
        self.topk_flat = torch.zeros(2 * n, dtype=i64, device=device)
        self.gates_flat = torch.zeros(2 * n, dtype=f32, device=device)
        self.padded_slots = torch.full((self.rows,), -1, dtype=i64, device=device)
        self.block_expert_ids = torch.full((self.max_blocks,), -1, dtype=i64, device=device)
        self.slot_to_row = torch.zeros(2 * n, dtype=i64, device=device)
        self.demand = torch.zeros(e, dtype=f32, device=device)
        self.expert_offsets = torch.zeros(e + 1, dtype=i32, device=device)
        self.sorted_slots = torch.zeros(2 * n, dtype=i32, device=device)
        self.slot_pos = torch.zeros(2 * n, dtype=i32, device=device)
        self.tiles = torch.zeros(self.max_tiles, 4, dtype=i32, device=device)


_ws_cache: dict[tuple, _Workspace] = {}


def _workspace(n: int, e: int, hidden: int, inter: int, x: torch.Tensor) -> _Workspace:
    key = (n, e, hidden, inter, x.device.index, x.dtype, BM)
    ws = _ws_cache.get(key)
    if ws is None:
        ws = _ws_cache[key] = _Workspace(n, e, hidden, inter, x.device, x.dtype)
    return ws


def _launch_router(x: torch.Tensor, router_weight: torch.Tensor, gates: torch.Tensor) -> None:
    n, hidden = x.shape
    call("tm_op1_router_gates", ptr(x), ptr(router_weight), n, hidden,
         router_weight.shape[0], ptr(gates), _DTYPE_CODE[x.dtype], _capi.stream_of(x.device))


def _launch_route_bucket(gates, accept, n, e, budget, tau, objective, block_m, max_blocks,
                         max_tiles, topk, gates_flat, padded, blk, s2r, demand, offsets,
                         sorted_slots, slot_pos, tiles, device) -> None:
    call("tm_op1_route_bucket", ptr(gates), ptr(accept), n, e, budget, float(tau),
         TM_OBJECTIVE[objective], block_m, max_blocks, max_tiles, ptr(topk),
         ptr(gates_flat), ptr(padded), ptr(blk), ptr(s2r), ptr(demand), ptr(offsets),
         ptr(sorted_slots), ptr(slot_pos), ptr(tiles), _capi.stream_of(device))


def _launch_route(x, router_weight, accept, budget, tau, objective, block_m, max_blocks,
                  max_tiles, gates, topk, gates_flat, padded, blk, s2r, demand, offsets,
                  sorted_slots, slot_pos, tiles) -> None:
    n, hidden = x.shape
    call("tm_op1_route", ptr(x), ptr(router_weight), ptr(accept), n, hidden,
         router_weight.shape[0], budget, float(tau), TM_OBJECTIVE[objective], block_m,
         max_blocks, max_tiles, ptr(gates), ptr(topk), ptr(gates_flat), ptr(padded), ptr(blk),
         ptr(s2r), ptr(demand), ptr(offsets), ptr(sorted_slots), ptr(slot_pos), ptr(tiles),
         _DTYPE_CODE[x.dtype], _capi.stream_of(x.device))


def _prep_accept(node_accept_prob: torch.Tensor, n: int) -> torch.Tensor:
    a = node_accept_prob
    if a.dtype != torch.float32 or not a.is_contiguous():
        a = a.float().contiguous()
    if a.numel() != n:
        raise ValueError(f"node_accept_prob must have {n} elements, got {a.numel()}")
    return a


def route_and_bucket(
    x: torch.Tensor,
    router_weight: torch.Tensor,
    node_accept_prob: torch.Tensor,
    expert_budget: int,
    block_m: int = BM,
    top1_threshold: float = 0.05,
    return_demand: bool = False,
    router_gates: torch.Tensor | None = None,
    routing_objective: str = "mass",
):
    """Returns (topk_ids [N,2], topk_gates [N,2], padded_slots, block_expert_ids,
    slot_to_row, max_blocks[, demand]) in fresh tensors, like the reference's
    torch composition (treemoe/kernels/op1_tree_moe.py:81-149)."""
    _require_device(x, router_weight, node_accept_prob)
    n = x.shape[0]
    e = router_weight.shape[0]
    _check_budget(expert_budget, e, routing_objective)
    if block_m not in (16, 32):
        raise ValueError("block_m must be 16 or 32")
    dev = x.device
    accept = _prep_accept(node_accept_prob, n)
    max_blocks = compact_block_capacity(2 * n, expert_budget, block_m)
    max_tiles = compact_block_limit(2 * n, expert_budget, TILE_M)
    i32, i64, f32 = torch.int32, torch.int64, torch.float32
    topk = torch.empty(2 * n, dtype=i64, device=dev)
    gflat = torch.empty(2 * n, dtype=f32, device=dev)
    padded = torch.empty(max_blocks * block_m, dtype=i64, device=dev)
    blk = torch.empty(max_blocks, dtype=i64, device=dev)
    s2r = torch.empty(2 * n, dtype=i64, device=dev)
    demand = torch.empty(e, dtype=f32, device=dev)
    offsets = torch.empty(e + 1, dtype=i32, device=dev)
    sorted_slots = torch.empty(2 * n, dtype=i32, device=dev)
    slot_pos = torch.empty(2 * n, dtype=i32, device=dev)
    tiles = torch.empty(max_tiles, 4, dtype=i32, device=dev)
    if router_gates is None:
        _require_half("x", x)
        _require_half("router_weight", router_weight, like=x)
        gates = torch.empty(n, e, dtype=torch.float32, device=dev)
        _launch_route(x, router_weight, accept, expert_budget, top1_threshold,
                      routing_objective, block_m, max_blocks, max_tiles, gates, topk, gflat,
                      padded, blk, s2r, demand, offsets, sorted_slots, slot_pos, tiles)
    else:
        gates = router_gates.float().contiguous()
        _launch_route_bucket(gates, accept, n, e, expert_budget, top1_threshold,
                             routing_objective, block_m, max_blocks, max_tiles, topk, gflat,
                             padded, blk, s2r, demand, offsets, sorted_slots, slot_pos, tiles,
                             dev)
    result = (topk.view(n, 2), gflat.view(n, 2), padded, blk, s2r, max_blocks)
    if return_demand:
        return (*result, demand)
    return result


class Routing:
    """Phase-1 result of tree_moe_forward: routing + bucketing, no expert
    weights touched (reference: treemoe/kernels/op1_tree_moe.py:568-638).

    The reference attributes are views of the workspace; ``expert_offsets``,
    ``sorted_slots``, ``slot_pos`` and ``tiles`` are the compact layout the
    GEMMs consume.  A later route_experts() call with the same shape rewrites
    the workspace, as in the reference."""

    __slots__ = ("ws", "router_gates", "topk_ids", "gates_flat", "padded_slots",
                 "block_expert_ids", "slot_to_row", "max_blocks", "launch_blocks",
                 "demand", "expert_offsets", "sorted_slots", "slot_pos", "tiles",
                 "max_tiles")

    def __init__(self, ws, router_gates, topk_ids, gates_flat, padded_slots,
                 block_expert_ids, slot_to_row, max_blocks, launch_blocks, demand,
                 expert_offsets, sorted_slots, slot_pos, tiles, max_tiles):
        self.ws = ws
        self.router_gates = router_gates
        self.topk_ids = topk_ids
        self.gates_flat = gates_flat
        self.padded_slots = padded_slots
        self.block_expert_ids = block_expert_ids
        self.slot_to_row = slot_to_row
        self.max_blocks = max_blocks
        self.launch_blocks = launch_blocks
        self.demand = demand
        self.expert_offsets = expert_offsets
        self.sorted_slots = sorted_slots
        self.slot_pos = slot_pos
        self.tiles = tiles
        self.max_tiles = max_tiles

    def expert_ids(self) -> list[int]:
        """Experts routed this layer (one small device-to-host copy)."""
        ids = self.block_expert_ids[: self.launch_blocks].tolist()
        return sorted({int(i) for i in ids if i >= 0})

    def exclude_experts(self, expert_ids) -> list[tuple[int, torch.Tensor, torch.Tensor]]:
        """Drop these experts from the device pass and return
        [(expert, token_idx, gates)] host tensors for a host-side FFN
        (reference :598-638).  As in the reference, their slots' gates in
        ``gates_flat`` are zeroed, their GEMM tiles and reference blocks are
        masked and their partial rows zeroed, so the fixed-order combine adds
        exact zeros for them."""
        picked: list[tuple[int, torch.Tensor, torch.Tensor]] = []
        offsets = self.expert_offsets.tolist()
        drop = []
        rows = []
        cold_slots = []
        for e in expert_ids:
            e = int(e)
            lo, hi = offsets[e], offsets[e + 1]
            if hi <= lo:
                continue
            slots = self.sorted_slots[lo:hi].long()
            picked.append((e, (slots // 2).cpu(), self.gates_flat[slots].float().cpu()))
            drop.append(e)
            rows.append(torch.arange(lo, hi, device=slots.device))
            cold_slots.append(slots)
        if not picked:
            return picked
        self.gates_flat[torch.cat(cold_slots)] = 0.0
        drop_t = torch.tensor(drop, device=self.tiles.device)
        tile_e = self.tiles[:, 0]
        self.tiles[:, 0] = torch.where(torch.isin(tile_e.long(), drop_t),
                                       torch.full_like(tile_e, -1), tile_e)
        blk = self.block_expert_ids
        blk[torch.isin(blk, drop_t)] = -1
        self.ws.partial[:, torch.cat(rows)] = 0.0
        return picked


def _routing_of(ws: _Workspace, n: int, expert_budget: int) -> Routing:
    """The Routing handle over the workspace's routing buffers."""
    max_blocks = compact_block_capacity(2 * n, expert_budget, BM)
    launch_blocks = compact_block_limit(2 * n, expert_budget, BM)
    max_tiles = compact_block_limit(2 * n, expert_budget, TILE_M)
    return Routing(ws, ws.router_gates, ws.topk_flat.view(n, 2), ws.gates_flat,
                   ws.padded_slots[: max_blocks * BM], ws.block_expert_ids[:max_blocks],
                   ws.slot_to_row, max_blocks, launch_blocks, ws.demand, ws.expert_offsets,
                   ws.sorted_slots, ws.slot_pos, ws.tiles[:max_tiles], max_tiles)


def _check_router(x: torch.Tensor, router_weight: torch.Tensor) -> None:
    if router_weight.shape[1] != x.shape[1]:
        raise ValueError("router_weight must be [E, H] with H = x.shape[1]")


def route_experts(
    x: torch.Tensor,
    router_weight: torch.Tensor,
    node_accept_prob: torch.Tensor,
    expert_budget: int,
    inter: int,
    top1_threshold: float = 0.05,
    routing_objective: str = "mass",
) -> Routing:
    """Phase 1 of tree_moe_forward: router + op3 budget routing + bucketing.
    Reads only the router weights; ``inter`` is the FFN size (sizes the
    workspace)."""
    _check_budget(expert_budget, router_weight.shape[0], routing_objective)
    _require_device(x, router_weight, node_accept_prob)
    _require_half("x", x)
    _require_half("router_weight", router_weight, like=x)
    _check_router(x, router_weight)
    n, hidden = x.shape
    e = router_weight.shape[0]
    ws = _workspace(n, e, hidden, inter, x)
    accept = _prep_accept(node_accept_prob, n)
    r = _routing_of(ws, n, expert_budget)
    _launch_route(x, router_weight, accept, expert_budget, top1_threshold, routing_objective,
                  BM, r.max_blocks, r.max_tiles, ws.router_gates, ws.topk_flat, ws.gates_flat,
                  r.padded_slots, r.block_expert_ids, ws.slot_to_row, ws.demand,
                  ws.expert_offsets, ws.sorted_slots, ws.slot_pos, r.tiles)
    return r


# At few tokens the tiled gate/up launch routes its own jobs and writes the
# routing outputs itself (tm_op1_prefill_gemm1_routed): the budget routing and
# bucketing launch and its launch gap leave the layer's critical path.  Limits
# of that entry point (one token per lane of a wave, a token's gates in
# registers):
SELF_ROUTED_MAX_TOKENS = 64
SELF_ROUTED_MAX_EXPERTS = 16
_SELF_ROUTED_MAX_BLOCKS = 256      # compact_block_capacity(2T, B, BM)


def self_routed(num_tokens: int, expert_budget: int, num_experts: int, inter: int) -> bool:
    """True when tree_moe_forward (without a precomputed routing) runs the
    routing inside the gate/up launch: the tiled GEMMs at few tokens."""
    return (uses_tiled_gemms(num_tokens, expert_budget, num_experts, inter)
            and num_tokens <= SELF_ROUTED_MAX_TOKENS
            and num_experts <= SELF_ROUTED_MAX_EXPERTS
            and compact_block_capacity(2 * num_tokens, expert_budget, BM)
            <= _SELF_ROUTED_MAX_BLOCKS)


def tree_moe_forward(
    x: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    w3: torch.Tensor,
    router_weight: torch.Tensor,
    node_accept_prob: torch.Tensor,
    expert_budget: int,
    out: torch.Tensor | None = None,
    deterministic: bool = True,
    routing: Routing | None = None,
    routing_objective: str = "mass",
) -> torch.Tensor:
    """op1 entry point (reference :711-802).

    Always bitwise deterministic: the down projection writes K-split partials
    and the combine sums them in a fixed order, so ``deterministic=False``
    (the reference's atomic variant) returns the same bits.  ``routing`` is a
    precomputed phase-1 handle from route_experts(); None routes inline."""
    return _forward(x, w1, w2, w3, router_weight, node_accept_prob, expert_budget, out,
                    routing, routing_objective)


def _forward(x, w1, w2, w3, router_weight, node_accept_prob, expert_budget, out, routing,
             routing_objective, on_phase=None) -> torch.Tensor:
    """tree_moe_forward's launches.  ``on_phase(name)``, when given, is called
    after the launches of each phase ("route", "gemm1", "gemm2", "combine"):
    the benchmark records its events there."""
    _check_budget(expert_budget, router_weight.shape[0], routing_objective)
    _require_device(x, w1, w2, w3, router_weight, node_accept_prob)
    dt = _require_half("x", x)
    for name, t in (("w1", w1), ("w2", w2), ("w3", w3), ("router_weight", router_weight)):
        _require_half(name, t, like=x)
    n, hidden = x.shape
    e, inter, h_w = w1.shape
    if h_w != hidden or w3.shape != w1.shape or tuple(w2.shape) != (e, hidden, inter):
        raise ValueError("expected w1, w3 [E, I, H] and w2 [E, H, I] matching x [T, H]")
    if hidden % 256 != 0 or inter % 256 != 0:
        raise ValueError("hidden and intermediate sizes must be multiples of 256")
    tiled = uses_tiled_gemms(n, expert_budget, e, inter)
    if routing is None and self_routed(n, expert_budget, e, inter):
        # router, then the gate/up launch that also routes and buckets
        _check_router(x, router_weight)
        stream = _capi.stream_of(x.device)
        ws = _workspace(n, e, hidden, inter, x)
        accept = _prep_accept(node_accept_prob, n)
        routing = _routing_of(ws, n, expert_budget)
        _launch_router(x, router_weight, ws.router_gates)
        if on_phase is not None:
            on_phase("route")
        call("tm_op1_prefill_gemm1_routed", ptr(x), ptr(w1), ptr(w3), ptr(ws.h),
             ptr(ws.router_gates), ptr(accept), n, hidden, inter, e, expert_budget, 0.05,
             TM_OBJECTIVE[routing_objective], BM, routing.max_blocks, routing.max_tiles,
             ptr(ws.topk_flat), ptr(ws.gates_flat), ptr(routing.padded_slots),
             ptr(routing.block_expert_ids), ptr(ws.slot_to_row), ptr(ws.demand),
             ptr(ws.expert_offsets), ptr(ws.sorted_slots), ptr(ws.slot_pos),
             ptr(routing.tiles), dt, stream)
        gemm1_done = True
    else:
        if routing is None:
            routing = route_experts(x, router_weight, node_accept_prob, expert_budget, inter,
                                    routing_objective=routing_objective)
        if on_phase is not None:
            on_phase("route")
        gemm1_done = False
    ws = routing.ws
    if (routing.topk_ids.shape[0] != n or ws.partial.shape[1] != 2 * n
            or ws.h.shape != (ws.max_tiles * TILE_M, inter) or ws.partial.shape[2] != hidden
            or ws.num_experts != e or routing.max_tiles > ws.max_tiles
            or ws.h.dtype != x.dtype):
        raise ValueError("routing was computed for a different shape")
    stream = _capi.stream_of(x.device)
    split = ws.split
    if tiled:
        split = _tiled_split(n, expert_budget, e, hidden, inter, ws)
        if not gemm1_done:
            call("tm_op1_prefill_gemm1", ptr(x), ptr(w1), ptr(w3), ptr(ws.h),
                 ptr(routing.sorted_slots), ptr(routing.expert_offsets), ptr(routing.tiles),
                 routing.max_tiles, n, hidden, inter, e, dt, stream)
        if on_phase is not None:
            on_phase("gemm1")
        call("tm_op1_prefill_gemm2", ptr(ws.h), ptr(w2), ptr(ws.partial),
             ptr(routing.gates_flat), ptr(routing.sorted_slots), ptr(routing.expert_offsets),
             ptr(routing.tiles), routing.max_tiles, split, n, hidden, inter, e, dt, stream)
    else:
        call("tm_op1_gemm1", ptr(x), ptr(w1), ptr(w3), ptr(ws.h), ptr(routing.sorted_slots),
             ptr(routing.tiles), routing.max_tiles, n, hidden, inter, e, dt, stream)
        if on_phase is not None:
            on_phase("gemm1")
        call("tm_op1_gemm2", ptr(ws.h), ptr(w2), ptr(ws.partial), ptr(routing.gates_flat),
             ptr(routing.sorted_slots), ptr(routing.tiles), routing.max_tiles, ws.split, n,
             hidden, inter, e, dt, stream)
    if on_phase is not None:
        on_phase("gemm2")
    if out is not None:
        if out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
            raise ValueError("out must be a contiguous tensor like x")
        result = out
    else:
        result = torch.empty_like(x)
    call("tm_op1_combine", ptr(ws.partial), ptr(routing.slot_pos), ptr(result), n, hidden,
         split, dt, stream)
    if on_phase is not None:
        on_phase("combine")
    return result
