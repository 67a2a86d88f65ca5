"""CPU: host-side logic of the package (validation, layouts, workspaces,
KV-cache bookkeeping, synthetic workloads).  No GPU work is launched."""

from __future__ import annotations

import pytest
import torch

from tests.conftest import make_moe_inputs


def test_budget_and_objective_validation_messages():
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    g = torch.Generator().manual_seed(0)
    x, w1, w2, w3, router, accept = make_moe_inputs(8, 4, 256, 256, g, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match=r"expert_budget must be in \[2, 4\]"):
        m.tree_moe_forward(x, w1, w2, w3, router, accept, 5)
    with pytest.raises(ValueError, match="routing_objective"):
        m.route_experts(x, router, accept, 2, 256, routing_objective="x")


def test_cpu_tensors_fail_loudly():
    from treemoe_spec_amd.kernels import op1_tree_moe as m
    from treemoe_spec_amd.kernels import op4_commit as o

    g = torch.Generator().manual_seed(0)
    x, w1, w2, w3, router, accept = make_moe_inputs(8, 4, 256, 256, g, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm"):
        m.tree_moe_forward(x, w1, w2, w3, router, accept, 2)
    with pytest.raises(RuntimeError, match="ROCm"):
        m.route_and_bucket(x, router, accept, 2)
    with pytest.raises(RuntimeError, match="ROCm"):
        o.fused_verify_commit(torch.zeros(2, 8), None, torch.zeros(2), None, [[1], []])
    with pytest.raises(RuntimeError, match="ROCm"):
        o.fused_verify_commit(torch.zeros(2, 8), torch.zeros(2, 8), torch.zeros(2), None,
                              [[1], []], temperature=0.7)
    with pytest.raises(ValueError, match="temperature"):
        o.fused_verify_commit(torch.zeros(2, 8), None, torch.zeros(2), None, [[1], []],
                              temperature=-1.0)
    with pytest.raises(ValueError, match="rep_penalty"):
        o.fused_verify_commit(torch.zeros(2, 8), None, torch.zeros(2), None, [[1], []],
                              rep_penalty=0.0)


def test_tree_depth_bounds_the_sampling_commit():
    from treemoe_spec_amd.kernels.op4_commit import _tree_depth

    assert _tree_depth([[]]) == 0
    assert _tree_depth([[1, 2], [3], [], [4], []]) == 3
    assert _tree_depth([[1], [2], [3], []]) == 3
    # a malformed list with a back edge still stops at N - 1
    assert _tree_depth([[1], [0, 2], [1]]) == 2
    # nodes unreachable from the root do not count
    assert _tree_depth([[], [2], []]) == 0


def test_block_m_env_is_validated(monkeypatch):
    import importlib

    import treemoe_spec_amd.kernels.op1_tree_moe as m

    monkeypatch.setenv("TREEMOE_BLOCK_M", "24")
    with pytest.raises(ValueError, match="TREEMOE_BLOCK_M"):
        importlib.reload(m)
    monkeypatch.setenv("TREEMOE_BLOCK_M", "16")
    importlib.reload(m)


def test_workspace_kat():
    """Reference KAT tests/test_op1.py:377-391: T=64 -> 16 blocks, 15 launched,
    256 padded rows (BM16)."""
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    assert m.compact_block_capacity(128, 8, 16) == 16
    assert m.compact_block_limit(128, 8, 16) == 15
    assert m.compact_block_capacity(128, 8, 16) * 16 == 256
    assert m.compact_block_limit(128, 8, m.TILE_M) == 9


@pytest.mark.parametrize("inter,split", [(14336, 2), (3584, 2), (512, 2), (1024, 2), (256, 1)])
def test_split_selection(inter, split):
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    assert m._split_for(inter) == split
    with pytest.raises(ValueError):
        m._split_for(200)


def test_tiled_down_gemm_split_rule():
    """The tiled down GEMM takes 4 K segments when split 2 would launch less
    than one round of 256 CUs (config 3), else the workspace's split (config
    5); the partials of 4 segments are allocated only when small."""
    from types import SimpleNamespace

    from treemoe_spec_amd.kernels import op1_tree_moe as m

    ws = m._Workspace(64, 8, 4096, 14336, "cpu", torch.bfloat16)  # config 2/3 shape
    assert ws.split == 2 and ws.partial.shape == (4, 128, 4096)
    # config 3: <= 1 + 4 real M-tiles x 16 column blocks x 2 = 160 jobs < 256
    assert m._tiled_split(64, 4, 8, 4096, 14336, ws) == 4
    # config 5: 32 + 8 M-tiles x 16 x 2 jobs fill the CUs; its partials stay at 2
    big = SimpleNamespace(split=2, partial=torch.empty(2, 1, 1))
    assert m._tiled_split(2048, 8, 8, 4096, 14336, big) == 2
    wide = SimpleNamespace(split=2, partial=torch.empty(4, 1, 1))
    assert m._tiled_split(2048, 8, 8, 4096, 14336, wide) == 2
    # a workspace without room for 4 segments keeps its split
    assert m._tiled_split(64, 4, 8, 4096, 14336, big) == 2
    # 4 segments must keep (I / 4) % 64 == 0
    assert m._tiled_split(64, 4, 8, 4096, 14336 + 128, wide) == 2
    # large T: 4-segment partials would exceed the cap, so only 2 are allocated
    assert m.TILED_SPLIT_WIDE * 2 * 4096 * 4096 * 4 > m._TILED_WIDE_MAX_BYTES


def test_children_csr_packing():
    from treemoe_spec_amd.kernels.op4_commit import _children_csr

    children = [[1, 2], [3], [], []]
    csr, edges = _children_csr(children, 4, "cpu")
    csr = csr.tolist()
    assert csr[:4] == [0, 2, 3, 3] and csr[4:8] == [2, 1, 0, 0] and csr[8:] == [1, 2, 3]
    assert edges == 3
    # a tree padded with edge-free slots (the engine's num_valid < N) has fewer
    # than N - 1 edges, and the count says so
    csr, edges = _children_csr([[1], [], [], []], 4, "cpu")
    assert edges == 1 and csr.tolist()[8:] == [1]
    csr, edges = _children_csr([[], [], [], []], 4, "cpu")
    assert edges == 0 and csr.tolist()[8:] == [0]
    with pytest.raises(ValueError):
        _children_csr([[5], [], [], []], 4, "cpu")
    with pytest.raises(ValueError):
        _children_csr([[1]], 4, "cpu")


def test_cached_csr_checks_the_node_count_on_a_hit():
    """The same children list passed again with another N is rejected, not
    served from the cache at offsets sized for the first N."""
    from treemoe_spec_amd.kernels import op4_commit as o

    children = [[1, 2], [3], [], []]
    csr, edges = o._cached_csr(children, 4, "cpu")
    again, _ = o._cached_csr(children, 4, "cpu")
    assert again is csr and edges == 3
    with pytest.raises(ValueError, match="list 8 nodes, got 4"):
        o._cached_csr(children, 8, "cpu")
    with pytest.raises(ValueError, match="list 3 nodes, got 4"):
        o._cached_csr(children, 3, "cpu")


def test_op4_scratch_key_separates_streams_and_threads():
    """The greedy path's internal buffers are keyed by stream and host thread:
    a kv=None call returns with its kernels still queued, so a call on a
    second stream must not share its partials, and each thread reads its own
    count word."""
    import threading

    from treemoe_spec_amd.kernels import op4_commit as o

    k1 = o._scratch_key(64, 0, 0x1000)
    assert k1 == o._scratch_key(64, 0, 0x1000)
    assert k1 != o._scratch_key(64, 0, 0x2000)      # another stream
    assert k1 != o._scratch_key(64, 1, 0x1000)      # another device
    assert k1 != o._scratch_key(32, 0, 0x1000)      # another tree size
    other = []
    th = threading.Thread(target=lambda: other.append(o._scratch_key(64, 0, 0x1000)))
    th.start()
    th.join()
    assert other[0] != k1                           # another host thread


def test_kv_cache_bookkeeping_page16():
    from treemoe_spec_amd.kv_cache import MixtralConfig, PagedKVCache

    cfg = MixtralConfig(num_layers=2, num_kv_heads=2, head_dim=8)
    kv = PagedKVCache(cfg, 12, device="cpu", dtype=torch.float32, page_size=16, tree_size=64)
    assert kv.tree_pages == [0, 1, 2, 3] and kv.tree_block == 0
    kv._ensure_capacity(40)
    assert len(kv.block_table) == 3 and all(p >= 4 for p in kv.block_table)
    assert kv.slot_of(17) == (kv.block_table[1], 1)
    with pytest.raises(RuntimeError, match="out of blocks"):
        kv._ensure_capacity(16 * 9)
    kv.reset()
    assert kv.seq_len == 0 and kv.block_table == []
    k = torch.randn(50, 2, 8)
    kv.write_tree(1, k, k + 1)
    assert torch.equal(kv.k[1, 1, :16], k[16:32]) and torch.equal(kv.v[1, 3, :2], k[48:50] + 1)


def test_kv_cache_reference_layout():
    from treemoe_spec_amd.kv_cache import BLOCK_SIZE, MixtralConfig, PagedKVCache

    kv = PagedKVCache(MixtralConfig(num_layers=1, num_kv_heads=1, head_dim=4), 4,
                      device="cpu", dtype=torch.float32)
    assert kv.block_size == BLOCK_SIZE == 64 and kv.tree_pages == [0]
    kv._ensure_capacity(65)
    assert kv.block_table == [1, 2]


def test_workloads_are_seeded():
    from treemoe_spec_amd.workloads import draw_activations, op4_workload

    a = draw_activations(8, 64, 8, 2, "normal1.5")
    b = draw_activations(8, 64, 8, 2, "normal1.5")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert torch.all(a[0][:, 0] == 1.0)
    w1 = op4_workload(n=32, vocab=500, max_depth=4, seed=9)
    w2 = op4_workload(n=32, vocab=500, max_depth=4, seed=9)
    assert torch.equal(w1.logits, w2.logits) and w1.children == w2.children
    assert max(w1.depth) <= 4
    for node, kids in enumerate(w1.children):
        toks = [int(w1.tokens[c]) for c in kids]
        assert len(toks) == len(set(toks)) and all(c > node for c in kids)


def test_moe_adapter_host_logic(monkeypatch):
    """The engine hook's host logic (benchmarks/bench_e2e.py:482-504, 654-658):
    accept from current_accept_prob when it matches the row count, else ones;
    the layer's budget from current_layer_budgets, else the default; the
    demand handed to the observer; the routing reused by the GEMMs."""
    from types import SimpleNamespace

    import treemoe_spec_amd.moe_adapter as ad

    calls = []
    routing = SimpleNamespace(demand=torch.tensor([3.0, 1.0]))

    def fake_route(x, router, accept, budget, inter, top1_threshold, routing_objective):
        calls.append(("route", accept.clone(), budget, inter, top1_threshold,
                      routing_objective))
        return routing

    def fake_forward(x, w1, w2, w3, router, accept, budget, routing=None, deterministic=True):
        calls.append(("forward", budget, routing, deterministic))
        return x + 1

    monkeypatch.setattr(ad, "route_experts", fake_route)
    monkeypatch.setattr(ad, "tree_moe_forward", fake_forward)
    fn = ad.make_moe_fn(expert_budget=6, top1_threshold=0.1, routing_objective="critical_path",
                        deterministic=False, tree_size=4, device="cpu")
    lw = SimpleNamespace(router=None, w1=torch.zeros(2, 24, 8), w2=None, w3=None)
    x = torch.zeros(4, 8)
    assert torch.equal(fn.current_accept_prob, torch.ones(4))
    fn.current_accept_prob = torch.tensor([0.9, 0.5, 0.2, 0.01])
    seen = []
    fn.demand_observer = lambda li, d: seen.append((li, d))
    out = fn(x, lw, 1)
    assert torch.equal(out, x + 1)
    kind, accept, budget, inter, tau, objective = calls[0]
    assert torch.equal(accept, torch.tensor([0.9, 0.5, 0.2, 0.01]))
    assert (budget, inter, tau, objective) == (6, 24, 0.1, "critical_path")
    assert calls[1] == ("forward", 6, routing, False)
    assert seen == [(1, routing.demand)]
    # per-layer budgets and a row count that differs from the tree
    fn.current_layer_budgets = torch.tensor([8, 3])
    calls.clear()
    fn(torch.zeros(3, 8), lw, 1)
    assert torch.equal(calls[0][1], torch.ones(3)) and calls[0][2] == 3


def test_kv_cache_append_gather_commit_tree():
    """The product cache carries the reference cache's model-facing methods
    (append, gather, gather_with_tail, commit_tree; treemoe/model/kv_cache.py:62-145)
    with the multi-page tree scratch."""
    from treemoe_spec_amd.kv_cache import MixtralConfig, PagedKVCache

    cfg = MixtralConfig(num_layers=2, num_kv_heads=2, head_dim=4)
    kv = PagedKVCache(cfg, 16, device="cpu", dtype=torch.float32, page_size=16, tree_size=40)
    kv._free = kv._free[::-1]          # a non-identity page order
    g = torch.Generator().manual_seed(0)
    rows = torch.randn(37, 2, 4, generator=g)
    kv.append(1, rows[:20], rows[:20] + 1, 0)
    kv.append(1, rows[20:], rows[20:] + 1, 20)
    assert kv.seq_len == 37
    k, v = kv.gather(1)
    assert torch.equal(k, rows) and torch.equal(v, rows + 1)
    tail = torch.randn(5, 2, 4, generator=g)
    fk, fv = kv.gather_with_tail(1, tail, tail - 1)
    assert torch.equal(fk, torch.cat([rows, tail])) and torch.equal(fv, torch.cat([rows + 1, tail - 1]))
    tree = torch.randn(40, 2, 4, generator=g)
    for layer in range(2):
        kv.write_tree(layer, tree + layer, tree - layer)
    kv.commit_tree(torch.tensor([0, 5, 17, 39, -1, -1]))
    assert kv.seq_len == 41
    for layer in (0, 1):
        k, v = kv.gather(layer)
        assert torch.equal(k[37:], tree[[0, 5, 17, 39]] + layer)
        assert torch.equal(v[37:], tree[[0, 5, 17, 39]] - layer)
    assert torch.equal(kv.gather(1)[0][:37], rows)
    # an empty prefix
    kv.reset()
    fk, _ = kv.gather_with_tail(0, tail, tail)
    assert torch.equal(fk, tail)


def test_op4_commit_host_logic_with_reference_cache(monkeypatch):
    """op4's commit glue on an object with exactly the reference cache's
    attributes (tree_block, page 64, no tree_pages / device_tables): the
    launch gets scratch page [tree_block], the block table after the
    reference's capacity growth (op4_commit.py:251) and seq_len; replaying the
    launch with the oracle commits [root] + path to seq_len, seq_len + 1, ..."""
    from oracle import op4_ref
    from tests.ref_layout_cache import RefLayoutKVCache
    from treemoe_spec_amd.kernels import op4_commit

    kv = RefLayoutKVCache(2, 2, 8, 6, device="cpu", dtype=torch.float32)
    kv.k.normal_(generator=torch.Generator().manual_seed(1))
    kv.v.normal_(generator=torch.Generator().manual_seed(2))
    kv._ensure_capacity(100)
    kv.seq_len = 100
    k0, v0 = kv.k.clone(), kv.v.clone()
    seen = {}

    def fake_call(name, *args):
        seen["name"], seen["args"] = name, args

    monkeypatch.setattr(op4_commit, "call", fake_call)
    monkeypatch.setattr(op4_commit, "_fast", None)
    slots = torch.tensor([3, 9, 30] + [-1] * 61)
    result = torch.tensor([7, 3, 30])
    op4_commit._commit(kv, slots.data_ptr(), result.data_ptr(), 64, 6, torch.device("cpu"), 0)
    assert seen["name"] == "tm_op4_kv_commit"
    a = seen["args"]
    assert a[9] == slots.data_ptr() and a[10] == result.data_ptr()
    assert a[8] == 64 and a[12] == 1 and a[14] == len(kv.block_table) and a[15] == 100
    assert a[16] == 6 and len(kv.block_table) * 64 >= 100 + 7
    table, scratch = op4_commit.device_tables_of(kv, "cpu")
    assert scratch.tolist() == [kv.tree_block] and table.tolist() == kv.block_table
    # replay what the kernel does with the oracle
    commit = torch.cat([torch.zeros(1, dtype=torch.long), slots])
    assert op4_ref.commit_tree(k0, v0, commit, scratch.tolist(), table.tolist(), 100) == 4
    for j, s in enumerate([0, 3, 9, 30]):
        blk, off = kv.slot_of(100 + j)
        assert torch.equal(k0[:, blk, off], kv.k[:, 0, s])
    # the table cache follows the host table
    kv._ensure_capacity(300)
    table2, _ = op4_commit.device_tables_of(kv, "cpu")
    assert table2.tolist() == kv.block_table
    with pytest.raises(ValueError, match="scratch"):
        op4_commit._commit(kv, slots.data_ptr(), result.data_ptr(), 65, 6, torch.device("cpu"), 0)


def test_routing_token_count_mismatch_raises_before_launch(monkeypatch):
    """A Routing computed for T tokens cannot be used with x of another T
    (same tile count: T=64 and T=65 both bound 9 tiles)."""
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    def no_launch(*a, **k):
        raise AssertionError("launched")

    monkeypatch.setattr(m, "call", no_launch)
    monkeypatch.setattr(m, "_require_device", lambda *t: None)
    e, h, i = 8, 256, 256
    ws = m._Workspace(64, e, h, i, "cpu", torch.bfloat16)
    ws65 = m._Workspace(65, e, h, i, "cpu", torch.bfloat16)
    assert ws.max_tiles == ws65.max_tiles
    r = m.Routing(ws, ws.router_gates, ws.topk_flat.view(64, 2), ws.gates_flat,
                  ws.padded_slots, ws.block_expert_ids, ws.slot_to_row, ws.max_blocks,
                  ws.max_blocks, ws.demand, ws.expert_offsets, ws.sorted_slots, ws.slot_pos,
                  ws.tiles, ws.max_tiles)
    bf = torch.bfloat16
    x = torch.zeros(65, h, dtype=bf)
    w1 = torch.zeros(e, i, h, dtype=bf)
    w2 = torch.zeros(e, h, i, dtype=bf)
    with pytest.raises(ValueError, match="different shape"):
        m.tree_moe_forward(x, w1, w2, w1, torch.zeros(e, h, dtype=bf), torch.ones(65), 8,
                           routing=r)


def test_gemm_path_rule():
    """The MFMA-tiled GEMMs run from 32 rows per routed expert, and from 8
    rows when the FFN is 3584 wide or more (the Mixtral decode shape T=64,
    B=8, I=14336 and its TP-2 and TP-4 shares take them); narrower FFN
    shares keep the weight-streaming GEMMs until 32 rows."""
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    assert m.uses_tiled_gemms(64, 8, 8, 14336)        # config 2: 16 rows, wide
    assert m.uses_tiled_gemms(32, 8, 8, 14336)        # 8 rows, wide
    assert not m.uses_tiled_gemms(16, 8, 8, 14336)    # 4 rows
    assert m.uses_tiled_gemms(64, 8, 8, 7168)         # the TP-2 share
    assert m.uses_tiled_gemms(64, 8, 8, 3584)         # the TP-4 share
    assert not m.uses_tiled_gemms(64, 8, 8, 1792)     # TP-8 streams
    assert not m.uses_tiled_gemms(64, 8, 8)           # no width given: 32-row rule
    assert m.uses_tiled_gemms(64, 4, 8, 3584)         # config 3: 32 rows
    assert m.uses_tiled_gemms(128, 8, 8, 1792)



def test_tiled_gate_up_tile_rule():
    """The gate/up tile the library picks (named in bench lines): 256-row tiles
    from 384 rows per expert, the 64-row decode tile when the tile list
    leaves at most 16 rows per entry, else 128-row tiles."""
    from treemoe_spec_amd.kernels import op1_tree_moe as m

    def tiles(t, budget, e=8):
        return m.compact_block_limit(2 * t, budget, m.TILE_M)

    assert m.tiled_gate_up_tile(64, 8, tiles(64, 8)) == "Tile<64, 64, 3, 128, 256>"   # config 2
    assert m.tiled_gate_up_tile(64, 8, tiles(64, 4)) == "Tile<128, 64, 3>"            # config 3
    assert m.tiled_gate_up_tile(2048, 8, tiles(2048, 8)) == "Tile<256, 32, 4>"        # config 5
    assert m.tiled_gate_up_tile(32, 8, tiles(32, 8)) == "Tile<64, 64, 3, 128, 256>"
    assert m.tiled_gate_up_tile(128, 8, tiles(128, 8)) == "Tile<128, 64, 3>"


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with a message before
    touching a device."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    proc = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120, cwd=root)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr


def test_bench_median():
    import bench

    assert bench.median([3.0, 1.0, 2.0]) == 2.0
    assert bench.median([4.0, 1.0, 3.0, 2.0]) == 2.5
