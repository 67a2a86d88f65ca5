"""op1 layers and tree attention captured in a HIP graph (torch.cuda.CUDAGraph).

Serving loops capture whole verification steps to hide launch overhead, so
every launch of these paths must be capturable: no host synchronisation, no
allocation outside torch's graph pool, no memset node.  Bar: every replay of
the captured call equals the eager call's output bit for bit, with the
program's own eager work and synchronisations between the replays (a graph
whose nodes depended on state left by the capture-time call, or on memsets,
would drift from the second replay on).
"""

from __future__ import annotations

import pytest
import torch

from oracle import attn_ref
from tests.conftest import make_moe_inputs

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)


def _op1():
    from treemoe_spec_amd.kernels import op1_tree_moe

    return op1_tree_moe


def _capture(fn):
    """Warm fn up on a side stream (workspace allocation happens outside the
    capture), then capture one call; returns the graph and its output."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _replays_match(g, out, want, eager_between):
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r} differs from the eager call"
        eager_between()
        torch.cuda.synchronize()


@pytest.mark.parametrize("path,t,budget", [
    ("tiled", 64, 8),          # routing inside the gate/up launch
    ("tiled", 64, 4),
    ("tiled_bucket", 64, 4),   # router + bucketing launches, then the tiled pair
    ("stream", 64, 8),         # the weight-streaming pair
    ("tiled", 512, 8),         # many rows per expert: the 256-row ping-pong tiles
])
def test_op1_graph_replays_equal_eager(path, t, budget, monkeypatch):
    _say(f"graph capture op1 path={path} t={t} B={budget}")
    m = _op1()
    monkeypatch.setattr(m, "TILED_MIN_ROWS", 1 << 30 if path == "stream" else 1)
    monkeypatch.setattr(m, "TILED_MIN_ROWS_WIDE", 1 << 30 if path == "stream" else 1)
    if path == "tiled_bucket":
        monkeypatch.setattr(m, "SELF_ROUTED_MAX_TOKENS", 0)
    e, h, i = (8, 512, 1024) if t <= 64 else (2, 512, 1024)
    g = torch.Generator().manual_seed(900 + t + budget)
    x, w1, w2, w3, router, accept = make_moe_inputs(t, e, h, i, g, dtype=torch.bfloat16)
    dev = [a.cuda() for a in (x, w1, w2, w3, router, accept)]
    budget = min(budget, e)
    fwd = lambda: m.tree_moe_forward(*dev, budget)
    want = fwd().clone()
    torch.cuda.synchronize()
    graph, out = _capture(fwd)
    # eager work of the same shape on other inputs between the replays
    other = [a.clone() for a in dev]
    other[0].mul_(-1.0)
    _replays_match(graph, out, want,
                   lambda: m.tree_moe_forward(*other, budget))


def test_tree_attention_graph_replays_equal_eager():
    _say("graph capture tree attention")
    from treemoe_spec_amd.kernels.tree_attention import tree_attention
    from treemoe_spec_amd.kv_cache import MixtralConfig, PagedKVCache

    n, hq, kvh, seq_len, page = 64, 32, 8, 1000, 16
    g = torch.Generator().manual_seed(31)
    cfg = MixtralConfig(num_layers=1, num_kv_heads=kvh, head_dim=128, num_heads=hq)
    kv = PagedKVCache(cfg, (n + page - 1) // page + (seq_len + page - 1) // page + 4,
                      device="cuda", dtype=torch.bfloat16, page_size=page, tree_size=n)
    kv.k.copy_(torch.randn(kv.k.shape, generator=g).to(torch.bfloat16))
    kv.v.copy_(torch.randn(kv.v.shape, generator=g).to(torch.bfloat16))
    kv._ensure_capacity(seq_len)
    kv.seq_len = seq_len
    q = torch.randn(n, hq, 128, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(n, kvh, 128, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(n, kvh, 128, generator=g).to(torch.bfloat16).cuda()
    parent = [-1] + [int(torch.randint(0, j, (1,), generator=g)) for j in range(1, n)]
    mask = attn_ref.ancestor_mask(parent).cuda()
    att = lambda: tree_attention(q, k, v, kv, 0, mask)
    want = att().clone()
    torch.cuda.synchronize()
    graph, out = _capture(att)
    q2 = q.flip(0).contiguous()
    _replays_match(graph, out, want, lambda: tree_attention(q2, k, v, kv, 0, mask))
