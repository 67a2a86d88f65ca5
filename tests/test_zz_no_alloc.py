"""tm_op4_argmax_walk_noalloc (the allocation-free variant, scratch in a
static device array) against tm_op4_argmax_walk (caller's workspace): same
argmax, accepted path, tokens and result, on two calls in a row, the second
with a smaller input, and for both argmax modes."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(seed, n, v, dtype):
    from treemoe_spec_amd.workloads import random_tree

    g = torch.Generator().manual_seed(seed)
    parent, children, tokens, _ = random_tree(g, n, 8, v)
    logits = torch.randn(n, v, generator=g) * 3
    for node in range(n):
        if children[node] and node % 3 != 2:
            logits[node, tokens[children[node][0]]] += 50.0
    return logits.to(dtype).cuda(), tokens.cuda(), children


def _run(name, logits, tokens, children, softmax_argmax, workspace):
    from treemoe_spec_amd import _capi
    from treemoe_spec_amd.kernels.op4_commit import _children_csr

    n, v = logits.shape
    dt = _capi.TM_DTYPE_F32 if logits.dtype == torch.float32 else _capi.TM_DTYPE_BF16
    csr, edges = _children_csr(children, n, "cuda")
    argmax = torch.full((n,), -7, dtype=torch.int32, device="cuda")
    out = torch.full((2 * n + 3,), -7, dtype=torch.int64, device="cuda")
    p = _capi.ptr
    args = [p(logits), dt, n, v, logits.stride(0), p(tokens), p(csr), p(csr) + 4 * n,
            p(csr) + 8 * n, edges, 8, softmax_argmax, p(argmax), p(out), p(out) + 8 * n,
            p(out) + 16 * n]
    if workspace:
        args.append(p(torch.empty(n * _capi.TM_OP4_MAX_PARTS * 8, dtype=torch.uint8,
                                  device="cuda")))
    _capi.call(name, *args, _capi.stream_of(logits.device))
    torch.cuda.synchronize()
    return argmax.cpu(), out.cpu()


@pytest.mark.parametrize("softmax_argmax", [0, 1])
def test_noalloc_matches_workspace_entry_point(softmax_argmax):
    print(f"noalloc argmax walk softmax_argmax={softmax_argmax}", flush=True)
    for seed, n, v, dtype in ((1, 64, 32000, torch.bfloat16), (2, 16, 5000, torch.float32)):
        logits, tokens, children = _case(seed, n, v, dtype)
        want = _run("tm_op4_argmax_walk", logits, tokens, children, softmax_argmax, True)
        got = _run("tm_op4_argmax_walk_noalloc", logits, tokens, children, softmax_argmax,
                   False)
        assert torch.equal(got[0], want[0]), (n, v)
        assert torch.equal(got[1], want[1]), (n, v)
        assert int(got[1][2 * n + 1]) >= 0


def test_noalloc_rejects_more_nodes_than_its_scratch():
    from treemoe_spec_amd import _capi

    n = _capi.TM_OP4_NOALLOC_MAX_NODES + 1
    rc = _capi.lib().tm_op4_argmax_walk_noalloc(0, 0, n, 10, 10, 0, 0, 0, 0, n - 1, 8, 0, 0, 0,
                                                0, 0, 0)
    assert rc == 1001
