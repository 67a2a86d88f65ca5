"""Seeded synthetic workloads for the op1/op4 benchmark configurations.

Recipes (fixed so that every run, test and CPU baseline sees the same bits):

* op1: a CPU ``torch.Generator`` seeded with ``seed`` draws, in this order,
  x [T, H] ~ N(0, 1), W_g [E, H] ~ N(0, 0.02) and, when the config has one, a
  per-expert router bias b [E]; all FP32, then cast to bf16.  The bias is folded
  into the unchanged API as a constant feature: x[:, 0] = 1 and W_g[:, 0] = b.
  Expert weights w1, w3 [E, I, H] and w2 [E, H, I] ~ N(0, 0.02) are drawn, in
  that order, by a generator on ``weight_device`` seeded with ``seed + 1000``
  (device generation keeps the 2.8 GB Mixtral draw to a fraction of a second).
  accept = ones(T) unless stated.
* op4: ``op4_workload``: random tree (parent ~ U{0..i-1}, depth <= max_depth),
  children in ascending index order, distinct sibling tokens, logits
  ~ N(0, 3) with a planted accepted path and exact-tie rows, KV ~ N(0, 1).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

OP1_CONFIGS = {
    # name: (T, H, I, E, budget, seed, bias)
    "config1_cpu_small": (64, 1024, 3584, 8, 8, 0, None),
    "config2_mixtral_t64_b8": (64, 4096, 14336, 8, 8, 1, None),
    "config3_mixtral_t64_b4_skew": (64, 4096, 14336, 8, 4, 2, "normal1.5"),
    "config5_mixtral_t2048_zipf": (2048, 4096, 14336, 8, 8, 4, "zipf1.2"),
}


@dataclass
class Op1Inputs:
    name: str
    x: torch.Tensor
    w1: torch.Tensor
    w2: torch.Tensor
    w3: torch.Tensor
    router: torch.Tensor
    accept: torch.Tensor
    budget: int
    seed: int
    meta: dict = field(default_factory=dict)

    @property
    def shape(self) -> tuple[int, int, int, int]:
        t, h = self.x.shape
        e, i, _ = self.w1.shape
        return t, h, i, e


def draw_activations(t: int, h: int, e: int, seed: int, bias: str | None = None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, h, generator=g)
    router = torch.randn(e, h, generator=g) * 0.02
    b = None
    if bias == "normal1.5":
        b = torch.randn(e, generator=g) * 1.5
    elif bias == "zipf1.2":
        r = (torch.randperm(e, generator=g) + 1).float()
        b = -1.2 * torch.log(r)
    if b is not None:
        x[:, 0] = 1.0
        router[:, 0] = b
    return x.to(torch.bfloat16), router.to(torch.bfloat16), b


def draw_weights(e: int, h: int, i: int, seed: int, device="cpu"):
    g = torch.Generator(device=device).manual_seed(seed + 1000)
    out = []
    for shape in ((e, i, h), (e, i, h), (e, h, i)):
        w = torch.empty(shape, dtype=torch.bfloat16, device=device)
        w.normal_(0.0, 0.02, generator=g)
        out.append(w)
    w1, w3, w2 = out
    return w1, w2, w3


def op1_workload(name: str, device="cuda", weight_device=None,
                 weights: tuple | None = None) -> Op1Inputs:
    t, h, i, e, budget, seed, bias = OP1_CONFIGS[name]
    return op1_inputs(t, h, i, e, budget, seed, bias, device=device,
                      weight_device=weight_device, weights=weights, name=name)


def op1_inputs(t, h, i, e, budget, seed, bias=None, device="cuda", weight_device=None,
               weights=None, name="custom") -> Op1Inputs:
    x, router, b = draw_activations(t, h, e, seed, bias)
    if weights is None:
        wdev = weight_device or device
        w1, w2, w3 = draw_weights(e, h, i, seed, device=wdev)
    else:
        w1, w2, w3 = weights
    accept = torch.ones(t, dtype=torch.float32)
    return Op1Inputs(name=name, x=x.to(device), w1=w1.to(device), w2=w2.to(device),
                     w3=w3.to(device), router=router.to(device), accept=accept.to(device),
                     budget=budget, seed=seed, meta={"bias": None if b is None else b.tolist()})


def op1_algorithmic_bytes(t: int, h: int, i: int, e: int, n_active: int) -> int:
    """Compulsory HBM bytes of one op1 layer: active experts' w1, w3, w2, plus
    x, out, W_g and accept (workspace round trips excluded)."""
    return n_active * 3 * h * i * 2 + t * h * 2 * 2 + e * h * 2 + 4 * t


def op1_flops(t: int, h: int, i: int, e: int) -> int:
    """Router GEMV + 2 slots per token x (gate, up, down) GEMMs."""
    return 2 * t * h * e + 2 * t * 3 * 2 * h * i


def random_tree(g: torch.Generator, n: int, max_depth: int | None = None,
                vocab: int = 32000):
    """parent[i] ~ U{0..i-1} (resampled while depth > max_depth); children in
    ascending index order; sibling tokens distinct."""
    parent = [-1]
    depth = [0]
    for i in range(1, n):
        while True:
            p = int(torch.randint(0, i, (1,), generator=g))
            if max_depth is None or depth[p] + 1 <= max_depth:
                break
        parent.append(p)
        depth.append(depth[p] + 1)
    children = [[] for _ in range(n)]
    for i in range(1, n):
        children[parent[i]].append(i)
    tokens = torch.randint(0, vocab, (n,), generator=g)
    for kids in children:
        seen = set()
        for c in kids:
            while int(tokens[c]) in seen:
                tokens[c] = (tokens[c] + 1) % vocab
            seen.add(int(tokens[c]))
    return parent, children, tokens, depth


@dataclass
class Op4Inputs:
    logits: torch.Tensor          # [N, V]
    tokens: torch.Tensor          # [N] int64
    parent: torch.Tensor          # [N] int64
    children: list
    planted_path: list
    max_depth: int
    depth: list


def op4_workload(n: int = 64, vocab: int = 32000, max_depth: int = 8, seed: int = 3,
                 dtype=torch.bfloat16, tie_rows: int = 4) -> Op4Inputs:
    """Tree + logits on the CPU.  Acceptance is planted along a random root
    path of random length 0..max_depth (the accepted child's token gets
    max + 1), and ``tie_rows`` nodes get an exact tie of their maximum at an
    earlier index (first occurrence must win)."""
    g = torch.Generator().manual_seed(seed)
    parent, children, tokens, depth = random_tree(g, n, max_depth, vocab)
    logits = (torch.randn(n, vocab, generator=g) * 3.0).to(dtype).float()
    length = int(torch.randint(0, max_depth + 1, (1,), generator=g))
    path = []
    node = 0
    for _ in range(length):
        if not children[node]:
            break
        c = children[node][int(torch.randint(0, len(children[node]), (1,), generator=g))]
        logits[node, int(tokens[c])] = logits[node].max() + 1.0
        path.append(c)
        node = c
    for _ in range(tie_rows):
        r = int(torch.randint(0, n, (1,), generator=g))
        j = int(logits[r].argmax())
        if j > 0:
            k = int(torch.randint(0, j, (1,), generator=g))
            logits[r, k] = logits[r, j]
    return Op4Inputs(logits=logits.to(dtype), tokens=tokens.long(),
                     parent=torch.tensor(parent), children=children, planted_path=path,
                     max_depth=max_depth, depth=depth)


def op4_algorithmic_bytes(n: int, vocab: int, logit_bytes: int, num_committed: int,
                          layers: int, row_bytes: int) -> int:
    """logits read once + K and V rows read and written."""
    return n * vocab * logit_bytes + 2 * 2 * num_committed * layers * row_bytes


__all__ = ["OP1_CONFIGS", "Op1Inputs", "op1_workload", "op1_inputs", "op1_algorithmic_bytes",
           "op1_flops", "random_tree", "op4_workload", "Op4Inputs", "op4_algorithmic_bytes"]
