"""Test harness: a tiny Mixtral-shaped target driven like the reference's
SpecDecodeEngine (treemoe/engine/loop.py:150-200), with the hot path on this
build's kernels:

* attention of every forward = ``tree_attention`` over the paged cache (a
  one-node tree for an AR step; the draft tree's ancestor mask for a
  verification step), which also stores the forward's K/V in the scratch pages;
* the MoE of every layer = ``make_moe_fn`` (route_experts + tree_moe_forward);
* verification and commit = ``fused_verify_commit`` with the cache, which moves
  [root] + accepted path from the scratch pages to the sequence tail.

Projections, norms, RoPE and the LM head are float32 torch (plumbing).  An AR
step is a verification step of a one-node tree: nothing to accept, the root is
committed and the bonus token (argmax of its logits) is the next token.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class TinyConfig:
    num_layers: int = 2
    num_experts: int = 8
    hidden_dim: int = 512
    intermediate_dim: int = 512
    num_heads: int = 4
    num_kv_heads: int = 2
    head_dim: int = 128
    vocab_size: int = 256
    page_size: int = 16
    tree_size: int = 16
    rope_theta: float = 1e4
    rms_eps: float = 1e-5


@dataclass
class Layer:
    ln1: torch.Tensor
    ln2: torch.Tensor
    wq: torch.Tensor
    wk: torch.Tensor
    wv: torch.Tensor
    wo: torch.Tensor
    router: torch.Tensor
    w1: torch.Tensor
    w2: torch.Tensor
    w3: torch.Tensor


def random_model(cfg: TinyConfig, seed: int, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    h, i, e = cfg.hidden_dim, cfg.intermediate_dim, cfg.num_experts
    qd, kd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim

    def r(*shape, scale=0.02, dtype=torch.float32):
        return (torch.randn(*shape, generator=g) * scale).to(dtype).to(device)

    layers = [Layer(ln1=torch.ones(h, device=device), ln2=torch.ones(h, device=device),
                    wq=r(qd, h, scale=h ** -0.5), wk=r(kd, h, scale=h ** -0.5),
                    wv=r(kd, h, scale=h ** -0.5), wo=r(h, qd, scale=qd ** -0.5),
                    router=r(e, h, dtype=torch.bfloat16),
                    w1=r(e, i, h, scale=h ** -0.5, dtype=torch.bfloat16),
                    w2=r(e, h, i, scale=i ** -0.5, dtype=torch.bfloat16),
                    w3=r(e, i, h, scale=h ** -0.5, dtype=torch.bfloat16))
              for _ in range(cfg.num_layers)]
    embed = r(cfg.vocab_size, h, scale=1.0)
    lm_head = r(cfg.vocab_size, h, scale=h ** -0.5)
    return layers, embed, lm_head


def rms_norm(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rope(x, positions, theta):
    """Rotate-half RoPE, float32: x [T, heads, hd], positions [T]."""
    hd = x.shape[-1]
    inv = theta ** (-torch.arange(0, hd, 2, device=x.device, dtype=torch.float32) / hd)
    ang = positions.float()[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[:, None, :]
    x1, x2 = x[..., : hd // 2], x[..., hd // 2:]
    return x * cos + torch.cat([-x2, x1], -1) * sin


class TinyEngine:
    def __init__(self, cfg: TinyConfig, model, num_pages: int = 64, device="cuda"):
        from treemoe_spec_amd.kv_cache import MixtralConfig, PagedKVCache
        from treemoe_spec_amd.moe_adapter import make_moe_fn

        self.cfg = cfg
        self.layers, self.embed, self.lm_head = model
        kcfg = MixtralConfig(num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads,
                             head_dim=cfg.head_dim, num_heads=cfg.num_heads)
        self.kv = PagedKVCache(kcfg, num_pages, device=device, page_size=cfg.page_size,
                               tree_size=cfg.tree_size)
        self.moe_fn = make_moe_fn(expert_budget=cfg.num_experts, tree_size=cfg.tree_size,
                                  device=device)
        self.device = device

    def forward(self, tokens, positions, tree_mask):
        from treemoe_spec_amd.kernels.tree_attention import tree_attention

        cfg = self.cfg
        t = tokens.shape[0]
        x = self.embed[tokens]
        for li, lw in enumerate(self.layers):
            h = rms_norm(x, lw.ln1, cfg.rms_eps)
            q = rope((h @ lw.wq.T).view(t, cfg.num_heads, cfg.head_dim), positions,
                     cfg.rope_theta)
            k = rope((h @ lw.wk.T).view(t, cfg.num_kv_heads, cfg.head_dim), positions,
                     cfg.rope_theta)
            v = (h @ lw.wv.T).view(t, cfg.num_kv_heads, cfg.head_dim)
            o = tree_attention(q.to(torch.bfloat16).contiguous(),
                               k.to(torch.bfloat16).contiguous(),
                               v.to(torch.bfloat16).contiguous(), self.kv, li, tree_mask)
            x = x + o.float() @ lw.wo.T
            h2 = rms_norm(x, lw.ln2, cfg.rms_eps).to(torch.bfloat16)
            x = x + self.moe_fn(h2, lw, li).float()
        return rms_norm(x, 1.0, cfg.rms_eps) @ self.lm_head.T

    def verify(self, tokens, parent, children, depth):
        """One verification step over a tree whose root is the last token
        (uncommitted); returns (accepted tokens, bonus, logits)."""
        from treemoe_spec_amd.kernels.op4_commit import fused_verify_commit
        from oracle.attn_ref import ancestor_mask

        n = tokens.shape[0]
        positions = torch.tensor([self.kv.seq_len + d for d in depth], device=self.device)
        mask = ancestor_mask(parent).to(self.device)
        logits = self.forward(tokens, positions, mask)
        res = fused_verify_commit(logits.float(), None, tokens, None, children, kv=self.kv,
                                  max_depth=max(depth) if n > 1 else 0)
        num = int(res.num_accepted)
        accepted = res.accepted_tokens[:num].tolist()
        return accepted, int(res.bonus_token), logits

    def ar_step(self, token: int):
        t = torch.tensor([token], device=self.device)
        _, bonus, logits = self.verify(t, [-1], [[]], [0])
        return bonus, logits[0]


def ar_generate(engine: TinyEngine, prompt: list[int], n: int):
    """Greedy AR: returns the n next tokens and each step's top-2 logit margin."""
    for tok in prompt[:-1]:
        engine.ar_step(tok)
    out, margins = [], []
    tok = prompt[-1]
    while len(out) < n:
        tok, logits = engine.ar_step(tok)
        top = logits.float().topk(2).values
        margins.append(float(top[0] - top[1]))
        out.append(tok)
    return out, margins


def planted_tree(root: int, truth: list[int], vocab: int, g: torch.Generator,
                 depth_max: int = 3, follow: float = 0.75):
    """Root plus two children per node to depth_max (15 nodes).  Child 0 of a
    node on the planted path proposes the true next token with probability
    `follow`; every other child proposes a random token.  Parents precede
    children (DFS order is not needed by the kernels)."""
    tokens, parent, depth, on_path = [root], [-1], [0], [True]
    frontier = [0]
    for d in range(1, depth_max + 1):
        nxt = []
        for p in frontier:
            for c in range(2):
                tok = int(torch.randint(0, vocab, (1,), generator=g))
                planted = on_path[p] and c == 0 and d - 1 < len(truth) \
                    and float(torch.rand(1, generator=g)) < follow
                if planted:
                    tok = truth[d - 1]
                tokens.append(tok)
                parent.append(p)
                depth.append(d)
                on_path.append(planted)
                nxt.append(len(tokens) - 1)
        frontier = nxt
    children = [[] for _ in tokens]
    for i, p in enumerate(parent):
        if p >= 0:
            children[p].append(i)
    return tokens, parent, children, depth


def spec_generate(engine: TinyEngine, prompt: list[int], n: int, truth: list[int],
                  seed: int):
    """Speculative decoding with planted trees; returns (tokens, steps, accepted)."""
    g = torch.Generator().manual_seed(seed)
    for tok in prompt[:-1]:
        engine.ar_step(tok)
    out = []
    root = prompt[-1]
    steps = accepted_total = 0
    while len(out) < n:
        tokens, parent, children, depth = planted_tree(root, truth[len(out):],
                                                       engine.cfg.vocab_size, g)
        t = torch.tensor(tokens, device=engine.device)
        accepted, bonus, _ = engine.verify(t, parent, children, depth)
        out.extend(accepted + [bonus])
        accepted_total += len(accepted)
        steps += 1
        root = bonus
    return out[:n], steps, accepted_total
