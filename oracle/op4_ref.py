"""TEST INFRASTRUCTURE ONLY: restatement of the op4 reference.

* ``tree_verify``  treemoe/ref/verify_ref.py:35-103 (greedy branch exactly;
  sampling branch with the generator's draws on the logits' device, or with
  injected uniforms and bonus exponentials).  Depth is unbounded, as in the
  reference.
* ``exp_race``     torch.multinomial(p, 1, generator)'s one-sample draw
  (argmax of p / e, e = empty_like(p).exponential_(1, generator)), which
  the bonus of the sampling branch (verify_ref.py:87) is.
* ``commit_tree``  treemoe/model/kv_cache.py:88-106 generalised to a page size
  P: tree slot s lives in scratch page ``scratch_pages[s // P]`` at offset
  ``s % P``; sequence position q lives in ``block_table[q // P]`` at ``q % P``.
"""

from __future__ import annotations

import torch


def tree_verify(target_logits: torch.Tensor, draft_probs: torch.Tensor,
                tree_tokens: torch.Tensor, children: list[list[int]],
                temperature: float = 0.0, uniforms: torch.Tensor | None = None,
                generator: torch.Generator | None = None,
                bonus_exp: torch.Tensor | None = None, return_residual: bool = False):
    """Returns (accepted_slots [N], accepted_tokens [N], bonus, num_accepted)
    (+ the final residual when return_residual).  Without injected uniforms
    the draws come from ``generator`` on the logits' device in the
    reference's order (rand(N), then multinomial's exponentials); with
    bonus_exp the sampling-mode bonus is ``exp_race(residual, bonus_exp)``."""
    n = target_logits.shape[0]
    slots: list[int] = []
    toks: list[int] = []
    if temperature != 0.0 and uniforms is None:
        uniforms = torch.rand(n, generator=generator, device=target_logits.device)
    node = 0
    while True:
        if temperature == 0.0:
            best = int(target_logits[node].argmax())
            residual = None
        else:
            residual = torch.softmax(target_logits[node] / temperature, dim=-1)
        taken = -1
        for c in children[node]:
            tok = int(tree_tokens[c])
            if temperature == 0.0:
                ok = tok == best
            else:
                q = draft_probs[c]
                ratio = (residual[tok] / q[tok].clamp_min(1e-20)).clamp(max=1.0)
                ok = bool(uniforms[c] < ratio)
                if not ok:
                    residual = (residual - q).clamp_min(0)
                    residual = residual / residual.sum().clamp_min(1e-20)
            if ok:
                taken = c
                break
        if taken < 0:
            if temperature == 0.0:
                bonus = best
            elif bonus_exp is not None:
                bonus = exp_race(residual, bonus_exp)
            else:
                bonus = int(torch.multinomial(residual, 1, generator=generator))
            break
        slots.append(taken)
        toks.append(int(tree_tokens[taken]))
        node = taken
    acc_slots = torch.full((n,), -1, dtype=torch.long)
    acc_toks = torch.full((n,), -1, dtype=torch.long)
    if slots:
        acc_slots[: len(slots)] = torch.tensor(slots)
        acc_toks[: len(toks)] = torch.tensor(toks)
    if return_residual:
        return acc_slots, acc_toks, bonus, len(slots), residual
    return acc_slots, acc_toks, bonus, len(slots)


def exp_race(probs: torch.Tensor, e: torch.Tensor) -> int:
    """First index of the largest probs[j] / e[j] in fp32 (IEEE division):
    the index torch.multinomial(probs, 1, generator) returns when e is
    empty_like(probs).exponential_(1, generator) from the same state."""
    return int(torch.argmax(probs.float() / e.float()))


def rep_penalty_inplace(logits: torch.Tensor, prev_tokens, penalty: float) -> None:
    """Reference `_postprocess_softmax_kernel` pass 0
    (treemoe/kernels/op4_commit.py:53-57) on every row: for each prev token in
    order, x = x / penalty if x > 0 else x * penalty, each time loaded from and
    stored to the tensor (so bf16 rows round after every application)."""
    v = logits.shape[1]
    for t in [int(t) for t in prev_tokens]:
        if t < 0 or t >= v:
            continue
        col = logits[:, t].float()
        col = torch.where(col > 0, col / penalty, col * penalty)
        logits[:, t] = col.to(logits.dtype)


def commit_tree(k: torch.Tensor, v: torch.Tensor, commit_slots: torch.Tensor,
                scratch_pages: list[int], block_table: list[int], seq_len: int) -> int:
    """Copy the K/V rows of the valid (>= 0) tree slots in ``commit_slots`` to
    positions seq_len, seq_len+1, ...; returns the number of rows committed.
    k, v: [L, pages, P, kvh, hd] (any device, modified in place)."""
    page = k.shape[2]
    valid = commit_slots[commit_slots >= 0].tolist()
    if not valid:
        return 0
    src_p = torch.tensor([scratch_pages[s // page] for s in valid], dtype=torch.long)
    src_o = torch.tensor([s % page for s in valid], dtype=torch.long)
    pos = [seq_len + j for j in range(len(valid))]
    dst_p = torch.tensor([block_table[q // page] for q in pos], dtype=torch.long)
    dst_o = torch.tensor([q % page for q in pos], dtype=torch.long)
    dev = k.device
    src_p, src_o, dst_p, dst_o = (t.to(dev) for t in (src_p, src_o, dst_p, dst_o))
    k[:, dst_p, dst_o] = k[:, src_p, src_o]
    v[:, dst_p, dst_o] = v[:, src_p, src_o]
    return len(valid)
