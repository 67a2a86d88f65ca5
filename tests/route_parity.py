"""The rule that routing ids are compared by against the reference's torch
router (used by tests/test_gpu_route_parity.py on the GPU and by
tests/test_route_parity_rule.py on planted cases on the CPU).

Rows whose expert ids differ between the device and torch are classified:

* an exact tie: torch's gates at the device's picks equal, position by
  position, its gates at its own picks, so the rows differ only in which of
  two exactly equal experts is taken.  torch.topk orders exact ties in an
  implementation-defined way; the device must take the lowest id among the
  tied kept experts, as the reference's routing kernel does with its
  first-occurrence argmax (treemoe/kernels/op1_tree_moe.py:226-232);
* a logit difference: the row has a logit that differs from torch's, or the
  keep set differs.

Anything else is an error.  ``require_bit_exact`` is the parity bar: equal
keep sets and no row explained by a logit difference, only exact ties.
"""

from __future__ import annotations

import torch


def classify_id_rows(ids_d: torch.Tensor, ids_t: torch.Tensor, gates_t: torch.Tensor,
                     keep_d: set, keep_t: set, logit_differs: torch.Tensor):
    """Returns (tie_rows, logit_rows).  ids_* [T, 2]; gates_t [T, E] torch's
    gates; keep_* the kept experts; logit_differs [T, E] bool."""
    rows = (ids_d != ids_t).any(1)
    tie_rows, logit_rows = [], []
    for r in rows.nonzero().flatten().tolist():
        gd = gates_t[r, ids_d[r]]
        gt = gates_t[r, ids_t[r]]
        if keep_d == keep_t and torch.equal(gd, gt):
            for k in range(2):
                if int(ids_d[r, k]) != int(ids_t[r, k]):
                    tied = [j for j in keep_d if gates_t[r, j] == gd[k]
                            and j not in ids_d[r, :k].tolist()]
                    assert int(ids_d[r, k]) == min(tied), (
                        f"row {r} slot {k}: exact tie among {sorted(tied)} resolved to "
                        f"{int(ids_d[r, k])}, not the lowest id")
            tie_rows.append(r)
            continue
        assert keep_d != keep_t or bool(logit_differs[r].any()), (
            f"row {r}: ids {ids_d[r].tolist()} vs torch {ids_t[r].tolist()} with identical "
            "logits and keep set and unequal gates")
        logit_rows.append(r)
    return tie_rows, logit_rows


def require_bit_exact(keep_d: set, keep_t: set, logit_rows: list) -> None:
    """The bar at the benchmark configurations: the keep sets are equal and
    every differing row is an exact tie."""
    assert keep_d == keep_t, f"keep set {sorted(keep_d)} differs from torch's {sorted(keep_t)}"
    assert not logit_rows, (
        f"rows {logit_rows} pick other experts than torch because a bf16 logit differs")
