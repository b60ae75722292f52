"""Row packing policy restated in plain Python. TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

  eligible_anchor_starts  count_eligible_anchor_starts (aspec/controller/packing.py:43-67)
  pack_rows               pack_work_aware_rows         (aspec/controller/packing.py:87-167)

Pinned by tests/test_oracle_packing.py: the reference's own test vectors (tests/test_packing.py:35-70),
hand-derived placements, brute-force enumeration of eligible starts, and the policy's invariants
(row capacity, oldest-sample seeding, best fit at every placement, max_selected, rank order).
"""

from __future__ import annotations


def eligible_anchor_starts(runs, sample_length, block_size):
    """Supervised positions p (odd runs of the alternating run-length mask) with
    p + block_size <= sample_length."""
    if sample_length <= 0 or block_size <= 0:
        return 0
    total = 0
    start = 0
    supervised = False
    for n in runs:
        if n < 0:
            raise ValueError("packed_loss_mask run lengths must be non-negative")
        if supervised:
            last_anchor = sample_length - block_size  # inclusive
            lo, hi = start, min(start + n - 1, last_anchor)
            total += max(0, hi - lo + 1)
        start += n
        supervised = not supervised
    return total


def pack_rows(lengths, useful_work, dp_size, max_seq_length, max_selected=None):
    """(rank_rows, row_tokens) as lists, or None for a pool smaller than dp_size. Inputs are assumed
    valid (the product validates)."""
    if len(lengths) < dp_size:
        return None
    rows = [[r] for r in range(dp_size)]
    used = [lengths[r] for r in range(dp_size)]
    rest = list(range(dp_size, len(lengths)))

    def before(a, b):
        da, db = useful_work[a] / lengths[a], useful_work[b] / lengths[b]
        for x, y in ((da, db), (useful_work[a], useful_work[b]), (lengths[a], lengths[b])):
            if x != y:
                return x > y
        return a < b

    # selection sort by the visiting order: quadratic, fine for the sizes the tests use
    ordered = []
    while rest:
        best = rest[0]
        for c in rest[1:]:
            if before(c, best):
                best = c
        ordered.append(best)
        rest.remove(best)

    taken = dp_size
    for i in ordered:
        if max_selected is not None and taken >= max_selected:
            break
        target = None
        for r in range(dp_size):
            if used[r] + lengths[i] > max_seq_length:
                continue
            if target is None or used[r] > used[target]:  # least slack; first row wins ties
                target = r
        if target is None:
            continue
        rows[target].append(i)
        used[target] += lengths[i]
        taken += 1

    ranks = list(range(dp_size))
    ranks.sort(key=lambda r: (-used[r], r))
    return [rows[r] for r in ranks], [used[r] for r in ranks]
