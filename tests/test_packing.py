"""Row packing policy (host only, CPU): the oracle pinned against the reference's own test vectors
(aspec tests/test_packing.py:35-70), hand-derived placements and brute force, then the native
library (`aspec_pack_work_aware_rows`, `aspec_count_eligible_anchor_starts`) bit-exact against the
oracle and against the policy's invariants."""

import time

import numpy as np
import pytest

from aspec_amd import packing as P
from oracle import packing as O


# ---- oracle pins -------------------------------------------------------------------------------

def test_oracle_reference_vectors():
    # tests/test_packing.py:35-48 of the reference: packed 18 tokens, 52 useful starts, 0, 1, 2 kept.
    # By hand: seeds 0 (7) and 1 (6); visiting order 2 (density 10, work 30), 4 (10, 20), 3 (0.5);
    # 2 fits both rows and leaves no slack in row 0; 4 only fits row 1; 3 fits nowhere.
    rows, tokens = O.pack_rows([7, 6, 3, 4, 2], [1, 1, 30, 2, 20], 2, 10)
    assert rows == [[0, 2], [1, 4]]
    assert tokens == [10, 8]
    # tests/test_packing.py:56-66: 68 unit samples on 4 ranks of 32 tokens, at most 64 selected.
    # By hand: all densities tie, so candidates go in index order, each to the fullest row that fits:
    # row 0 takes 4..34 (32 tokens), row 1 takes 35..63 before the limit of 64 samples stops it.
    rows, tokens = O.pack_rows([1] * 68, [1] * 68, 4, 32, max_selected=64)
    assert rows == [[0, *range(4, 35)], [1, *range(35, 64)], [2], [3]]
    assert tokens == [32, 30, 1, 1]
    # tests/test_packing.py:69-70: "2,8", length 10, block 4 -> supervised 2..9, anchors up to 6.
    assert O.eligible_anchor_starts([2, 8], 10, 4) == 5


def test_oracle_eligible_starts_brute_force():
    rng = np.random.default_rng(0)
    for _ in range(300):
        runs = rng.integers(0, 7, size=rng.integers(0, 8)).tolist()
        total = sum(runs)
        length = int(rng.integers(0, total + 4))
        block = int(rng.integers(0, 6))
        supervised = np.zeros(max(total, 1), bool)
        at = 0
        for k, n in enumerate(runs):
            supervised[at:at + n] = k % 2 == 1
            at += n
        want = sum(1 for p in range(total) if supervised[p] and block > 0 and p + block <= length) if length > 0 else 0
        assert O.eligible_anchor_starts(runs, length, block) == want


def test_oracle_single_rank_is_greedy_by_density():
    # One rank: the seed stays, then samples are taken in visiting order while they still fit.
    # Densities of samples 1..5: 1, 2, 0.5, 2, 3; samples 2 and 4 tie at 2 and work (8 > 6) puts
    # 2 first, so the visiting order is 5, 2, 4, 1, 3. Tokens: 5 -> 6 -> 10; 4 (3) and 1 (4) no
    # longer fit under 12; 3 (2) fills the row to 12.
    rows, tokens = O.pack_rows([5, 4, 4, 2, 3, 1], [0, 4, 8, 1, 6, 3], 1, 12)
    assert rows == [[0, 5, 2, 3]]
    assert tokens == [12]


def _check_invariants(rows, tokens, lengths, work, dp, cap, max_selected):
    flat = [i for r in rows for i in r]
    assert len(flat) == len(set(flat))
    assert sorted(r[0] for r in rows) == list(range(dp))  # every row is seeded by one of the oldest
    assert all(sum(lengths[i] for i in r) == t <= cap for r, t in zip(rows, tokens))
    assert all(tokens[k] >= tokens[k + 1] for k in range(dp - 1))
    if max_selected is not None:
        assert len(flat) <= max_selected
    # replay in visiting order: each placed sample went to a fullest fitting row, each skipped one fit
    # nowhere (or the selection limit was reached)
    where = {i: k for k, r in enumerate(rows) for i in r}
    used = {k: lengths[r[0]] for k, r in enumerate(rows)}
    order = sorted(range(dp, len(lengths)), key=lambda i: (-(work[i] / lengths[i]), -work[i], -lengths[i], i))
    taken = dp
    for i in order:
        if max_selected is not None and taken >= max_selected:
            assert i not in where
            continue
        fits = [k for k in used if used[k] + lengths[i] <= cap]
        if not fits:
            assert i not in where
            continue
        k = where[i]
        assert used[k] == max(used[f] for f in fits)
        used[k] += lengths[i]
        taken += 1
    assert used == dict(enumerate(tokens))


def test_oracle_invariants_on_random_pools():
    rng = np.random.default_rng(1)
    for trial in range(60):
        dp = int(rng.integers(1, 6))
        cap = int(rng.integers(4, 40))
        n = int(rng.integers(dp, dp + 30))
        lengths = rng.integers(1, cap + 1, size=n).tolist()
        work = rng.integers(0, 12, size=n).tolist()
        max_selected = None if trial % 3 else int(rng.integers(dp, n + 2))
        rows, tokens = O.pack_rows(lengths, work, dp, cap, max_selected)
        _check_invariants(rows, tokens, lengths, work, dp, cap, max_selected)


# ---- native library against the oracle ---------------------------------------------------------

def test_reference_cases_through_the_library():
    r = P.pack_work_aware_rows([7, 6, 3, 4, 2], [1, 1, 30, 2, 20], dp_size=2, max_seq_length=10)
    assert r.rank_rows == [[0, 2], [1, 4]]
    assert r.selected_indices == (0, 1, 2, 4)
    assert (r.packed_tokens, r.useful_anchor_starts, r.capacity_tokens) == (18, 52, 20)
    assert r.fill_ratio == pytest.approx(0.9)
    r = P.pack_work_aware_rows([1] * 68, [1] * 68, dp_size=4, max_seq_length=32, max_selected=64)
    assert len(r.selected_indices) == 64
    assert P.count_eligible_anchor_starts("2,8", sample_length=10, block_size=4) == 5
    assert P.count_eligible_anchor_starts([2, 8], sample_length=10, block_size=0) == 0
    assert P.pack_work_aware_rows([3], [1], dp_size=2, max_seq_length=10) is None


def test_library_errors_match_the_reference():
    with pytest.raises(ValueError, match="can never fit"):
        P.pack_work_aware_rows([11], [1], dp_size=1, max_seq_length=10)
    with pytest.raises(ValueError, match=r"0:0, 2:12; max_seq_length=10"):
        P.pack_work_aware_rows([0, 3, 12], [1, 1, 1], dp_size=1, max_seq_length=10)
    with pytest.raises(ValueError, match="same size"):
        P.pack_work_aware_rows([1, 2], [1], dp_size=1, max_seq_length=10)
    with pytest.raises(ValueError, match="must be positive"):
        P.pack_work_aware_rows([1], [1], dp_size=0, max_seq_length=10)
    with pytest.raises(ValueError, match="at least dp_size"):
        P.pack_work_aware_rows([1, 1], [1, 1], dp_size=2, max_seq_length=10, max_selected=1)
    with pytest.raises(ValueError, match="non-integer"):
        P.count_eligible_anchor_starts("2,x", sample_length=10, block_size=4)
    with pytest.raises(ValueError, match="non-negative"):
        P.count_eligible_anchor_starts("2,-1", sample_length=10, block_size=4)


def test_library_eligible_starts_match_oracle_batched():
    rng = np.random.default_rng(2)
    masks, lengths, want = [], [], []
    for _ in range(500):
        runs = rng.integers(0, 40, size=rng.integers(0, 12)).tolist()
        length = int(rng.integers(-2, sum(runs) + 8))
        masks.append(",".join(map(str, runs)) if len(masks) % 2 else runs)
        lengths.append(length)
        want.append(O.eligible_anchor_starts(runs, length, 16))
    assert P.count_eligible_anchor_starts_batch(masks, lengths, 16) == want


@pytest.mark.parametrize("seed", range(8))
def test_library_matches_oracle_on_random_pools(seed):
    rng = np.random.default_rng(100 + seed)
    for trial in range(25):
        dp = int(rng.integers(1, 9))
        cap = int(rng.integers(8, 4097))
        n = int(rng.integers(0, dp + 120))
        # few distinct lengths and works so that density, work and length ties all occur
        lengths = rng.choice([1, 2, 3, 6, cap // 3 + 1, cap // 2, cap], size=n).tolist()
        work = (rng.integers(0, 4, size=n) * rng.choice([1, 2, 3], size=n)).tolist()
        max_selected = None if trial % 4 else int(rng.integers(dp, dp + 60))
        got = P.pack_work_aware_rows(lengths, work, dp_size=dp, max_seq_length=cap, max_selected=max_selected)
        want = O.pack_rows(lengths, work, dp, cap, max_selected)
        if want is None:
            assert got is None
            continue
        rows, tokens = want
        assert got.rank_rows == rows
        assert got.packed_tokens == sum(tokens)
        assert got.selected_indices == tuple(sorted(i for r in rows for i in r))
        assert got.useful_anchor_starts == sum(work[i] for r in rows for i in r)


def test_library_density_ties_are_exact_double_quotients():
    # 1/3 and 2/6 are the same double, as are 3/30 and 1/10, so work breaks both ties: the visiting
    # order is 2, 1, 3, 4. Tokens 10 -> 16 -> 19; 3 (30) does not fit under 40; 4 (10) gives 29.
    lengths, work = [10, 3, 6, 30, 10], [0, 1, 2, 3, 1]
    r = P.pack_work_aware_rows(lengths, work, dp_size=1, max_seq_length=40)
    assert r.rank_rows == [[0, 2, 1, 4]]
    assert r.packed_tokens == 29
    assert O.pack_rows(lengths, work, 1, 40) == ([[0, 2, 1, 4]], [29])


def test_library_large_pool_invariants_and_speed():
    rng = np.random.default_rng(3)
    n, dp, cap = 200_000, 512, 32768
    lengths = rng.integers(1, 8192, size=n).tolist()
    work = rng.integers(0, 4096, size=n).tolist()
    t0 = time.perf_counter()
    r = P.pack_work_aware_rows(lengths, work, dp_size=dp, max_seq_length=cap)
    elapsed = time.perf_counter() - t0
    tokens = [sum(lengths[i] for i in row) for row in r.rank_rows]
    assert all(t <= cap for t in tokens)
    assert all(tokens[k] >= tokens[k + 1] for k in range(dp - 1))
    assert sorted(row[0] for row in r.rank_rows) == list(range(dp))
    assert r.fill_ratio > 0.99
    assert elapsed < 5.0, elapsed
