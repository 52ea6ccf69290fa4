"""CPU check of the row-group partition of the varlen multi-query path
(dvattention_amd/csrc/dv_chunk.hip, dv_varlen_groups): tokens of a varlen call
with two or more packed tokens per sequence on average are cut into groups of
up to 16 consecutive tokens of one sequence, found from the running maximum of
cu_seqlens_q instead of a per-token search.

The partition below follows the kernel's steps (running maximum M, runs
[max(0, M[i-1]), min(T, M[i])) and the trailing run of sequence 0, group
counts, exclusive scan, binary search of each group's run) and is checked
against the oracle's direct definition of a token's sequence
(oracle.varlen_token_to_seq: the first i with t < cu_seqlens_q[i + 1]) on
random, sorted and malformed tables: every token lies in exactly one group,
each group holds 1-16 consecutive tokens of the one sequence the oracle
assigns to all of them, and the group count stays within the host's bound
T // 16 + W + 1 that sizes the table.
"""
import numpy as np
import pytest

from oracle import dvattn_oracle as O

TOK_BLK = 16


def groups_of(cu, T):
    W = len(cu) - 1
    M = np.maximum.accumulate(np.asarray(cu[1:], dtype=np.int64))
    runs = []
    for i in range(W + 1):
        a = 0 if i == 0 else max(0, int(M[i - 1]))
        b = T if i == W else min(T, int(M[i]))
        runs.append((a, b, 0 if i == W else i))
    cnt = [(b - a + TOK_BLK - 1) // TOK_BLK if b > a else 0 for a, b, _ in runs]
    base = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int64)
    total = int(base[-1])
    out = []
    for g in range(total):
        lo, hi = 0, W
        while lo < hi:  # the last run whose first group is <= g
            mid = (lo + hi + 1) // 2
            if base[mid] <= g:
                lo = mid
            else:
                hi = mid - 1
        a, b, w = runs[lo]
        t0 = a + (g - int(base[lo])) * TOK_BLK
        out.append((t0, min(TOK_BLK, b - t0), w))
    return out


def check(cu, T):
    seq = O.varlen_token_to_seq(np.asarray(cu, dtype=np.int64), T)
    groups = groups_of(cu, T)
    W = len(cu) - 1
    assert len(groups) <= T // TOK_BLK + W + 1
    seen = np.zeros(T, dtype=np.int64)
    for t0, n, w in groups:
        assert 1 <= n <= TOK_BLK and 0 <= t0 and t0 + n <= T, (cu, T, t0, n)
        assert all(seq[t] == w for t in range(t0, t0 + n)), (cu, T, t0, n, w, seq[t0:t0 + n])
        seen[t0:t0 + n] += 1
    assert (seen == 1).all(), (cu, T, seen)


@pytest.mark.parametrize("seed", range(400))
def test_varlen_groups_random_tables(seed):
    rng = np.random.default_rng(seed)
    W = int(rng.integers(1, 12))
    kind = seed % 4
    if kind == 0:    # sorted, runs of 0-40 tokens
        cu = [0] + np.cumsum(rng.integers(0, 41, size=W)).tolist()
        T = max(1, cu[-1])
    elif kind == 1:  # sorted, then some tokens past the table
        cu = [0] + np.cumsum(rng.integers(0, 20, size=W)).tolist()
        T = cu[-1] + int(rng.integers(1, 30))
    else:            # arbitrary values, negative and past T included
        T = int(rng.integers(1, 120))
        cu = [0] + rng.integers(-5, T + 20, size=W).tolist()
    check(cu, T)


def test_varlen_groups_edges():
    check([0, 16], 16)                       # one full group
    check([0, 17], 17)                       # 16 + 1
    check([0, 0, 0], 9)                      # every token past the table
    check([0, 4, 2, 5], 6)                   # a run emptied by an earlier larger entry
    check([0, 5, 20, 30], 12)                # entries past T
    check([0, 10, -3, 25, 12], 30)
    check(list(16 * np.arange(17)), 256)     # configuration 5 packed as varlen tokens
