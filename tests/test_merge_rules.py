"""The merge shortcuts of the search kernels against the full merge rules.

Both kernels drop, once the frontier B is full, every new key ranked at or
above B's last entry before sorting; the directional kernel also starts its
rank merge and dedup at the smallest new key's insertion point. These tests
replay random hops with both the full rule (sort B + new keys, dedup, clip
to bw) and the shortcut and require the same frontier. Keys are (distance,
id) pairs over tiny ranges, so ties and repeated ids are frequent.

Full rules:
  * plain search (beam_search.cuh sort/dedup/clip, device_kernels.cuh:
    154-288): keys with equal (distance, id) collapse to one, clip to bw;
  * directional search (merge_sort_tail and dedup_results,
    device_kernels.cuh:290-408): the sorted new keys merge after equal
    head keys, an entry is dropped when its id equals the previous
    entry's id, clip to bw.
"""

import random

INV = 0x7FFFFFFF


def _plain_full(B, T, bw):
    return sorted(set(B) | set(T))[:bw]


def _plain_short(B, T, bw):
    if len(B) == bw:
        T = [t for t in T if t < B[-1]]
    if not T:
        return list(B)
    return sorted(set(B) | set(T))[:bw]


def _dir_full(B, T, bw):
    tagged = sorted([(b, 0, i) for i, b in enumerate(B)] + [(t, 1, i) for i, t in enumerate(sorted(T))])
    merged = [x[0] for x in tagged]
    out = [c for m, c in enumerate(merged) if c[1] != (INV if m == 0 else merged[m - 1][1])]
    return out[:bw]


def _dir_short(B, T, bw):
    cnt = len(B)
    if cnt == bw:
        T = [t for t in T if t < B[-1]]
    if not T:
        return list(B)
    T = sorted(T)
    nb = [None] * (cnt + len(T))
    lo = [sum(1 for b in B if b <= t) for t in T]
    for i, t in enumerate(T):
        nb[i + lo[i]] = t
    lo0 = lo[0]
    for j in range(lo0, cnt):
        nb[j + sum(1 for t in T if t < B[j])] = B[j]
    assert all(x is not None for x in nb[lo0:])
    id0 = INV if lo0 == 0 else B[lo0 - 1][1]
    out = list(B[:lo0])
    for m in range(lo0, len(nb)):
        prev = id0 if m == lo0 else nb[m - 1][1]
        if nb[m][1] != prev:
            out.append(nb[m])
    return out[:bw]


def _replay(full, short, trials, seed):
    rng = random.Random(seed)
    for _ in range(trials):
        bw = rng.randint(1, 12)
        n_id, n_dist = rng.randint(1, 10), rng.randint(1, 6)
        key = lambda: (rng.randint(0, n_dist), rng.randint(0, n_id))
        B = [key()]
        for _ in range(rng.randint(0, 6)):
            B = full(B, [key() for _ in range(rng.randint(0, 8))], bw)
        T = [key() for _ in range(rng.randint(0, 8))]
        assert short(B, T, bw) == full(B, T, bw), (bw, B, T)


def test_plain_filter_matches_full_merge():
    _replay(_plain_full, _plain_short, 20000, 1)


def test_directional_filter_and_partial_merge_match_full_merge():
    _replay(_dir_full, _dir_short, 20000, 2)


def test_directional_rule_needs_the_filter_bound():
    """Sanity of the harness: a shortcut that also drops keys equal to or just
    below B's last entry disagrees with the full rule somewhere."""
    def too_eager(B, T, bw):
        if len(B) == bw and len(B) > 1:
            T = [t for t in T if t < B[-2]]
        return _dir_full(B, T, bw)

    try:
        _replay(_dir_full, too_eager, 20000, 3)
    except AssertionError:
        return
    raise AssertionError("the replay did not catch an over-eager filter")
