"""CPU checks of the k-NN kernel's candidate networks (torchbvh_amd/csrc/knn.hip).

A bucket's candidates enter the k-list through fixed compare-exchange
networks; their tables are read here from the kernel source and proved on the
CPU, so a mistyped comparator or rank fails before any GPU run:

* the 6- and 8-input sorting networks sort every 0/1 input (the 0-1
  principle: a comparator network that sorts all 0/1 sequences sorts all
  sequences, Knuth, TAOCP vol. 3, 5.3.4);
* the 6 + 6 merge (kMerge66, kRank12) turns every pair of sorted 0/1 halves
  into a sorted sequence of 12, read in rank order;
* the half-cleaner + bitonic merge with MergePlan's pruning keeps exactly
  the K smallest keys of list and candidates, against a sorted union, for
  K = 4, 8, 16, 32 and 6, 8 or 12 candidates (absent ones are the empty key).
"""

from __future__ import annotations

import itertools
import random
import re
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parents[1] / "torchbvh_amd" / "csrc" / "knn.hip"


def _pairs(text: str) -> list[tuple[int, int]]:
    return [(int(a), int(b)) for a, b in re.findall(r"\{\s*(\d+)\s*,\s*(\d+)\s*\}", text)]


def _tables():
    s = SRC.read_text()
    sort_fn = s[s.index("void sort_candidates("):s.index("template <int K, int M>\nstruct MergePlan")]
    net6_txt = sort_fn[sort_fn.index("constexpr int net[12][2]"):sort_fn.index("} else {")]
    net8_txt = sort_fn[sort_fn.index("constexpr int net[19][2]"):]
    m66_txt = s[s.index("constexpr int kMerge66[17][2]"):s.index("constexpr int kRank12")]
    rank_txt = s[s.index("constexpr int kRank12[12]"):]
    rank = [int(x) for x in re.search(r"kRank12\[12\]\s*=\s*\{([^}]*)\}", rank_txt).group(1).split(",")]
    return _pairs(net6_txt)[:12], _pairs(net8_txt)[:19], _pairs(m66_txt)[:17], rank


NET6, NET8, MERGE66, RANK12 = _tables()


def _run(net, v):
    v = list(v)
    for a, b in net:
        if v[a] > v[b]:
            v[a], v[b] = v[b], v[a]
    return v


def _plan(K: int, m: int) -> list[int]:
    """MergePlan<K, m>::needed, restated: an exchange runs unless both of its
    slots still hold the list's own (sorted) entries."""
    touched = ((1 << m) - 1) << (K - m)
    needed = []
    h = K // 2
    while h >= 1:
        bits, nxt = 0, touched
        for i in range(K):
            if i & h == 0 and ((touched >> i) | (touched >> (i + h))) & 1:
                bits |= 1 << i
                nxt |= (1 << i) | (1 << (i + h))
        needed.append(bits)
        touched = nxt
        h //= 2
    return needed


def _merge(best, sorted_c, K):
    """merge_candidates' half-cleaner and pruned bitonic merge."""
    m = min(K, len(sorted_c))
    best = list(best)
    for i in range(m):
        best[K - m + i] = min(best[K - m + i], sorted_c[m - 1 - i])
    h, s = K // 2, 0
    plan = _plan(K, m)
    while h >= 1:
        for i in range(K):
            if i & h == 0 and (plan[s] >> i) & 1:
                lo, hi = best[i], best[i + h]
                best[i], best[i + h] = min(lo, hi), max(lo, hi)
        h //= 2
        s += 1
    return best


def test_tables_have_expected_sizes():
    assert len(NET6) == 12 and len(NET8) == 19 and len(MERGE66) == 17
    assert sorted(RANK12) == list(range(12))


@pytest.mark.parametrize("n,net", [(6, NET6), (8, NET8)])
def test_sorting_networks_sort_all_01_inputs(n, net):
    for bits in itertools.product((0, 1), repeat=n):
        assert _run(net, bits) == sorted(bits), bits


def test_six_plus_six_merge_sorts_all_sorted_01_halves():
    halves = [tuple([0] * z + [1] * (6 - z)) for z in range(7)]
    for a in halves:
        for b in halves:
            v = _run(MERGE66, a + b)
            assert [v[r] for r in RANK12] == sorted(a + b), (a, b)
    # and the full 12-input sort (two 6-sorts, then the merge) on all 0/1 inputs
    for bits in itertools.product((0, 1), repeat=12):
        v = _run(NET6, bits[:6]) + _run(NET6, bits[6:])
        v = _run(MERGE66, v)
        assert [v[r] for r in RANK12] == sorted(bits)


@pytest.mark.parametrize("K", [4, 8, 16, 32])
@pytest.mark.parametrize("B", [6, 8, 12])
def test_merge_keeps_the_k_smallest(K, B):
    empty = 10**9
    rng = random.Random(K * 100 + B)
    for _ in range(4000):
        pool = rng.sample(range(5000), K + B)
        filled = rng.randint(0, K)
        best = sorted(pool[:filled]) + [empty] * (K - filled)
        present = rng.randint(0, B)
        cand = pool[K:K + present] + [empty] * (B - present)
        rng.shuffle(cand)
        if B == 6:
            sc = _run(NET6, cand)
        elif B == 8:
            sc = _run(NET8, cand)
        else:
            v = _run(MERGE66, _run(NET6, cand[:6]) + _run(NET6, cand[6:]))
            sc = [v[r] for r in RANK12]
        assert _merge(best, sc, K) == sorted(best + cand)[:K]


@pytest.mark.parametrize("K,m,count", [(16, 6, 30), (32, 6, 66), (32, 12, 76), (16, 12, 32), (8, 8, 12)])
def test_merge_plan_sizes(K, m, count):
    assert sum(bin(x).count("1") for x in _plan(K, m)) == count


def test_checks_catch_a_dropped_comparator():
    """Each network minus any one comparator fails the 0/1 check, so the
    tests above would catch a mistyped table."""
    for n, net in ((6, NET6), (8, NET8)):
        for drop in range(len(net)):
            bad = net[:drop] + net[drop + 1:]
            assert any(_run(bad, b) != sorted(b) for b in itertools.product((0, 1), repeat=n)), (n, drop)
    for drop in range(len(MERGE66)):
        bad = MERGE66[:drop] + MERGE66[drop + 1:]
        fails = False
        for bits in itertools.product((0, 1), repeat=12):
            v = _run(bad, _run(NET6, bits[:6]) + _run(NET6, bits[6:]))
            if [v[r] for r in RANK12] != sorted(bits):
                fails = True
                break
        assert fails, drop
