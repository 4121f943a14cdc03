"""torch.topk's CPU selection, restated -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference selects kept blocks and tile entries with torch.topk
(legacy/sparse_modeling.py:568, :649, :707, :1339, :1446, :1514).  On the CPU,
torch.topk (ATen native/TopKImpl.h, topk_impl_loop) turns each slice into
(value, index) pairs compared by value only -- NaN above every number and equal
to NaN, -0 == +0 -- and runs std::partial_sort(first, first + k, last) when
k * 64 <= n, else std::nth_element(first, first + k - 1, last); the first k
pairs are the kept entries.  Which of several equal values are kept is fixed
by those two algorithms.  They come from GCC's libstdc++ (a dependency of the
torch build, not part of the reference tree): bits/stl_algo.h __introselect,
__unguarded_partition_pivot, __move_median_to_first, __unguarded_partition,
__insertion_sort, __unguarded_linear_insert, __heap_select and
bits/stl_heap.h __make_heap, __adjust_heap, __push_heap, __pop_heap, whose
published algorithms are restated here.  The comparator `a before b` is
key(a) > key(b) on numerics.ordered_keys.

Each partition step is evaluated in its data-parallel form: the left scan of
the unguarded partition stops at positions whose key is <= the pivot's, the
right scan at keys >= the pivot's; the i-th left stop (ascending) is swapped
with the i-th right stop (descending) while it lies before it, and the cut is
min(next left stop, last right stop swapped).  That is the same permutation
the sequential scans produce (the scans only pass untouched positions and
stop at swapped ones).

Pinned against torch.topk itself on tie-heavy inputs with NaN and -0 through
both the partial-sort and the introselect branch (tests/test_oracle_select.py).
"""
from __future__ import annotations

import numpy as np

from .numerics import ordered_keys


class _Pairs:
    """(key, index) pairs as two int64 arrays; `before(i, j)` is the libstdc++ comparator."""

    def __init__(self, keys: np.ndarray):
        self.k = keys.astype(np.int64)
        self.i = np.arange(keys.size, dtype=np.int64)

    def before(self, a: int, b: int) -> bool:
        return bool(self.k[a] > self.k[b])

    def swap(self, a: int, b: int) -> None:
        self.k[a], self.k[b] = self.k[b], self.k[a]
        self.i[a], self.i[b] = self.i[b], self.i[a]

    def get(self, a: int):
        return int(self.k[a]), int(self.i[a])

    def put(self, a: int, v) -> None:
        self.k[a], self.i[a] = v


def _move_median_to_first(p: _Pairs, result: int, a: int, b: int, c: int) -> None:
    if p.before(a, b):
        if p.before(b, c):
            p.swap(result, b)
        elif p.before(a, c):
            p.swap(result, c)
        else:
            p.swap(result, a)
    elif p.before(a, c):
        p.swap(result, a)
    elif p.before(b, c):
        p.swap(result, c)
    else:
        p.swap(result, b)


def _partition(p: _Pairs, first: int, last: int) -> int:
    """__unguarded_partition(first + 1, last, pivot = first) in its data-parallel form."""
    piv = p.k[first]
    seg = p.k[first:last]
    pos = np.arange(first, last, dtype=np.int64)
    is_l = seg <= piv
    is_l[0] = False  # the left scan starts at first + 1
    left = pos[is_l]
    right = pos[seg >= piv][::-1]
    n = min(left.size, right.size)
    ok = left[:n] < right[:n]
    m = n if ok.all() else int(np.argmin(ok))
    cut = int(left[m]) if m < left.size else last
    if m >= 1:
        cut = min(cut, int(right[m - 1]))
    a, b = left[:m], right[:m]
    p.k[a], p.k[b] = p.k[b].copy(), p.k[a].copy()
    p.i[a], p.i[b] = p.i[b].copy(), p.i[a].copy()
    return cut


def _insertion_sort(p: _Pairs, first: int, last: int) -> None:
    if first == last:
        return
    for i in range(first + 1, last):
        if p.before(i, first):
            val = p.get(i)
            p.k[first + 1:i + 1] = p.k[first:i].copy()
            p.i[first + 1:i + 1] = p.i[first:i].copy()
            p.put(first, val)
        else:
            val = p.get(i)
            j, nxt = i, i - 1
            while val[0] > p.k[nxt]:
                p.put(j, p.get(nxt))
                j, nxt = nxt, nxt - 1
            p.put(j, val)


def _adjust_heap(p: _Pairs, first: int, hole: int, length: int, value) -> None:
    top = second = hole
    while second < (length - 1) // 2:
        second = 2 * (second + 1)
        if p.before(first + second, first + second - 1):
            second -= 1
        p.put(first + hole, p.get(first + second))
        hole = second
    if (length & 1) == 0 and second == (length - 2) // 2:
        second = 2 * (second + 1)
        p.put(first + hole, p.get(first + second - 1))
        hole = second - 1
    parent = (hole - 1) // 2  # __push_heap
    while hole > top and p.k[first + parent] > value[0]:
        p.put(first + hole, p.get(first + parent))
        hole = parent
        parent = (hole - 1) // 2
    p.put(first + hole, value)


def _make_heap(p: _Pairs, first: int, last: int) -> None:
    length = last - first
    if length < 2:
        return
    parent = (length - 2) // 2
    while True:
        _adjust_heap(p, first, parent, length, p.get(first + parent))
        if parent == 0:
            return
        parent -= 1


def _heap_select(p: _Pairs, first: int, middle: int, last: int) -> None:
    _make_heap(p, first, middle)
    for i in range(middle, last):
        if p.before(i, first):  # __pop_heap(first, middle, i)
            value = p.get(i)
            p.put(i, p.get(first))
            _adjust_heap(p, first, 0, middle - first, value)


def _lg(n: int) -> int:
    return n.bit_length() - 1


def _nth_element(p: _Pairs, nth: int) -> None:
    first, last = 0, p.k.size
    if first == last or nth == last:
        return
    depth = 2 * _lg(last - first)
    while last - first > 3:
        if depth == 0:
            _heap_select(p, first, nth + 1, last)
            p.swap(first, nth)
            return
        depth -= 1
        mid = first + (last - first) // 2
        _move_median_to_first(p, first, first + 1, mid, last - 1)
        cut = _partition(p, first, last)
        if cut <= nth:
            first = cut
        else:
            last = cut
    _insertion_sort(p, first, last)


def topk_row(v: np.ndarray, k: int) -> np.ndarray:
    """Indices torch.topk(v, k) keeps for a 1-D float32 v (as a set: the first k pairs)."""
    v = np.asarray(v, dtype=np.float32).ravel()
    n = v.size
    if k <= 0:
        return np.zeros(0, dtype=np.int64)
    if k >= n:
        return np.arange(n, dtype=np.int64)
    p = _Pairs(ordered_keys(v))
    if k * 64 <= n:
        _heap_select(p, 0, k, n)  # partial_sort: the set is fixed here, sort_heap only orders it
    else:
        _nth_element(p, k - 1)
    return p.i[:k].copy()


def topk_keep(v: np.ndarray, k: int) -> np.ndarray:
    """Boolean mask of the entries torch.topk(v, k, dim=-1) keeps, per row of the last axis."""
    v = np.asarray(v, dtype=np.float32)
    flat = v.reshape(-1, v.shape[-1]) if v.ndim > 0 else v.reshape(1, 1)
    keep = np.zeros(flat.shape, dtype=bool)
    for r in range(flat.shape[0]):
        keep[r, topk_row(flat[r], k)] = True
    return keep.reshape(v.shape)
