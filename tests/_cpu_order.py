"""Models of two CPU orders the reference's results depend on (test infrastructure).

* ``column_sum_model(sq)`` -- the summation order of torch's CPU ``t.sum(0)`` over a row-major
  [n, C] fp32 tensor, which ``act_square.add_((inp ** 2).sum(0))`` runs
  (gptq_utils/gptq_plus_utils.py:856).  Columns [0, 32 floor(C/32)) are each one four-level
  cascade over the n rows (level power p = max(4, ceil(log2 n) // 4), blocks of 2^p); the
  remaining columns are four interleaved cascades over rows m, m + 4, ... plus the n mod 4
  leftover rows, combined as ((s0 + s1) + s2) + s3.  (For C mod 32 in [4, 8) torch reduces the
  first four of those columns with the plain cascade for some n; the model does not cover them.)
* ``std_sort(keys)`` -- libstdc++'s ``std::sort`` (introsort: median of three, unguarded Hoare
  partition, depth budget 2 floor(log2 n) then heap sort, final insertion sort at 16) over
  (key, index) pairs with torch's descending comparator, which is what
  ``torch.argsort(x, descending=True)`` returns on CPU (gptq_plus_utils.py:1046), ties included.
* ``adversarial_keys(n)`` -- McIlroy's adversary against that sort: keys that exhaust its depth
  budget, so the heap-sort branch runs.

The tests check both models against torch itself, so they pin the orders the HIP kernels follow.
"""
from __future__ import annotations

import math

import numpy as np


def _ceil_log2(n):
    return 0 if n <= 1 else int(math.ceil(math.log2(n)))


def cascade(x):
    """Four-level cascade sum over axis 0 of a float32 array (any trailing shape)."""
    n = x.shape[0]
    lp = max(4, _ceil_log2(n) // 4)
    step = 1 << lp
    mask = step - 1
    acc = [np.zeros(x.shape[1:], np.float32) for _ in range(4)]
    i = 0
    while i + step <= n:
        for _ in range(step):
            acc[0] = (acc[0] + x[i]).astype(np.float32)
            i += 1
        for j in range(1, 4):
            acc[j] = (acc[j] + acc[j - 1]).astype(np.float32)
            acc[j - 1] = np.zeros_like(acc[j - 1])
            if (i & (mask << (j * lp))) != 0:
                break
    while i < n:
        acc[0] = (acc[0] + x[i]).astype(np.float32)
        i += 1
    for j in range(1, 4):
        acc[0] = (acc[0] + acc[j]).astype(np.float32)
    return acc[0]


def interleaved_sum(col):
    """Four interleaved cascades over one column, leftover rows into the first, then combined."""
    n = col.shape[0]
    k = n // 4
    p = cascade(col[:4 * k].reshape(k, 4)).copy() if k > 0 else np.zeros(4, np.float32)
    for i in range(4 * k, n):
        p[0] = np.float32(p[0] + col[i])
    for j in range(1, 4):
        p[0] = np.float32(p[0] + p[j])
    return p[0]


def column_sum_model(sq):
    sq = np.asarray(sq, dtype=np.float32)
    n, C = sq.shape
    out = np.zeros(C, np.float32)
    ca = (C // 32) * 32
    if ca:
        out[:ca] = cascade(sq[:, :ca])
    for c in range(ca, C):
        out[c] = interleaved_sum(sq[:, c])
    return out


def model_covers(C):
    """Whether column_sum_model claims torch's order for every column of width C."""
    return not (4 <= C % 32 < 8)


# ---------------------------------------------------------------------------------------------
# libstdc++ std::sort on (key, index) pairs, descending comparator with NaN first

def _before(a, b):
    return (math.isnan(a[0]) and not math.isnan(b[0])) or (a[0] > b[0])


class _Sorter:
    def __init__(self, comp=_before):
        self.comp = comp
        self.heap_calls = 0

    def median_to_first(self, A, result, a, b, c):
        cp = self.comp
        if cp(A[a], A[b]):
            if cp(A[b], A[c]):
                A[result], A[b] = A[b], A[result]
            elif cp(A[a], A[c]):
                A[result], A[c] = A[c], A[result]
            else:
                A[result], A[a] = A[a], A[result]
        elif cp(A[a], A[c]):
            A[result], A[a] = A[a], A[result]
        elif cp(A[b], A[c]):
            A[result], A[c] = A[c], A[result]
        else:
            A[result], A[b] = A[b], A[result]

    def partition(self, A, first, last, pivot):
        cp = self.comp
        while True:
            while cp(A[first], A[pivot]):
                first += 1
            last -= 1
            while cp(A[pivot], A[last]):
                last -= 1
            if not first < last:
                return first
            A[first], A[last] = A[last], A[first]
            first += 1

    def push_heap(self, A, first, hole, top, value):
        parent = (hole - 1) // 2
        while hole > top and self.comp(A[first + parent], value):
            A[first + hole] = A[first + parent]
            hole = parent
            parent = (hole - 1) // 2
        A[first + hole] = value

    def adjust_heap(self, A, first, hole, ln, value):
        top = hole
        second = hole
        while second < (ln - 1) // 2:
            second = 2 * (second + 1)
            if self.comp(A[first + second], A[first + second - 1]):
                second -= 1
            A[first + hole] = A[first + second]
            hole = second
        if (ln & 1) == 0 and second == (ln - 2) // 2:
            second = 2 * (second + 1)
            A[first + hole] = A[first + second - 1]
            hole = second - 1
        self.push_heap(A, first, hole, top, value)

    def heap_sort(self, A, first, last):
        self.heap_calls += 1
        ln = last - first
        if ln >= 2:
            parent = (ln - 2) // 2
            while True:
                self.adjust_heap(A, first, parent, ln, A[first + parent])
                if parent == 0:
                    break
                parent -= 1
        while last - first > 1:
            last -= 1
            value = A[last]
            A[last] = A[first]
            self.adjust_heap(A, first, 0, last - first, value)

    def introsort(self, A, first, last, depth):
        stack = [(first, last, depth)]
        while stack:
            first, last, depth = stack.pop()
            while last - first > 16:
                if depth == 0:
                    self.heap_sort(A, first, last)
                    break
                depth -= 1
                mid = first + (last - first) // 2
                self.median_to_first(A, first, first + 1, mid, last - 1)
                cut = self.partition(A, first + 1, last, first)
                stack.append((cut, last, depth))
                last = cut

    def insertion_sort(self, A):
        cp = self.comp
        for i in range(1, len(A)):
            val = A[i]
            j = i
            while j > 0 and cp(val, A[j - 1]):
                A[j] = A[j - 1]
                j -= 1
            A[j] = val

    def sort(self, A):
        n = len(A)
        if n > 1:
            self.introsort(A, 0, n, 2 * int(math.floor(math.log2(n))))
            self.insertion_sort(A)
        return A


def std_sort(keys):
    """Indices in the order torch.argsort(keys, descending=True) returns on CPU."""
    keys = np.asarray(keys, dtype=np.float32)
    A = [(float(keys[i]), i) for i in range(keys.shape[0])]
    _Sorter().sort(A)
    return np.array([a[1] for a in A], dtype=np.int64)


def adversarial_keys(n):
    """McIlroy's adversary: freezes values lazily so each median-of-three pivot lands near an
    end; returns float32 keys (distinct) that drive the sort into its heap-sort branch."""
    gas = n + 1
    val = [gas] * n
    st = {"solid": 0, "cand": 0}

    def comp(a, b):
        ia, ib = a[1], b[1]
        if val[ia] == gas and val[ib] == gas:
            if ia == st["cand"]:
                val[ia] = st["solid"]
            else:
                val[ib] = st["solid"]
            st["solid"] += 1
        if val[ia] == gas:
            st["cand"] = ia
        elif val[ib] == gas:
            st["cand"] = ib
        return val[ia] < val[ib]

    _Sorter(comp).sort([(0.0, i) for i in range(n)])
    return np.array([float(n + 2 - v) for v in val], np.float32)


def heap_sort_runs(keys):
    keys = np.asarray(keys, dtype=np.float32)
    s = _Sorter()
    s.sort([(float(keys[i]), i) for i in range(keys.shape[0])])
    return s.heap_calls
