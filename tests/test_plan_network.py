"""The plan kernel's two sorts, restated on the CPU.

Up to 8192 keys (in LDS): each 64-key chunk is ranked by counting, then sorted
runs are merged pairwise, a key moving to (start of the pair) + (its index in
its run) + (keys of the partner run below it, by binary lifting).  The
restatement applies the kernel's index formulas (run = 2^lg, partner base
((i >> lg) ^ 1) << lg, destination ((i >> lg) & ~1) * run + (i & (run - 1)) +
count) and checks that every round writes each position exactly once, reads
only indices below n, and ends sorted.

Above 8192 keys, csrc/qw_plan.hip sorts the keys of an expert with more than 8192 routes in
global memory with a bitonic network whose compare-exchanges all put the
smaller key first (mirror pairing in the first stage of each merge), skipping
every pair whose upper index is past the key count n instead of padding to a
power of two.  This restatement applies the kernel's exact index formulas,
stage by stage, and checks that the pairs of a stage are disjoint (so the
kernel's threads may apply them in any order) and that the result is sorted,
for key counts from just above the LDS limit to 64K.
"""

import numpy as np
import pytest


def network_stages(n: int):
    p2 = 1
    while p2 < n:
        p2 <<= 1
    i = np.arange(p2 // 2)
    size = 2
    while size <= p2:
        half = size >> 1
        blk, j = i // half, i % half
        yield blk * size + j, blk * size + size - 1 - j
        stride = half >> 1
        while stride > 0:
            lo = 2 * i - (i & (stride - 1))
            yield lo, lo + stride
            stride >>= 1
        size <<= 1


def run_network(keys: np.ndarray) -> np.ndarray:
    keys = keys.copy()
    n = len(keys)
    for lo, hi in network_stages(n):
        touched = np.concatenate([lo, hi])
        assert len(np.unique(touched)) == len(touched), "a stage touches an index twice"
        live = hi < n  # pairs past n compare against +infinity: nothing moves
        lo, hi = lo[live], hi[live]
        a, b = keys[lo], keys[hi]
        swap = a > b
        keys[lo[swap]], keys[hi[swap]] = b[swap], a[swap]
    return keys


@pytest.mark.parametrize("n", [8193, 9000, 12345, 16384, 16385, 20000, 40000, 65536])
def test_large_expert_network_sorts(n):
    rng = np.random.default_rng(n)
    # unique 64-bit keys shaped like the kernel's: (inverted weight order) << 32 | route id
    weights = rng.integers(0, 1 << 20, size=n, dtype=np.uint64)  # few distinct weights: many equal high halves
    routes = rng.permutation(n).astype(np.uint64)
    keys = (weights << np.uint64(32)) | routes
    assert np.array_equal(run_network(keys), np.sort(keys))


def test_network_on_sorted_and_reversed_inputs():
    for n in (8193, 10000):
        keys = np.arange(n, dtype=np.uint64) * np.uint64(3)
        assert np.array_equal(run_network(keys), keys)
        assert np.array_equal(run_network(keys[::-1].copy()), keys)


def lds_sort(keys: np.ndarray) -> np.ndarray:
    """The in-LDS path: 64-key chunk counting, then merge rounds (vectorised per round)."""
    n = len(keys)
    buf = np.empty(n, np.uint64)
    for base in range(0, n, 64):
        chunk = keys[base:base + 64]
        rank = (chunk[None, :] < chunk[:, None]).sum(axis=1)
        buf[base + rank] = chunk
    src, lg = buf, 6
    while (1 << lg) < n:
        run = 1 << lg
        i = np.arange(n)
        pb = ((i >> lg) ^ 1) << lg
        pe = np.minimum(pb + run, n)
        length = np.where(pb < n, pe - pb, 0)
        k = src[i]
        cnt = np.zeros(n, np.int64)
        step = run
        while step >= 1:  # binary lifting over the powers of two <= run
            j = cnt + step - 1
            inside = j < length
            idx = np.where(inside, pb + j, 0)
            assert idx.max() < n
            cnt = np.where(inside & (src[idx] < k), cnt + step, cnt)
            step >>= 1
        dst_pos = ((i >> lg) & ~1) * run + (i & (run - 1)) + cnt
        assert len(np.unique(dst_pos)) == n and dst_pos.max() < n, "a merge round writes a position twice"
        dst = np.empty(n, np.uint64)
        dst[dst_pos] = k
        src, lg = dst, lg + 1
    return src


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 127, 128, 129, 300, 1000, 1398, 2049, 4097, 8191, 8192])
def test_lds_sort_sorts(n):
    rng = np.random.default_rng(n + 7)
    weights = rng.integers(0, 1 << 10, size=n, dtype=np.uint64)  # many equal high halves
    routes = rng.permutation(n).astype(np.uint64)
    keys = (weights << np.uint64(32)) | routes
    assert np.array_equal(lds_sort(keys), np.sort(keys))
