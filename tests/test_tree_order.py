"""The order in which the reduce kernel sums the 32 per-token maxima.

The reference sums them with a shuffle-down tree over 32 lanes
(kernels.cu:195-198: for o = 16, 8, 4, 2, 1, lane l += lane l + o), and
S_cand is compared bit for bit. The reduce kernel evaluates that tree in one
thread for documents of three or more tokens (`tree_sum32` in
kernels_candidates.hip): the leaves in bit-reversed order (position r holds
token rev5(r)) with one partial sum per level, i.e. a balanced pairwise sum.
These checks restate both evaluations in float32 and show that they agree
bit for bit on sparse and dense leaf sets, while a natural-order pairwise
sum (the plausible slip of forgetting the bit reversal) and a sequential sum
do not."""
import numpy as np


def shuffle_down_tree(x):
    v = x.astype(np.float32).copy()
    for o in (16, 8, 4, 2, 1):
        src = np.concatenate([v[o:], v[32 - o:]])  # lanes past the end read their own value
        v = (v + src).astype(np.float32)
    return v[0]


def rev5(r):
    return int(format(r, "05b")[::-1], 2)


def counter_tree(x):
    """tree_sum32's evaluation: leaf rev5(r) at position r, one partial sum per
    level, the left operand being the lower positions."""
    part = [None] * 5
    s = np.float32(0)
    for r in range(32):
        s = np.float32(x[rev5(r)])
        for k in range(5):
            if (r >> k) & 1 == 0:
                part[k] = s
                break
            s = np.float32(part[k] + s)
    return s


def natural_pairwise(x):
    v = list(x.astype(np.float32))
    while len(v) > 1:
        v = [np.float32(v[i] + v[i + 1]) for i in range(0, len(v), 2)]
    return v[0]


def sequential(x):
    s = np.float32(0)
    for t in x.astype(np.float32):
        s = np.float32(s + t)
    return s


def leaf_sets(n, seed):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        x = np.zeros(32, np.float32)
        k = int(rng.integers(1, 33))
        idx = rng.choice(32, k, replace=False)
        x[idx] = (rng.random(k) * 10.0 ** rng.uniform(-3, 3, k)).astype(np.float32)
        yield x


def bits(v):
    return np.float32(v).view(np.uint32)


def test_bit_reversed_pairwise_is_the_shuffle_down_tree():
    for x in leaf_sets(3000, 5):
        assert bits(counter_tree(x)) == bits(shuffle_down_tree(x))


def test_rev5_is_an_involution_on_five_bits():
    assert sorted(rev5(r) for r in range(32)) == list(range(32))
    assert all(rev5(rev5(r)) == r for r in range(32))
    assert [rev5(r) for r in (1, 2, 3, 16)] == [16, 8, 24, 1]


def test_other_orders_differ():
    wrong_pairwise = wrong_sequential = 0
    for x in leaf_sets(1000, 6):
        t = bits(shuffle_down_tree(x))
        wrong_pairwise += bits(natural_pairwise(x)) != t
        wrong_sequential += bits(sequential(x)) != t
    assert wrong_pairwise > 100 and wrong_sequential > 100
