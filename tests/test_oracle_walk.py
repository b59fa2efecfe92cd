"""The oracle's selector walk (crates/cuda/csrc/dflash2.cu:436-519) and its keyed choice (crates/cuda/csrc/keyed.cuh:
50-112), pinned by the known answers of crates/spec/src/lib.rs:391-493 (the CPU walk; on these exact small values the
kernel's 32-lane float sums equal the CPU's sequential ones) and by try_choose itself (pinned by the 5000 fixture
cases): keyed_choose over NaN-free candidates is try_choose with top_k = k."""
import numpy as np

from oracle import oracle as O

V = 64


def f16(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def codebook(fn, rank):
    return f16([fn(i) for i in range(V)]).reshape(V, rank)


def walk(anchor, cands, unary, hidden, pred, succ, sampling=None):
    rank = len(hidden[0])
    ids = np.array(cands, dtype=np.int32)
    vals = np.array(unary, dtype=np.float32)
    gate = np.array(hidden, dtype=np.float32)
    out, conf, margin = O.selector_walk([anchor], ids, vals, gate, True, codebook(pred, rank), codebook(succ, rank), 1, len(cands),
                                        sampling)
    return list(out)


def keyed(T, first_position=0, top_p=1.0, min_p=0.0, seed=0):
    s = np.zeros(1, dtype=O.WALK_SAMPLING_DTYPE)
    s[0] = (seed, first_position, T, top_p, min_p, 1, 0)
    return s


def test_known_answers_of_the_reference_walk():
    z2 = lambda i: [0.0, 0.0]  # noqa: E731
    # selector_greedy_and_keyed
    assert walk(1, [[10, 11], [20, 21]], [[0.0, 1.0], [2.0, 0.0]], [[1.0, 1.0], [1.0, 1.0]], z2, z2) == [11, 20]
    assert walk(1, [[10, 11], [20, 21]], [[0.0, 1.0], [2.0, 0.0]], [[1.0, 1.0], [1.0, 1.0]], z2, z2, keyed(1e-6, 5)) == [11, 20]
    # selector_bilinear_term_can_flip_choice: 0 + 2 beats 0.5
    assert walk(3, [[10, 11]], [[0.0, 0.5]], [[1.0, 1.0]], lambda i: [1.0, 1.0], lambda i: [1.0, 1.0] if i == 10 else [0.0, 0.0]) == [10]
    # selector_depends_on_the_previous_token
    pred = lambda i: [1.0] if i == 1 else [-1.0]  # noqa: E731
    succ = lambda i: [1.0] if i == 10 else [0.0]  # noqa: E731
    assert walk(2, [[1, 2], [10, 11]], [[1.0, 0.0], [0.0, 0.0]], [[1.0], [1.0]], pred, succ) == [1, 10]
    assert walk(1, [[1, 2], [10, 11]], [[0.0, 1.0], [0.0, 0.0]], [[1.0], [1.0]], pred, succ) == [2, 11]
    # greedy_walk_breaks_ties_to_the_lowest_id: the keyed choice at temperature 0 orders ties by id (12); the device
    # kernel's unkeyed argmax keeps the first maximum (30), a difference of the reference's own two walks
    assert walk(1, [[30, 12, 20]], [[1.0, 1.0, 0.5]], [[0.0, 0.0]], z2, z2, keyed(0.0)) == [12]
    assert walk(1, [[30, 12, 20]], [[1.0, 1.0, 0.5]], [[0.0, 0.0]], z2, z2) == [30]


def test_keyed_choose_is_try_choose_over_all_candidates():
    rng = np.random.default_rng(4)
    for case in range(3000):
        k = int(rng.integers(1, 65))
        scores = (rng.standard_normal(k) * rng.choice([0.1, 1.0, 5.0])).astype(np.float32)
        if case % 5 == 0:
            scores = np.round(scores).astype(np.float32)  # ties
        ids = rng.permutation(1000)[:k].astype(np.int32)
        T = float(rng.choice([0.0, 0.3, 0.8, 1.0, 1.7]))
        top_p = float(rng.choice([1.0, 0.9, 0.5, 0.0]))
        min_p = float(rng.choice([0.0, 0.05, 0.3]))
        seed, pos = int(rng.integers(1 << 62)), int(rng.integers(1 << 30))
        i, _ = O.keyed_choose(scores, ids, seed, T, top_p, min_p, pos)
        s = O.Sampling(seed=seed, temperature=T, top_k=k, top_p=top_p, min_p=min_p)
        st, want = O.try_choose(scores, ids.astype(np.uint32), pos, s)
        assert st == O.ROW_OK and int(ids[i]) == want, case


def test_margins_and_nan_order():
    # margin at temperature 0: the score gap to the runner-up; one candidate: 30
    i, m = O.keyed_choose([3.0, 1.0, 2.5], [5, 6, 7], 0, 0.0, 1.0, 0.0, 0)
    assert i == 0 and abs(m - 0.5) < 1e-7
    assert O.keyed_choose([3.0], [5], 0, 0.7, 1.0, 0.0, 0)[1] == 30.0
    # NaN scores sort last: never chosen while a number is there, chosen when every score is NaN
    assert O.keyed_choose([np.nan, 1.0, np.nan], [1, 2, 3], 0, 0.0, 1.0, 0.0, 0)[0] == 1
    assert O.keyed_choose([np.nan, np.nan], [9, 4], 0, 0.0, 1.0, 0.0, 0)[0] in (0, 1)
