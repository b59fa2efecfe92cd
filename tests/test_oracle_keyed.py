"""The CPU oracle's Mode K half against REXL3's own fixtures and known answers.

Pins: testdata/fixtures/sampling.json (copied to tests/golden/sampling.json) as read by crates/sampling/tests/xcheck.rs,
the unit tests of crates/sampling/src/lib.rs:307-462, crates/sampling/tests/coupling.rs, crates/spec/src/lib.rs:309-314.
"""
import hashlib
import json
import math
import os
import struct

import numpy as np
import pytest

from oracle import oracle as O
from tests.common import Rng, fnv

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
FIX = json.load(open(os.path.join(GOLDEN, "sampling.json")))

TEMPS = [0.0, 0.3, 0.6, 1.0, 1.5]
TOPK = [0, 1, 5, 20]
TOPP = [1.0, 0.95, 0.8, 0.5, 0.0]
MINP = [0.0, 0.0, 0.05, 0.2]


def xcheck_case(i: int):
    """crates/sampling/tests/xcheck.rs:38-59."""
    r = Rng(1000 + i)
    n = 1 + r.next() % 28
    mode = r.next() % 3
    vals = []
    for _ in range(n):
        x = r.next()
        base = np.float32(np.float32(np.float32(x >> 40) / np.float32(16777216.0)) * np.float32(16.0)) - np.float32(8.0)
        base = np.float32(base)
        if mode == 0:
            vals.append(base)
        elif mode == 1:
            vals.append(np.float32(x >> 61))
        else:
            vals.append(np.float32(base * np.float32(3.0)))
    ids = [(j * 5003 + r.next() % 5003) for j in range(n)]
    temperature = TEMPS[r.next() % 5]
    top_k = TOPK[r.next() % 4]
    top_p = TOPP[r.next() % 5]
    min_p = MINP[r.next() % 4]
    seed = r.next() >> 1
    position = r.next() % 300000
    return (np.array(vals, dtype=np.float32), np.array(ids, dtype=np.uint32), position,
            O.Sampling(seed, temperature, top_k, top_p, min_p))


def all_cases():
    return [xcheck_case(i) for i in range(FIX["cases"])]


def test_uniform_bits_match_fixture():
    """crates/sampling/tests/xcheck.rs:61-73."""
    buf = bytearray()
    for seed in [0, 1, (1 << 63) - 1, 123456789]:
        for pos in range(32):
            for tid in range(32):
                buf += struct.pack("<d", O.uniform(seed, pos, tid))
    assert fnv(bytes(buf)) == FIX["uniform_fnv"]


def test_seed_for_matches_fixture():
    """crates/sampling/tests/xcheck.rs:75-82."""
    for e in FIX["seed_for"]:
        assert O.seed_for(e["tokens"], e["salt"]) == e["seed"]


def test_seed_for_is_sha256_of_the_string_form():
    """crates/sampling/src/lib.rs:421-432, with hashlib as the independent SHA-256."""
    tokens = [0, 7, 4294967295, 12, 100]
    for salt in [0, 9, (1 << 64) - 1]:
        s = ",".join(str(t) for t in tokens) + "|" + str(salt)
        d = hashlib.sha256(s.encode()).digest()
        assert O.seed_for(tokens, salt) == int.from_bytes(d[:8], "little") & ((1 << 63) - 1)
        assert O.sha256(s.encode()) == d
    d = hashlib.sha256(b"|5").digest()
    assert O.seed_for([], 5) == int.from_bytes(d[:8], "little") & ((1 << 63) - 1)
    for n in [0, 55, 56, 63, 64, 65, 119, 120, 1000]:
        data = bytes((i * 7 + 3) & 0xFF for i in range(n))
        assert O.sha256(data) == hashlib.sha256(data).digest()


def test_choose_matches_fixture_and_inputs_are_the_same():
    """crates/sampling/tests/xcheck.rs:84-125: all 5000 cases, temperature-0 exact ties checked as lowest id."""
    expected = FIX["choose"]
    inp = bytearray()
    mism = []
    greedy_ties = 0
    for i, (vals, ids, pos, s) in enumerate(all_cases()):
        inp += vals.tobytes() + ids.tobytes() + struct.pack("<QQ", pos, s.seed)
        st, got = O.try_choose(vals, ids, pos, s)
        assert st == O.ROW_OK
        top = vals.max()
        tied = [int(t) for t, v in zip(ids, vals) if v == top]
        if s.temperature == 0.0 and len(tied) > 1:
            assert got == min(tied)
            greedy_ties += 1
            continue
        if got != expected[i]:
            mism.append(i)
    assert fnv(bytes(inp)) == FIX["inputs_fnv"], "case generation differs from the fixture's"
    assert not mism, f"{len(mism)} of {FIX['cases']} differ: {mism[:20]}"
    assert greedy_ties > 0


def test_unit_open_edges():
    """crates/sampling/src/lib.rs:391-398."""
    assert O.unit_open(0) > 0.0
    assert O.unit_open((1 << 64) - 1) < 1.0
    assert O.unit_open((1 << 64) - 1 - 0x7FF) < 1.0
    assert math.isfinite(math.log(-math.log(O.unit_open((1 << 64) - 1))))
    assert O.unit_open(0) == 2.0 ** -54
    for p in range(1000):
        u = O.uniform(7, p, p * 31)
        assert 0.0 < u < 1.0


def test_pairwise_sum_closed_forms():
    """crates/sampling/src/lib.rs:440-444, and numpy's own pairwise sum on awkward lengths."""
    assert O.pairwise_sum(np.arange(300, dtype=np.float64)) == sum(range(300))
    rng = np.random.default_rng(5)
    for n in [0, 1, 7, 8, 9, 15, 16, 127, 128, 129, 255, 256, 257, 1000, 4099]:
        a = rng.standard_normal(n) * 10.0 ** rng.integers(-5, 5, n)
        assert O.pairwise_sum(a) == np.add.reduce(a), n


def s(**kw):
    d = dict(seed=0, temperature=1.0, top_k=20, top_p=0.95, min_p=0.0)
    d.update(kw)
    return O.Sampling(d["seed"], d["temperature"], d["top_k"], d["top_p"], d["min_p"])


def test_unit_known_answers():
    """crates/sampling/src/lib.rs:311-389 and crates/sampling/tests/coupling.rs."""
    # ties resolve by id before noise
    for p in range(200):
        assert O.try_choose([1.0] * 5, [9, 3, 1, 2, 7], p, s(top_k=3, top_p=1.0))[1] in (1, 2, 3)
    # candidate order is irrelevant
    vals, ids = [0.3, 2.0, -1.0, 2.0, 0.9], [4, 8, 1, 2, 6]
    for p in range(100):
        assert O.try_choose(vals, ids, p, s(seed=99)) == O.try_choose(vals[::-1], ids[::-1], p, s(seed=99))
    for p in range(100):
        assert O.try_choose([0.1, 5.0, 4.9, -2.0], [0, 1, 2, 3], p, s(temperature=0.0))[1] == 1
    for p in range(200):
        assert O.try_choose([1.0, 3.0, 3.0, 3.0, 0.0], [10, 7, 4, 9, 1], p, s(seed=p * 3, temperature=0.0, top_k=0))[1] == 4
    assert O.try_choose([-0.0, 0.0], [9, 2], 0, s(temperature=0.0, top_k=0))[1] == 2
    # errors
    assert O.try_choose([], [], 0, s())[0] == O.ROW_NO_CANDIDATES
    assert O.try_choose([1.0], [1, 2], 0, s())[0] == "LengthMismatch"
    assert O.try_choose([1.0, float("nan")], [1, 2], 0, s())[0] == O.ROW_NAN_LOGIT
    for bad in [s(min_p=1.5), s(min_p=math.inf), s(min_p=-0.1), s(top_p=1.5), s(top_p=math.nan), s(temperature=-1.0),
                s(temperature=math.nan), s(temperature=math.inf)]:
        assert O.try_choose([1.0, 2.0], [1, 2], 0, bad)[0] == O.ROW_INVALID_PARAMS
    assert O.try_top_candidates([0.0, float("nan")], 1)[0] == O.ROW_NAN_LOGIT
    assert O.try_choose([1.0, 2.0, 0.5], [1, 2, 3], 0, s(min_p=1.0)) == (O.ROW_OK, 2)
    # coupling: greedy has no noise; the same token draws the same noise across rows
    for position in range(64):
        for seed in [0, 7, 12345, ((1 << 64) - 1) >> 1]:
            assert O.try_choose([0.3, 2.0, -1.0, 2.0, 0.9], [4, 8, 1, 2, 6], position,
                                s(seed=seed, temperature=0.0, top_k=0, top_p=0.0))[1] == 2
    for position in [3, 1000, 123_456_789]:
        t = s(seed=7, top_k=4, top_p=1.0)
        assert O.try_choose([0.1, 0.2, 0.3, 0.4], [10, 20, 30, 40], position, t) == \
            O.try_choose([0.4, 0.3, 0.2, 0.1], [40, 30, 20, 10], position, t)


def test_keyed_draw_is_the_gumbel_argmax_restated_in_python():
    """Independent restatement: argmax of v/T + (-ln(-ln u)) over the kept prefix, with math.exp/math.log and the
    fixture-pinned uniform; top_p by numpy cumsum over probs normalised by numpy's pairwise sum."""
    rng = np.random.default_rng(11)
    for trial in range(400):
        n = int(rng.integers(1, 40))
        vals = (rng.standard_normal(n) * 2).astype(np.float32)
        ids = rng.choice(100000, size=n, replace=False).astype(np.uint32)
        T = float(rng.choice([0.3, 0.7, 1.0, 1.3]))
        k = int(rng.choice([0, 1, 5, 20]))
        tp = float(rng.choice([1.0, 0.9, 0.5]))
        mp = float(rng.choice([0.0, 0.05, 0.2]))
        seed, pos = int(rng.integers(0, 2**62)), int(rng.integers(0, 10**6))
        order = sorted(range(n), key=lambda i: (-float(vals[i]), int(ids[i])))
        kk = min(k, n) if k > 0 else n
        sc = np.array([float(vals[i]) / T for i in order[:kk]])
        keep = kk
        if 0 < tp < 1:
            pr = np.exp(sc - sc.max())
            pr = pr / np.add.reduce(pr)
            c = np.cumsum(pr)
            keep = min(int(np.sum(c < tp)) + 1, kk)
        if mp > 0:
            fl = sc[0] + math.log(mp)
            keep = max(1, int(np.sum(sc[:keep] >= fl)))
        best, bs = 0, -math.inf
        for j in range(keep):
            u = O.uniform(seed, pos, int(ids[order[j]]))
            sco = sc[j] + (-math.log(-math.log(u)))
            if sco > bs:
                bs, best = sco, j
        want = int(ids[order[best]])
        assert O.try_choose(vals, ids, pos, s(seed=seed, temperature=T, top_k=k, top_p=tp, min_p=mp))[1] == want


def test_top_candidates_matches_a_full_sort():
    """crates/sampling/src/lib.rs:400-419."""
    r = 12345
    for n in [1, 2, 7, 50, 300]:
        logits = []
        for _ in range(n):
            r = (r * 6364136223846793005 + 1442695040888963407) & ((1 << 64) - 1)
            logits.append(float(r >> 60) - 8.0)
        full = sorted(range(n), key=lambda i: (-logits[i], i))
        for count in [0, 1, 5, n, n + 3]:
            st, ids, vals = O.try_top_candidates(logits, count)
            take = min(count, n)
            assert st == 0
            assert list(ids) == full[:take]
            assert list(vals) == [logits[i] for i in full[:take]]


def test_accept_known_answers():
    """crates/spec/src/lib.rs:309-314 and the tree walk of crates/spec/src/tree.rs:417-438."""
    assert O.accept([1, 2, 3], [1, 2, 4, 9]) == 2
    assert O.accept([5], [6, 1]) == 0
    assert O.accept([], [6]) == 0
    # tree: root 0 -> children 1 (tok 5), 2 (tok 7); 1 -> 3 (tok 9); 2 -> 4 (tok 9)
    tokens = [0, 5, 7, 9, 9]
    parents = [-1, 0, 0, 1, 2]
    assert O.accept_tree(tokens, parents, [7, 0, 9, 0, 0]) == [0, 2, 4]
    assert O.accept_tree(tokens, parents, [5, 9, 0, 1, 0]) == [0, 1, 3]
    assert O.accept_tree(tokens, parents, [6, 9, 9, 0, 0]) == [0]
    # duplicate tokens among children: the first such row wins
    assert O.accept_tree([0, 5, 5], [-1, 0, 0], [5, 1, 1]) == [0, 1]


def test_keyed_pick_matches_golden_hashes():
    """testdata/gpu/golden_glm_keyed.txt (generator crates/cuda/tests/glm_keyed.rs:266-296): the oracle's keyed pick
    reproduces every one of the 84 (ids, vals) hashes the reference's device kernel wrote."""
    from tests.golden_glm import golden_case, golden_lines
    lines = golden_lines(os.path.join(GOLDEN, "golden_glm_keyed.txt"))
    assert len(lines) == 84
    for count, rows, depth, hid, hval in lines:
        ids, vals, recs = golden_case(count, rows, depth, O.KEYED_ROW_DTYPE)
        oi, ov = O.keyed_pick_rows(ids, vals, recs, depth)
        assert fnv(oi.astype("<i4").tobytes()) == hid, (count, rows, depth)
        assert fnv(ov.astype("<f4").tobytes()) == hval, (count, rows, depth)
