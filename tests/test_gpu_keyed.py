"""The keyed sampler on the GPU: gb_glm_keyed_pick against the reference's golden hashes and the oracle's try_choose,
the fused gbs_keyed_sample_rows against the oracle's top-(k+8) + try_choose, and the accept steps.
Follows crates/cuda/tests/glm_keyed.rs:94-296 and crates/cuda/tests/glue.rs:1213-1250."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from rexl3_amd import sampling as S
from rexl3_amd import workloads as W
from tests.common import Rng, fnv
from tests.golden_glm import candidates, golden_case, golden_lines, settings
from tests.gpu_util import dev, host, log, need_gpu

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_device_keyed_pick_reproduces_the_golden_hashes():
    """testdata/gpu/golden_glm_keyed.txt: all 84 (ids, vals) hashes of the reference's device keyed pick."""
    need_gpu()
    for count, rows, depth, hid, hval in golden_lines(os.path.join(GOLDEN, "golden_glm_keyed.txt")):
        ids, vals, recs = golden_case(count, rows, depth, S.KEYED_ROW_DTYPE)
        oi, ov = S.keyed_pick(dev(ids), dev(vals), recs, depth)
        oi, ov = host(oi), host(ov)
        assert fnv(oi.astype("<i4").tobytes()) == hid, (count, rows, depth)
        assert fnv(ov.astype("<f4").tobytes()) == hval, (count, rows, depth)


def test_device_keyed_pick_is_try_choose_on_the_same_candidates():
    """crates/cuda/tests/glm_keyed.rs:94-139: 0 mismatches allowed."""
    need_gpu()
    rng = Rng(0x6B657965)
    checked = 0
    for count in [8, 28, 32, 48, 64]:
        for depth in [0, 1, 2, 3]:
            n = 200
            lists, recs = [], np.zeros(n, dtype=S.KEYED_ROW_DTYPE)
            for r in range(n):
                lists.append(candidates(rng, count))
                s = settings(rng, count)
                p = rng.next() % 6000
                recs[r] = (s["seed"], p, s["temperature"], s["top_p"], s["min_p"], s["top_k"], int(r % 5 != 0))
            ids = np.array([l[0] for l in lists], dtype=np.int32)
            vals = np.array([l[1] for l in lists], dtype=np.float32)
            gi, gv = S.keyed_pick(dev(ids), dev(vals), recs, depth)
            wi, wv = O.keyed_pick_rows(ids, vals, recs, depth)
            gi, gv = host(gi), host(gv)
            mism = np.nonzero(gi != wi)[0]
            assert mism.size == 0, f"count {count} depth {depth}: rows {mism[:10]}"
            assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32))
            checked += n
    log(f"{checked} rows, 0 mismatches")


def test_device_keyed_pick_over_the_5000_fixture_cases():
    """tests/golden/sampling.json (testdata/fixtures/sampling.json): every case as a device row, candidates sorted."""
    need_gpu()
    from tests.test_oracle_keyed import FIX, all_cases
    cases = all_cases()
    count = 28
    ids = np.zeros((len(cases), count), dtype=np.int32)
    vals = np.full((len(cases), count), -np.inf, dtype=np.float32)
    recs = np.zeros(len(cases), dtype=S.KEYED_ROW_DTYPE)
    ns = []
    for i, (v, d, pos, s) in enumerate(cases):
        order = sorted(range(len(v)), key=lambda j: (-float(v[j]), int(d[j])))
        n = len(v)
        ns.append(n)
        ids[i, :n] = d[order]
        vals[i, :n] = v[order]
        # pad with ids no case uses, below every value: only reachable through top_k 0 = "all", so pad by -inf and
        # restrict k to n through top_k when top_k is 0
        ids[i, n:] = 1_000_000 + np.arange(count - n)
        recs[i] = (s.seed, pos, s.temperature, s.top_p, s.min_p, s.top_k if s.top_k > 0 else n, 1)
    # rows of different n: run per n so that `count` equals the row's candidate number
    got = np.zeros(len(cases), dtype=np.int64)
    for n in sorted(set(ns)):
        rows = [i for i in range(len(cases)) if ns[i] == n]
        gi, _ = S.keyed_pick(dev(ids[rows, :n]), dev(vals[rows, :n]), recs[rows], 0)
        got[rows] = host(gi)
    expected = FIX["choose"]
    mism = []
    for i, (v, d, pos, s) in enumerate(cases):
        top = v.max()
        tied = [int(t) for t, x in zip(d, v) if x == top]
        want = min(tied) if (s.temperature == 0.0 and len(tied) > 1) else expected[i]
        if got[i] != want:
            mism.append(i)
    assert not mism, f"{len(mism)} mismatches: {mism[:10]}"


def test_fused_keyed_sampler_matches_topk_plus_try_choose():
    need_gpu()
    rng = np.random.default_rng(77)
    for dtype, rows, vocab in [(O.DTYPE_F32, 1, 151936), (O.DTYPE_F32, 37, 151936), (O.DTYPE_BF16, 64, 151936),
                               (O.DTYPE_F16, 9, 50000), (O.DTYPE_F32, 5, 100), (O.DTYPE_BF16, 3, 70)]:
        x = W.peaked_logits(int(rng.integers(1 << 30)), rows, vocab, 2.0, (4, 16), 6.0, 14.0)
        if dtype == O.DTYPE_BF16:
            data = W.to_bf16_bits(x)
            t = dev(data, torch.bfloat16)
        elif dtype == O.DTYPE_F16:
            data = x.astype(np.float16).view(np.uint16)
            t = dev(data, torch.float16)
        else:
            data = x
            t = dev(data)
        recs = np.zeros(rows, dtype=S.KEYED_ROW_DTYPE)
        for r in range(rows):
            recs[r] = (int(rng.integers(1 << 62)), int(rng.integers(1 << 20)), float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5])),
                       float(rng.choice([1.0, 0.95, 0.8, 0.5, 0.0])), float(rng.choice([0.0, 0.05, 0.2])),
                       int(rng.choice([1, 5, 20, 40, 56])), 1)
        depth = int(rng.integers(0, 4))
        log(f"fused keyed dtype={dtype} rows={rows} vocab={vocab}")
        gi, gs, gv = S.keyed_sample_rows(t, recs, depth, out_vals=True)
        wi, wv, ws = O.keyed_sample_rows(data, dtype, vocab, recs, depth)
        gi, gs, gv = host(gi), host(gs), host(gv)
        assert np.array_equal(gs, ws)
        assert np.array_equal(gi, wi), np.nonzero(gi != wi)[0][:10]
        assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32))


def test_fused_keyed_sampler_nan_and_invalid_rows():
    need_gpu()
    vocab = 4096
    x = np.random.default_rng(3).uniform(-3, 3, (6, vocab)).astype(np.float32)
    x[1, :4090] = np.nan  # 6 numbers left: fewer than top_k + 8 = 13 -> a NaN is a candidate
    x[2, 17] = np.nan     # one NaN: never a candidate
    recs = np.zeros(6, dtype=S.KEYED_ROW_DTYPE)
    for r in range(6):
        recs[r] = (r, 100, 1.0, 0.9, 0.0, 5, 1)
    recs[3]["top_k"] = 0
    recs[4]["temperature"] = -1.0
    recs[5]["top_p"] = 1.5
    gi, gs, _ = S.keyed_sample_rows(dev(x), recs, 0)
    wi, _, ws = O.keyed_sample_rows(x, O.DTYPE_F32, vocab, recs, 0)
    assert list(host(gs)) == list(ws) == [0, 2, 0, 3, 3, 3]
    assert np.array_equal(host(gi), wi)


def test_fused_keyed_rows_are_invariant():
    need_gpu()
    rng = np.random.default_rng(13)
    vocab = 151936
    x = (rng.integers(0, 40, (6, vocab)) * 0.5).astype(np.float32)  # many exact ties
    recs = np.zeros(6, dtype=S.KEYED_ROW_DTYPE)
    for r in range(6):
        recs[r] = (99, 1000 + r, 0.8, 0.9, 0.05, 20, 1)
    all_ids, _, _ = S.keyed_sample_rows(dev(x), recs, 1)
    all_ids = host(all_ids)
    for r in [0, 3, 5]:
        one, _, _ = S.keyed_sample_rows(dev(x[r:r + 1]), recs[r:r + 1], 1)
        assert host(one)[0] == all_ids[r]
    rev, _, _ = S.keyed_sample_rows(dev(x[::-1].copy()), recs[::-1].copy(), 1)
    assert np.array_equal(host(rev)[::-1], all_ids)


def test_choose_rows_api():
    need_gpu()
    x = np.random.default_rng(5).standard_normal((4, 1000)).astype(np.float32)
    s = S.Sampling(seed=7, temperature=0.9, top_k=20, top_p=0.9, min_p=0.0)
    got = S.choose_rows(dev(x), [10, 11, 12, 13], s)
    for r in range(4):
        _, cid, cv = O.try_top_candidates(x[r], 28)
        st, want = O.try_choose(cv, cid, 10 + r, O.Sampling(7, 0.9, 20, 0.9, 0.0))
        assert got[r] == want
    with pytest.raises(S.SamplingError):
        S.choose_rows(dev(x), [1, 2], s)


def test_greedy_gather_and_accept_steps():
    need_gpu()
    ids = np.arange(12, dtype=np.int32).reshape(3, 4)
    vals = np.array([[3, 2, 1, 0], [5, np.nan, 1, 0], [1, 1, 1, 1]], dtype=np.float32)
    oi, ov = S.greedy_gather(dev(ids), dev(vals))
    assert list(host(oi)) == [0, 4, 8]
    ov = host(ov)
    assert ov[0] == 3 and np.isnan(ov[1]) and ov[2] == 1
    rng = np.random.default_rng(8)
    n_seq, width = 300, 7
    samples = rng.integers(0, 4, (n_seq, width + 1)).astype(np.int32)
    drafts = samples[:, :width].copy()
    cut = rng.integers(0, width + 1, n_seq)
    for s in range(n_seq):
        if cut[s] < width:
            drafts[s, cut[s]] += 1
    acc = host(S.accept(dev(drafts), dev(samples)))
    for s in range(n_seq):
        assert acc[s] == O.accept(drafts[s], samples[s])
    # trees
    nodes = 12
    toks = rng.integers(0, 3, (50, nodes)).astype(np.int32)
    parents = np.zeros((50, nodes), dtype=np.int32)
    for t in range(50):
        parents[t, 0] = -1
        for r in range(1, nodes):
            parents[t, r] = rng.integers(0, r)
    smp = rng.integers(0, 3, (50, nodes)).astype(np.int32)
    path, plen = S.accept_tree(dev(toks), dev(parents), dev(smp))
    path, plen = host(path), host(plen)
    for t in range(50):
        want = O.accept_tree(toks[t], parents[t], smp[t])
        assert list(path[t, :plen[t]]) == want
        assert (path[t, plen[t]:] == -1).all()


def test_fused_keyed_workspace_reused_across_row_counts():
    """One workspace serves launches of different row counts (the arrival counters sit at fixed per-row offsets)."""
    need_gpu()
    vocab = 20_000
    shapes = [300, 2, 300, 64, 300]
    for i, rows in enumerate(shapes):
        x = W.peaked_logits(500 + i, rows, vocab, 2.0, (4, 16), 6.0, 14.0)
        recs = S.keyed_rows([S.Sampling(seed=5 + i, temperature=0.9, top_k=40, top_p=0.9, min_p=0.0)] * rows, list(range(rows)))
        log(f"keyed workspace reuse rows={rows}")
        gi, gs, _ = S.keyed_sample_rows(dev(x), recs, 0)
        wi, _, ws = O.keyed_sample_rows(x, O.DTYPE_F32, vocab, recs, 0)
        assert np.array_equal(host(gs), ws) and np.array_equal(host(gi), wi), rows


@pytest.mark.parametrize("dtype,rows,stride,valid", [(O.DTYPE_F32, 256, 151936, 151936), (O.DTYPE_BF16, 256, 151936, 151936),
                                                     (O.DTYPE_F16, 260, 20000, 19999), (O.DTYPE_F32, 256, 151940, 151933),
                                                     (O.DTYPE_F32, 300, 1001, 1001), (O.DTYPE_BF16, 257, 4098, 4097)])
def test_fused_keyed_full_batches(dtype, rows, stride, valid):
    """One block per row (256 rows and more): full vocabularies in every dtype, padded rows (valid < stride, columns
    past `valid` poisoned), and strides that rule out 16-byte loads."""
    need_gpu()
    rng = np.random.default_rng(rows + stride)
    x = W.peaked_logits(int(rng.integers(1 << 30)), rows, stride, 2.0, (4, 16), 6.0, 14.0)
    x[:, valid:] = 1e30  # never a candidate: past the valid columns
    x[5, :] = 0.5        # a row of one value
    x[7, rng.choice(valid, 100, replace=False)] = np.nan
    if dtype == O.DTYPE_BF16:
        data = W.to_bf16_bits(x)
        t = dev(data, torch.bfloat16)
    elif dtype == O.DTYPE_F16:
        data = np.clip(x, -6e4, 6e4).astype(np.float16).view(np.uint16)
        t = dev(data, torch.float16)
    else:
        data = x
        t = dev(data)
    recs = np.zeros(rows, dtype=S.KEYED_ROW_DTYPE)
    for r in range(rows):
        recs[r] = (int(rng.integers(1 << 62)), int(rng.integers(1 << 20)), float(rng.choice([0.0, 0.7, 1.0])),
                   float(rng.choice([1.0, 0.9, 0.5])), float(rng.choice([0.0, 0.05])), int(rng.choice([1, 20, 50, 56])), 1)
    log(f"fused keyed full batch dtype={dtype} rows={rows} stride={stride} valid={valid}")
    gi, gs, gv = S.keyed_sample_rows(t, recs, 2, valid=valid, out_vals=True)
    wi, wv, ws = O.keyed_sample_rows(data, dtype, valid, recs, 2)
    gi, gs, gv = host(gi), host(gs), host(gv)
    assert np.array_equal(gs, ws)
    assert np.array_equal(gi, wi), np.nonzero(gi != wi)[0][:10]
    assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32))


def test_tree_verify_on_device():
    """A tree round on the device: every node keyed-sampled at its own position (base + depth), then the accept walk;
    against the oracle's top-(k+8) + try_choose per row and accept_tree. Siblings share their depth's position; trees
    are built so that some drafts match the samples (long paths) and one tree holds a NaN row (a failed sequence)."""
    need_gpu()
    rng = np.random.default_rng(5)
    n_tree, nodes, vocab = 40, 15, 32_000
    rows = n_tree * nodes
    x = W.peaked_logits(77, rows, vocab, 2.0, (1, 3), 9.0, 14.0)  # few, high peaks: samples are predictable
    parents = np.zeros((n_tree, nodes), dtype=np.int32)
    depth = np.zeros((n_tree, nodes), dtype=np.int64)
    for t in range(n_tree):
        parents[t, 0] = -1
        for r in range(1, nodes):
            parents[t, r] = rng.integers(0, r)
            depth[t, r] = depth[t, parents[t, r]] + 1
    recs = np.zeros(rows, dtype=S.KEYED_ROW_DTYPE)
    base = rng.integers(100, 5000, n_tree)
    for t in range(n_tree):
        for r in range(nodes):
            recs[t * nodes + r] = (1234 + t, int(base[t] + depth[t, r]), [0.0, 0.7, 1.0][t % 3], 0.9, 0.0, 20, 1)
    # the oracle's samples, then tokens that follow them on some branches (so that paths go deep)
    wi, _, ws = O.keyed_sample_rows(x, O.DTYPE_F32, vocab, recs, 0)
    tokens = rng.integers(0, vocab, (n_tree, nodes)).astype(np.int32)
    for t in range(n_tree):
        for r in range(1, nodes):
            if rng.random() < 0.6:
                tokens[t, r] = wi[t * nodes + parents[t, r]]
    x[5 * nodes + 3, 17] = np.nan  # tree 5: row 3 has a NaN ... made a candidate below
    x[5 * nodes + 3, :] = np.nan
    wi, _, ws = O.keyed_sample_rows(x, O.DTYPE_F32, vocab, recs, 0)
    smp, path, plen, st = S.tree_verify(dev(x), recs, dev(tokens), dev(parents))
    smp, path, plen, st = host(smp), host(path), host(plen), host(st)
    assert np.array_equal(smp, wi)
    deep = 0
    for t in range(n_tree):
        rs = ws[t * nodes:(t + 1) * nodes]
        bad = rs[rs != 0]
        if bad.size:
            assert st[t] == bad[0] and plen[t] == 0 and (path[t] == -1).all()
            continue
        want = O.accept_tree(tokens[t], parents[t], wi[t * nodes:(t + 1) * nodes])
        assert st[t] == 0 and list(path[t, :plen[t]]) == want and (path[t, plen[t]:] == -1).all()
        deep += len(want) > 2
    assert st[5] == 2 and deep > 5


def test_device_keyed_pick_top_p_on_exact_running_sums():
    """Rows whose running probability sums land exactly on top_p (equal values: the quotients are exact powers of two)
    and a hair either side of it, so the device takes the ordered running sum rather than its lane-scan shortcut;
    against the oracle's try_choose."""
    need_gpu()
    rows, count = 96, 16
    ids = np.tile(np.arange(100, 100 + count, dtype=np.int32), (rows, 1))
    vals = np.zeros((rows, count), dtype=np.float32)
    vals[:, :8] = 1.0            # 8 equal leaders: probabilities sum to exact multiples of 1/8 of their mass
    vals[:, 8:] = -40.0
    recs = np.zeros(rows, dtype=S.KEYED_ROW_DTYPE)
    for r in range(rows):
        top_p = [0.25, 0.5, 0.75, 0.125 * (1 + r % 7)][r % 4]
        top_p = float(np.nextafter(top_p, 0.0 if r % 3 == 1 else 1.0)) if r % 3 else top_p
        recs[r] = (1000 + r, r, 1.0, top_p, 0.0, count, 1)
    gi, gv = S.keyed_pick(dev(ids), dev(vals), recs, 0)
    wi, wv = O.keyed_pick_rows(ids, vals, recs, 0)
    gi, gv = host(gi), host(gv)
    assert np.array_equal(gi, wi), np.nonzero(gi != wi)[0][:10]
    assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32))
