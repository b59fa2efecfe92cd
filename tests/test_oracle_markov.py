"""The oracle's DSV4 Markov walk (crates/cuda/csrc/dsv4_mtp_gpu.cu:1233-1480, 1662-1718) against an independent numpy
restatement: each thread's top 4 of its strided slice by a stable argsort, the bias as a float64 dot product, the
picks by lexsort. The oracle's kernel-order float arithmetic differs from float64 by rounding only, so the ids agree
on these draws (no near-ties) and the biased logits agree to float precision."""
import numpy as np

from oracle import oracle as O


def bf16_bits(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_vals(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def numpy_walk(logits, first, embed_b, head_b, rows, keyed, cand_k, seed, temperature, top_p, min_p, base_pos):
    lg = logits.astype(np.float64).copy()
    V = lg.shape[1]
    emb = bf16_vals(embed_b).astype(np.float64)
    hed = bf16_vals(head_b).astype(np.float64)
    ids = [first]
    conf = []
    for k in range(rows):
        cand = []
        for t in range(256):
            sl = logits[k, t::256]
            order = np.argsort(-sl, kind="stable")[:4]  # strict >: the first of equal values stays
            cand += [int(t + 256 * i) for i in order]
        tok = ids[-1]
        e = emb[tok] if 0 <= tok < V else np.zeros(256)
        sc = np.array([lg[k, v] + e @ hed[v] for v in cand])
        for v, s in zip(cand, sc):
            lg[k, v] = s
        order = np.lexsort((np.array(cand), -sc))
        if not keyed:
            ids.append(cand[order[0]])
            continue
        kk = min(max(cand_k, 1), 64)
        top = order[:kk]
        i, m = O.keyed_choose(sc[top].astype(np.float32), np.array(cand, np.int32)[top], seed, temperature, top_p, min_p, base_pos + k)
        ids.append(cand[top[i]])
        conf.append(1.0 / (1.0 + np.exp(-m)))
    return np.array(ids), np.array(conf), lg


def case(seed, V=2048, rows=5):
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    embed = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    head = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    return logits, embed, head


def test_fast_walk_matches_numpy():
    logits, embed, head = case(1)
    ids, _, lg = O.markov_walk(logits, 7, embed, head, 5)
    want, _, wl = numpy_walk(logits, 7, embed, head, 5, False, 1, 0, 1.0, 1.0, 0.0, 0)
    assert list(ids) == list(want)
    np.testing.assert_allclose(lg, wl, rtol=1e-5, atol=1e-5)
    changed = (lg != logits).sum(axis=1)
    assert (changed > 900).all() and (changed <= 1024).all()  # the 1024 candidates of each row, and nothing else


def test_keyed_walk_matches_numpy():
    logits, embed, head = case(2)
    for cand_k, t, p, mp in [(1, 0.7, 1.0, 0.0), (8, 0.7, 0.9, 0.0), (64, 1.3, 0.95, 0.05), (20, 0.0, 1.0, 0.0)]:
        ids, conf, _ = O.markov_walk(logits, 3, embed, head, 5, True, cand_k, 99, t, p, mp, 1000)
        want, wc, _ = numpy_walk(logits, 3, embed, head, 5, True, cand_k, 99, t, p, mp, 1000)
        assert list(ids) == list(want), (cand_k, t)
        np.testing.assert_allclose(conf, wc, rtol=1e-6)


def test_out_of_range_token_adds_nothing():
    logits, embed, head = case(3, rows=1)
    ids, _, lg = O.markov_walk(logits, 10**6, embed, head, 1)
    assert np.array_equal(lg, logits)  # a zero bias leaves every logit as it was (x + 0 = x)
    assert ids[1] == int(np.argmax(logits[0]))
