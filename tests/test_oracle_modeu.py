"""Pins of the oracle's extended pipeline (no reference code exists for it: crates/server/src/api.rs:196-206 refuses
penalties and grammars). Each check is an independent computation -- exact rationals (fractions.Fraction), closed forms,
numpy float64 -- chosen so that a dropped term, a wrong index or a wrong rounding in the C oracle fails it."""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O
from rexl3_amd import workloads as W

TWO44 = 1 << 44


def f32(x):
    return float(np.float32(x))


# ---------------------------------------------------------------- the integer mass

def test_mass_closed_forms():
    c2 = O.temp_scale(1.0)
    assert c2 == f32(1.44269504088896340736)
    for m in [0.0, -0.0, 1.5, -3.25, 1e30, -1e-30]:
        assert O.mass(m, m, c2) == TWO44
    # mass(M - d) ~ 2^44 * exp(-d), to the accuracy of an f32 exponent (relative 1e-6) while it is large
    rng = np.random.default_rng(0)
    for _ in range(4000):
        M = f32(rng.uniform(-20, 20))
        T = f32(rng.choice([0.3, 0.7, 1.0, 2.5]))
        c2 = O.temp_scale(T)
        l = f32(M - rng.uniform(0, 25))
        y = float(np.float32(np.float32(l) - np.float32(M)) * np.float32(c2))
        want = TWO44 * 2.0 ** y
        got = O.mass(l, M, c2)
        if want > 2**20:
            assert abs(got - want) <= 2e-6 * want + 1, (l, M, T, got, want)
    # below 2^-64 of the maximum the mass is exactly zero; -inf has no mass
    assert O.mass(-100.0, 0.0, O.temp_scale(1.0)) == 0
    assert O.mass(float("-inf"), 0.0, O.temp_scale(1.0)) == 0
    assert O.mass(0.0, float("inf"), O.temp_scale(1.0)) == 0


def test_mass_is_the_floor_of_the_polynomial_value():
    """For y = (l - M) * c2 the mass is floor(p(f) * 2^24) * 2^(n + 20) with n = rint(y), f = y - n and p the degree-7
    Taylor polynomial of 2^f in f32 Horner form; restated here with numpy float32 and fma emulated in float64 (exact
    for f32 operands: the product of two f32 fits a double exactly, and one rounding to f32 follows)."""
    coef = [np.float32(c) for c in [1.52527338e-05, 1.54035304e-04, 1.33335581e-03, 9.61812911e-03, 5.55041087e-02,
                                    2.40226507e-01, 6.93147181e-01, 1.0]]

    def fmaf(a, b, c):
        return np.float32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))

    def mass_py(l, M, c2):
        l, M, c2 = np.float32(l), np.float32(M), np.float32(c2)
        if l == M:
            return TWO44
        y = np.float32(np.float32(l - M) * c2)
        if not y >= -64:
            return 0
        n = np.float32(np.rint(y))
        f = np.float32(y - n)
        p = coef[0]
        for c in coef[1:]:
            p = fmaf(p, f, c)
        m = int(np.float32(p * np.float32(16777216.0)))
        sh = int(n) + 20
        return m << sh if sh >= 0 else (m >> -sh if sh > -32 else 0)

    rng = np.random.default_rng(1)
    for _ in range(3000):
        M = f32(rng.uniform(-5, 5))
        l = f32(M - abs(rng.standard_normal()) * rng.choice([0.01, 1, 10, 40]))
        c2 = O.temp_scale(f32(rng.choice([0.2, 0.8, 1.0, 1.7])))
        assert O.mass(l, M, c2) == mass_py(l, M, c2), (l, M, c2)


def test_mul_floor_is_exact():
    rng = np.random.default_rng(2)
    vals = [0.0, 1e-45, 2**-126, 0.5, 0.9, f32(1 - 2**-24), 0.1, 1.0]
    vals += [f32(v) for v in rng.uniform(0, 1, 300)]
    zs = [0, 1, 2, 3, 2**44, 2**63 - 1, 12345678901234567] + [int(z) for z in rng.integers(0, 2**62, 50)]
    for x in vals:
        for z in zs:
            got, exact = O.mul_floor(x, z)
            q = Fraction(float(np.float32(x))) * z
            assert got == math.floor(q), (x, z)
            assert exact == (q.denominator == 1)


def test_penalty_known_answers():
    p = O.RowParams(1.0, 1.0, 0.0, 2.0, 1.0, 0.5, 0, 0)
    rinv = f32(1.0 / 2.0)
    # x = 2, c = 3: 2 / 2 - (3 * 0.5 + 1) = -1.5 exactly; x = -2: -2 * 2 - 2.5 = -6.5
    assert O.lib().gbo_penalized_logit(2.0, 3, p, rinv) == -1.5
    assert O.lib().gbo_penalized_logit(-2.0, 3, p, rinv) == -6.5
    # a count of 0 (or below) leaves every bit, -0 and NaN payloads included
    for x in [0.0, -0.0, 1.0, -7.25, float("inf"), float("-inf")]:
        r = O.lib().gbo_penalized_logit(x, 0, p, rinv)
        assert np.float32(r).tobytes() == np.float32(x).tobytes()
    # identity parameters change nothing even with counts
    ident = O.RowParams(1.0, 1.0, 0.0, 1.0, 0.0, 0.0, 0, 0)
    for x in [3.5, -1e-40, -0.0]:
        assert np.float32(O.lib().gbo_penalized_logit(x, 9, ident, 1.0)).tobytes() == np.float32(x).tobytes()


# ---------------------------------------------------------------- the draw, against exact rationals

def row_params(**kw):
    d = dict(temperature=1.0, top_p=1.0, min_p=0.0, repetition=1.0, presence=0.0, frequency=0.0, top_k=0)
    d.update(kw)
    p = np.zeros(1, dtype=O.ROW_PARAMS_DTYPE)
    for k, v in d.items():
        p[k] = v
    return p[0]


def expected_kept(l, params):
    """The kept set and its masses by the pipeline's definition, in exact arithmetic on the oracle's masses:
    order (l desc, id asc); top-k; top-p as the smallest prefix whose mass reaches top_p of the top-k mass (the
    reference's searchsorted rule); min-p as the filter mass >= min_p * 2^44."""
    valid = [i for i in range(len(l)) if l[i] > -np.inf]
    order = sorted(valid, key=lambda i: (-float(l[i]), i))
    M = l[order[0]]
    c2 = O.temp_scale(float(params["temperature"]))
    K = order[:params["top_k"]] if 0 < params["top_k"] < len(order) else order
    E = {i: O.mass(float(l[i]), float(M), c2) for i in K}
    keep = len(K)
    tp = Fraction(float(params["top_p"]))
    if 0 < tp < 1:
        Z = sum(E.values())
        c = 0
        below = 0
        for i in K:
            c += E[i]
            if Fraction(c) < tp * Z:
                below += 1
        keep = min(below + 1, len(K))
    mp = Fraction(float(params["min_p"]))
    kept = [i for i in K[:keep] if mp == 0 or E[i] >= mp * TWO44]
    return sorted(kept), E


def draw_for(l, params, u):
    o = O.sample_row_detail(np.asarray(l, dtype=np.float32), O.DTYPE_F32, None, None, params, u)
    return o


def test_inverse_cdf_boundaries_match_exact_rationals():
    """For each kept token, the smallest f32 uniform (on the 2^-24 grid) that selects it and the one just below, from
    t = floor(u * Z) and the ascending-id cumulative masses computed with Fractions."""
    rng = np.random.default_rng(3)
    for trial in range(150):
        V = int(rng.integers(1, 13))
        l = (rng.standard_normal(V) * rng.choice([0.5, 2, 6])).astype(np.float32)
        if V > 3 and trial % 5 == 0:
            l[rng.integers(0, V)] = -np.inf
        if not np.isfinite(l).any():
            continue
        params = row_params(temperature=f32(rng.choice([0.3, 0.8, 1.0, 1.6])), top_k=int(rng.choice([0, 1, 2, 5])),
                            top_p=f32(rng.choice([1.0, 0.95, 0.5, 0.2])), min_p=f32(rng.choice([0.0, 0.05, 0.3])))
        kept, E = expected_kept(l, params)
        Z = sum(E[i] for i in kept)
        A = 0
        for i in kept:
            # smallest m in [0, 2^24) with floor(m * Z / 2^24) >= A
            m = -((-A * (1 << 24)) // Z)
            if m < (1 << 24):
                o = draw_for(l, params, f32(m / 2**24))
                assert o.status == 0 and o.id == i, (trial, i, m)
                assert o.z_kept == Z and o.kept == len(kept)
                assert abs(o.prob - E[i] / Z) <= 1e-6 * (E[i] / Z)
                if m > 0 and A > 0:
                    prev = kept[kept.index(i) - 1]
                    assert draw_for(l, params, f32((m - 1) / 2**24)).id == prev
            A += E[i]
        assert draw_for(l, params, 0.0).id == kept[0]
        assert draw_for(l, params, f32(1 - 2**-24)).id == kept[-1]


def test_closed_form_rows():
    l = np.array([1.0, 3.0, 3.0, -2.0, 0.5], dtype=np.float32)
    g = draw_for(l, row_params(temperature=0.0), 0.7)
    assert (g.id, g.greedy, g.prob) == (1, 1, 1.0)            # greedy: lowest id among tied maxima
    assert draw_for(l, row_params(top_k=1), 0.99).id == 1     # top_k 1 is the argmax
    assert draw_for(np.array([-np.inf, 2.0, -np.inf], np.float32), row_params(), 0.5).id == 1
    o = draw_for(np.array([-np.inf, -np.inf], np.float32), row_params(), 0.5)
    assert o.status == O.ROW_NO_CANDIDATES and o.id == -1
    o = draw_for(np.array([1.0, np.nan], np.float32), row_params(), 0.5)
    assert o.status == O.ROW_NAN_LOGIT
    for bad in [row_params(temperature=-1.0), row_params(top_p=1.5), row_params(min_p=-0.1), row_params(repetition=0.0),
                row_params(top_k=-1), row_params(presence=float("inf"))]:
        assert draw_for(l, bad, 0.5).status == O.ROW_INVALID_PARAMS
    for u in [1.0, -0.25, float("nan")]:
        assert draw_for(l, row_params(), u).status == O.ROW_INVALID_PARAMS
    # an all-equal row is uniform over every token: t = floor(u * V * 2^44) picks id floor(u * V)
    eq = np.full(10, 0.5, np.float32)
    for k in range(10):
        assert draw_for(eq, row_params(), f32(k / 10 + 0.01)).id == k


def test_logprob_is_the_float64_log_softmax():
    rng = np.random.default_rng(4)
    for _ in range(50):
        V = int(rng.integers(2, 3000))
        l = (rng.standard_normal(V) * 3).astype(np.float32)
        T = f32(rng.choice([0.5, 1.0, 2.0]))
        o = draw_for(l, row_params(temperature=T), f32(rng.uniform()))
        z = l.astype(np.float64) / float(T)
        ls = z - z.max()
        want = ls[o.id] - np.log(np.exp(ls).sum())
        assert abs(o.logprob - want) <= 1e-12 * max(1.0, abs(want))


def test_batch_driver_matches_rows_and_threads_do_not_matter():
    cfg = W.config4(rows=12)
    a = O.sample_rows(cfg["logits"], O.DTYPE_F32, None, cfg["mask"], cfg["params"], cfg["uniforms"], threads=1)
    b = O.sample_rows(cfg["logits"], O.DTYPE_F32, None, cfg["mask"], cfg["params"], cfg["uniforms"], threads=5)
    for k in a:
        assert np.array_equal(a[k], b[k])
    r = 7
    words = cfg["mask"].shape[1]
    o = O.sample_row_detail(cfg["logits"][r], O.DTYPE_F32, None, cfg["mask"][r], cfg["params"][r], float(cfg["uniforms"][r]))
    assert o.id == a["ids"][r] and words == (cfg["logits"].shape[1] + 31) // 32


# ---------------------------------------------------------------- speculative verification

def spec_rows(rng, width, V, T):
    target = (rng.standard_normal((width + 1, V)) * 1.5).astype(np.float32)
    draft = (target + rng.standard_normal((width + 1, V)).astype(np.float32) * 0.7).astype(np.float32)
    return target, draft


def masses(row, T):
    M = row.max()
    c2 = O.temp_scale(T)
    return [O.mass(float(v), float(M), c2) for v in row]


def test_spec_accept_rule_and_residual_against_rationals():
    """accept iff u * q(x) < p(x) in exact rationals; at the first rejection the token is the residual max(p - q, 0)'s
    inverse-CDF draw in ascending id order, exactly."""
    rng = np.random.default_rng(5)
    for trial in range(120):
        width, V, T = int(rng.integers(1, 4)), int(rng.integers(2, 9)), f32(rng.choice([0.7, 1.0, 1.4]))
        target, draft = spec_rows(rng, width, V, T)
        ids = rng.integers(0, V, width).astype(np.int32)
        ua = rng.uniform(0, 1, width).astype(np.float32)
        ur = np.float32(rng.uniform())
        temps = np.full(width + 1, T, np.float32)
        acc, toks, st = O.spec_verify(target[None], draft[None], 1, width, ids[None], temps, ua[None], np.array([ur]))
        assert st[0] == 0
        want_acc = width
        for j in range(width):
            Ep, Eq = masses(target[j], T), masses(draft[j], T)
            p = Fraction(Ep[ids[j]], sum(Ep))
            q = Fraction(Eq[ids[j]], sum(Eq))
            if not Fraction(float(ua[j])) * q < p:
                want_acc = j
                break
        assert acc[0] == want_acc
        assert list(toks[0, :want_acc]) == list(ids[:want_acc])
        j = want_acc
        Ep = masses(target[j], T)
        if j < width:
            Eq = masses(draft[j], T)
            w = [max(Fraction(a, sum(Ep)) - Fraction(b, sum(Eq)), 0) for a, b in zip(Ep, Eq)]
        else:
            w = [Fraction(a) for a in Ep]
        tot = sum(w)
        t = Fraction(float(ur)) * tot
        c = Fraction(0)
        want_tok = None
        for i, wi in enumerate(w):
            c += wi
            if wi > 0 and c > t:
                want_tok = i
                break
        # floor(u * R) in integers is the same comparison: c_int > floor(t_int) <=> c > t for integer-scaled sums
        assert toks[0, j] == want_tok, (trial, toks[0], want_tok)
        assert (toks[0, j + 1:] == -1).all()


def test_spec_marginal_is_the_target_distribution():
    """Rejection sampling keeps the target's marginal: for the first position, sum over drafts x of
    q(x) * [P(accept x) 1{y = x} + P(reject x) r(y)] == p(y), exactly, with the oracle's integer masses."""
    rng = np.random.default_rng(6)
    for _ in range(30):
        V, T = int(rng.integers(2, 7)), 1.0
        target, draft = spec_rows(rng, 1, V, T)
        Ep, Eq = masses(target[0], T), masses(draft[0], T)
        p = [Fraction(a, sum(Ep)) for a in Ep]
        q = [Fraction(b, sum(Eq)) for b in Eq]
        r = [max(a - b, 0) for a, b in zip(p, q)]
        R = sum(r)
        marg = [Fraction(0)] * V
        for x in range(V):
            acc = min(Fraction(1), p[x] / q[x]) if q[x] > 0 else Fraction(1)
            marg[x] += q[x] * acc
            if R > 0:
                for y in range(V):
                    marg[y] += q[x] * (1 - acc) * r[y] / R
        assert marg == p


def test_spec_greedy_and_errors():
    rng = np.random.default_rng(7)
    target, draft = spec_rows(rng, 3, 6, 1.0)
    am = [int(np.argmax(t)) for t in target]
    ids = np.array([am[0], am[1], (am[2] + 1) % 6], np.int32)
    temps = np.zeros(4, np.float32)
    acc, toks, st = O.spec_verify(target[None], draft[None], 1, 3, ids[None], temps, np.full((1, 3), 0.5, np.float32),
                                  np.array([0.5], np.float32))
    assert st[0] == 0 and acc[0] == 2 and list(toks[0]) == [am[0], am[1], am[2], -1]
    bad = ids.copy()
    bad[0] = 6
    assert O.spec_verify(target[None], draft[None], 1, 3, bad[None], temps, np.full((1, 3), 0.5, np.float32),
                         np.array([0.5], np.float32))[2][0] == O.ROW_INVALID_PARAMS
