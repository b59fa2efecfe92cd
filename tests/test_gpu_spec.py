"""Speculative verification (gbs_spec_verify) on the GPU against the oracle: accepted lengths and tokens bit-exact."""
import numpy as np
import pytest

from oracle import oracle as O
from rexl3_amd import sampling as S
from rexl3_amd import workloads as W
from tests.gpu_util import dev, host, log, need_gpu

pytestmark = pytest.mark.gpu


def run(cfg):
    acc, toks, st = S.spec_verify(dev(cfg["target"]), dev(cfg["draft"]), dev(cfg["draft_ids"]), dev(cfg["temperatures"]),
                                  dev(cfg["u_accept"]), dev(cfg["u_resample"]))
    wa, wt, ws = O.spec_verify(cfg["target"], cfg["draft"], cfg["n_seq"], cfg["width"], cfg["draft_ids"], cfg["temperatures"],
                               cfg["u_accept"], cfg["u_resample"], threads=8)
    return (host(acc), host(toks), host(st)), (wa, wt, ws)


def test_config5_small_vocab_many_sequences():
    need_gpu()
    cfg = W.config5(seed=21, n_seq=64, width=7, vocab=3000)
    (a, t, s), (wa, wt, ws) = run(cfg)
    assert np.array_equal(s, ws)
    assert np.array_equal(a, wa)
    assert np.array_equal(t, wt)
    log(f"accepted lengths {np.bincount(a, minlength=8)}")


def test_config5_full_vocab():
    need_gpu()
    cfg = W.config5(seed=5, n_seq=8, width=7)
    (a, t, s), (wa, wt, ws) = run(cfg)
    assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt)


def test_config5_at_its_own_shape():
    """Config 5 as the bench times it: 32 sequences x (7 drafts + 1 bonus) = 256 rows of 151,936 (the one-block-per-row
    kernel), with greedy rows whose maxima tie, and drafts the target gives no mass (certain rejections)."""
    need_gpu()
    cfg = W.config5(seed=5, n_seq=32, width=7)
    V = cfg["target"].shape[1]
    log("config5 32 x 8 x 151936")
    cfg["temperatures"][0:8] = 0.0                  # sequence 0 greedy; its rows' maxima tie at three ids
    for j in range(8):
        cfg["target"][j, [V - 1, 11 + j, V // 2]] = 40.0
    for s in (3, 9, 20):                            # certain rejection of draft 0 (p(x) = 0)
        r = s * 8
        cfg["target"][r, cfg["draft_ids"][s, 0]] = -np.inf
    (a, t, s), (wa, wt, ws) = run(cfg)
    assert (ws == 0).all()
    assert wa[3] == 0 and wa[9] == 0 and wa[20] == 0
    assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt)
    log(f"accepted lengths {np.bincount(a, minlength=8)}")


@pytest.mark.parametrize("n_seq", [6, 60])  # 24 rows: split kernels; 240 rows: one block per row
def test_spec_greedy_and_errors(n_seq):
    need_gpu()
    cfg = W.config5(seed=3, n_seq=n_seq, width=3, vocab=1000)
    cfg["temperatures"][0:4] = 0.0        # sequence 0 greedy
    cfg["draft_ids"][1, 1] = 1000          # invalid id
    cfg["target"][2 * 4 + 2, 5] = np.nan   # NaN in sequence 2
    cfg["u_resample"][3] = 1.0             # invalid
    cfg["draft"][4 * 4 + 1, :] = -np.inf   # empty draft row
    (a, t, s), (wa, wt, ws) = run(cfg)
    assert list(ws[:6]) == [0, 3, 2, 3, 1, 0]
    assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt)


def test_spec_workspace_reused_across_shapes():
    """One workspace serves launches of different shapes (the counters sit at fixed per-row and per-sequence offsets)."""
    need_gpu()
    for i, (n_seq, width) in enumerate([(40, 7), (2, 1), (40, 7), (9, 3), (40, 7)]):
        cfg = W.config5(seed=60 + i, n_seq=n_seq, width=width, vocab=3000)
        log(f"spec workspace reuse n_seq={n_seq} width={width}")
        (a, t, s), (wa, wt, ws) = run(cfg)
        assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt), (n_seq, width)


@pytest.mark.parametrize("n_seq", [12, 50])  # 48 rows: split kernels; 200 rows: one block per row
@pytest.mark.parametrize("vocab", [3001, 8196, 12288])
def test_spec_vocab_shapes_and_max_ties(vocab, n_seq):
    """Odd vocabularies (single-element loads), splits that end mid-iteration, and greedy rows whose maximum is tied
    (the lowest id wins, -0 ties +0)."""
    need_gpu()
    cfg = W.config5(seed=70 + vocab % 17, n_seq=n_seq, width=3, vocab=vocab)
    log(f"spec vocab={vocab} n_seq={n_seq}")
    cfg["temperatures"][0:4] = 0.0                       # sequence 0 greedy, tied maxima in every row
    for j in range(4):
        cfg["target"][j, :] = np.minimum(cfg["target"][j, :], 5.0)
        cfg["target"][j, [vocab - 1, 7 + j, vocab // 2]] = 30.0
    cfg["temperatures"][4:8] = 0.0                       # sequence 1 greedy, a row that is all zeros of both signs
    cfg["target"][5, :] = 0.0
    cfg["target"][5, : vocab // 3] = -0.0
    cfg["target"][6, :] = -np.inf
    cfg["target"][6, vocab - 2] = -0.0
    cfg["target"][6, vocab - 1] = 0.0
    (a, t, s), (wa, wt, ws) = run(cfg)
    assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt)


def test_spec_zero_residual_draws_target_argmax():
    """A rejected draft with zero residual mass everywhere (draft row == target row, the draft token at -inf in both)
    resamples the target's argmax, as the definition's fallback says."""
    need_gpu()
    cfg = W.config5(seed=91, n_seq=50, width=3, vocab=5000)
    for s in range(4):
        r = s * 4
        cfg["draft"][r] = cfg["target"][r]
        x = 17 + s
        cfg["target"][r, x] = -np.inf
        cfg["draft"][r, x] = -np.inf
        cfg["draft_ids"][s, 0] = x
    (a, t, s), (wa, wt, ws) = run(cfg)
    assert list(wa[:4]) == [0, 0, 0, 0]
    assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt)


@pytest.mark.parametrize("n_seq,vocab,pad", [(8, 3001, 7), (32, 2048, 64)])
def test_padded_rows(n_seq, vocab, pad):
    """Target and draft rows with a row stride above `vocab` (the lm_head's padded layout): the pad columns hold NaN and
    +inf, which must never be read; the results equal the oracle's on the unpadded rows. 32 sequences take the
    one-block-per-row kernel, 8 the split kernels."""
    need_gpu()
    cfg = W.config5(seed=31 + n_seq, n_seq=n_seq, width=7, vocab=vocab)
    R = cfg["target"].shape[0]
    tp = np.full((R, vocab + pad), np.nan, np.float32)
    dp = np.full((R, vocab + pad), np.inf, np.float32)
    tp[:, vocab + 1::2] = np.inf
    tp[:, :vocab] = cfg["target"]
    dp[:, :vocab] = cfg["draft"]
    log(f"padded spec rows n_seq={n_seq} vocab={vocab} stride={vocab + pad}")
    acc, toks, st = S.spec_verify(dev(tp), dev(dp), dev(cfg["draft_ids"]), dev(cfg["temperatures"]), dev(cfg["u_accept"]),
                                  dev(cfg["u_resample"]), vocab=vocab)
    wa, wt, ws = O.spec_verify(cfg["target"], cfg["draft"], n_seq, 7, cfg["draft_ids"], cfg["temperatures"], cfg["u_accept"],
                               cfg["u_resample"], threads=8)
    assert np.array_equal(host(st), ws) and np.array_equal(host(acc), wa) and np.array_equal(host(toks), wt)
    with pytest.raises(ValueError):
        S.spec_verify(dev(tp), dev(dp[:, :vocab].copy()), dev(cfg["draft_ids"]), dev(cfg["temperatures"]),
                      dev(cfg["u_accept"]), dev(cfg["u_resample"]), vocab=vocab)


def _ratio(cfg, r, x, T):
    """p(x) / q(x) of row r in float64: exact masses of the draft token over float64 sums of the row's masses."""
    c2 = O.temp_scale(T)
    t, d = cfg["target"][r], cfg["draft"][r]
    Mt, Md = float(t.max()), float(d.max())
    ep, eq = O.mass(float(t[x]), Mt, c2), O.mass(float(d[x]), Md, c2)
    zp = np.exp2((t.astype(np.float64) - Mt) * c2).sum() * 2.0**44
    zq = np.exp2((d.astype(np.float64) - Md) * c2).sum() * 2.0**44
    return (ep * zq) / (eq * zp) if eq else np.inf


@pytest.mark.parametrize("vocab", [32768, 151_936])
def test_spec_one_read_acceptance_on_the_boundary(vocab):
    """The one-block-per-row kernel decides a draft from float bounds on the mass sums and leaves the test open when u
    lies within their error of p(x) / q(x); the exact pass then settles it with the integer rule. Here every draft of
    the even sequences has u within 2^-20 of its ratio (either side), so open tests come in runs: a sequence's exact pass
    covers several rows before its first rejection. Accepted lengths and tokens equal the oracle's."""
    need_gpu()
    n_seq, width = 32 if vocab > 100_000 else 48, 4
    cfg = W.config5(seed=41, n_seq=n_seq, width=width, vocab=vocab)
    W1 = width + 1
    rng = np.random.default_rng(7)
    near = 0
    for s in range(0, n_seq, 2):
        for j in range(width):
            r = s * W1 + j
            x = int(cfg["draft_ids"][s, j])
            q = _ratio(cfg, r, x, float(cfg["temperatures"][r]))
            if q < 0.999:
                cfg["u_accept"][s, j] = np.float32(q * (1.0 + rng.uniform(-2.0**-20, 2.0**-20)))
                near += 1
    cfg["target"][1 * W1, 5] = np.inf                    # sequence 1: an infinite logit (no float bounds for its row)
    cfg["temperatures"][3 * W1:4 * W1] = 1e-30           # sequence 3: c2 near the float range's end
    log(f"spec boundary vocab={vocab} n_seq={n_seq}: {near} drafts with u at p(x)/q(x)")
    (a, t, s), (wa, wt, ws) = run(cfg)
    assert near >= n_seq
    assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt)
    log(f"accepted lengths {np.bincount(a, minlength=W1)}")


@pytest.mark.parametrize("n_seq,width,vocab", [(32, 7, 151_936), (50, 3, 8196), (8, 7, 151_936), (12, 3, 12_288)])
def test_spec_row_block_sweep_given_up(n_seq, width, vocab):
    """(256 and 200 rows: one block per row; 64 and 48 rows: the split row pass.) The row pass's sweep of the draw rows with a wait limit of 0: a block that looks before its sequence is decided
    gives up at once, so sequences mix the row-block sweep and the exact pass's own (forced from the host through the
    library's wait limit; every kernel exits normally). Results must equal the oracle's, then again with the default
    limit on the same workspace."""
    need_gpu()
    from rexl3_amd import _lib
    lib = _lib.load()
    cfg = W.config5(seed=77 + n_seq, n_seq=n_seq, width=width, vocab=vocab)
    log(f"spec sweep given up n_seq={n_seq} width={width} vocab={vocab}")
    prev = lib.gbs_spec_set_fuse_wait(0)
    try:
        (a, t, s), (wa, wt, ws) = run(cfg)
    finally:
        assert lib.gbs_spec_set_fuse_wait(prev) == 0
    assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt)
    (a, t, s), _ = run(cfg)
    assert np.array_equal(s, ws) and np.array_equal(a, wa) and np.array_equal(t, wt)
