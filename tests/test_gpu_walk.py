"""The draft head's selector walk on the device (gb_dflash_selector_walk_keyed / _ragged / gb_dflash_selector_walk)
against the oracle's restatement of crates/cuda/csrc/dflash2.cu:436-519: tokens bit-exact, and the pick's score and
margin bit-exact (the same float arithmetic in the same order)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from rexl3_amd import _lib
from rexl3_amd import sampling as S
from tests.gpu_util import dev, host, log, need_gpu

pytestmark = pytest.mark.gpu


def inputs(seed, n_seq, rows_total, k, rank, vocab, gate_f32):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, vocab, (rows_total, k)).astype(np.int32)
    vals = (rng.standard_normal((rows_total, k)) * 2).astype(np.float32)
    vals[rng.random((rows_total, k)) < 0.05] = 1.0  # ties among the unary scores
    gate = (rng.standard_normal((rows_total, rank)) * 0.5).astype(np.float32)
    if not gate_f32:
        gate = (gate.view(np.uint32) >> 16).astype(np.uint16)  # bf16 bits (truncated)
    pred = (rng.standard_normal((vocab, rank)) * 0.3).astype(np.float16).view(np.uint16)
    succ = (rng.standard_normal((vocab, rank)) * 0.3).astype(np.float16).view(np.uint16)
    anchor = rng.integers(0, vocab, n_seq).astype(np.int32)
    samp = np.zeros(n_seq, dtype=O.WALK_SAMPLING_DTYPE)
    for b in range(n_seq):
        samp[b] = (int(rng.integers(1 << 62)), int(rng.integers(1 << 20)), float(rng.choice([0.0, 0.5, 1.0, 1.5])),
                   float(rng.choice([1.0, 0.9, 0.6])), float(rng.choice([0.0, 0.05])), int(b % 3 != 0), 0)
    return anchor, ids, vals, gate, pred, succ, samp


def check_shapes(anchor, ids, gate, pred, succ, n_seq, rows_total, row_off=None):
    """Every index the kernel takes is inside the arrays it reads: ids and anchors below the codebooks' row count, one
    gate row per candidate row, row offsets from 0 to the row count, non-decreasing."""
    V = pred.shape[0]
    assert succ.shape[0] == V and pred.shape[1] == succ.shape[1] == gate.shape[1]
    assert anchor.shape == (n_seq,) and ids.shape[0] == rows_total == gate.shape[0]
    assert 0 <= ids.min() and ids.max() < V and 0 <= anchor.min() and anchor.max() < V
    if row_off is not None:
        assert row_off.shape == (n_seq + 1,) and row_off[0] == 0 and row_off[-1] == rows_total and (np.diff(row_off) >= 0).all()


def on_device(anchor, ids, vals, gate, gate_f32, pred, succ, samp, row_off=None):
    n_seq = anchor.shape[0]
    check_shapes(anchor, ids, gate, pred, succ, n_seq, ids.shape[0], row_off)
    # every device array stays bound to a name until the launch has been made and its results read
    d_anchor, d_ids, d_vals = dev(anchor), dev(ids), dev(vals)
    d_gate = dev(gate) if gate_f32 else dev(gate, torch.bfloat16)
    d_pred, d_succ = dev(pred, torch.float16), dev(succ, torch.float16)
    d_off = None if row_off is None else dev(row_off)
    t, c, m = S.selector_walk(d_anchor, d_ids, d_vals, d_gate, d_pred, d_succ, samp, d_off)
    torch.cuda.synchronize()
    return t, c, m


@pytest.mark.parametrize("k,rank,gate_f32", [(16, 256, False), (64, 33, True), (1, 8, True), (40, 300, False)])
def test_walk_uniform_blocks(k, rank, gate_f32):
    need_gpu()
    n_seq, rows, vocab = 24, 8, 5000
    log(f"walk k={k} rank={rank} gate_f32={gate_f32}")
    anchor, ids, vals, gate, pred, succ, samp = inputs(k * 7 + rank, n_seq, n_seq * rows, k, rank, vocab, gate_f32)
    for sampling in (samp, None):
        t, c, _ = on_device(anchor, ids, vals, gate, gate_f32, pred, succ, sampling)
        wt, wc, _ = O.selector_walk(anchor, ids, vals, gate, gate_f32, pred, succ, n_seq, rows, sampling)
        assert np.array_equal(host(t), wt)
        assert np.array_equal(host(c).view(np.uint32), wc.view(np.uint32))


def test_walk_ragged_with_margins_and_the_plain_launcher():
    need_gpu()
    rng = np.random.default_rng(11)
    n_seq, k, rank, vocab = 30, 32, 128, 4000
    lens = rng.integers(0, 17, n_seq)
    row_off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    anchor, ids, vals, gate, pred, succ, samp = inputs(3, n_seq, int(row_off[-1]), k, rank, vocab, False)
    t, c, m = on_device(anchor, ids, vals, gate, False, pred, succ, samp, row_off)
    wt, wc, wm = O.selector_walk(anchor, ids, vals, gate, False, pred, succ, n_seq, 0, samp, row_off)
    assert np.array_equal(host(t), wt)
    assert np.array_equal(host(c).view(np.uint32), wc.view(np.uint32))
    assert np.array_equal(host(m).view(np.uint32), wm.view(np.uint32))
    # the plain launcher is the keyed one with every sequence unkeyed
    n2, rows = 6, 5
    anchor, ids, vals, gate, pred, succ, _ = inputs(5, n2, n2 * rows, k, rank, vocab, True)
    check_shapes(anchor, ids, gate, pred, succ, n2, n2 * rows)
    out = torch.empty(n2 * rows, dtype=torch.int32, device="cuda")
    conf = torch.empty(n2 * rows, dtype=torch.float32, device="cuda")
    # every device array stays bound to a name until the launch has been made and its results read
    d_anchor, d_ids, d_vals, d_gate = dev(anchor), dev(ids), dev(vals), dev(gate)
    d_pred, d_succ = dev(pred, torch.float16), dev(succ, torch.float16)
    _lib.call("gb_dflash_selector_walk", S._ptr(d_anchor), S._ptr(d_ids), S._ptr(d_vals), S._ptr(d_gate), 1, S._ptr(d_pred),
              S._ptr(d_succ), n2, rows, k, rank, S._ptr(out), S._ptr(conf), S._stream(torch.device("cuda")))
    torch.cuda.synchronize()
    wt, wc, _ = O.selector_walk(anchor, ids, vals, gate, True, pred, succ, n2, rows, None)
    assert np.array_equal(host(out), wt) and np.array_equal(host(conf).view(np.uint32), wc.view(np.uint32))


def test_walk_known_answers_on_the_device():
    """crates/spec/src/lib.rs:391-493's cases through the device kernel (f16 codebooks of 64 ids, f32 gate)."""
    need_gpu()
    V = 64

    def cb(fn, rank):
        return np.asarray([fn(i) for i in range(V)], dtype=np.float16).view(np.uint16).reshape(V, rank)

    def walk(anchor, cands, unary, hidden, pred, succ, T=None):
        rank = len(hidden[0])
        samp = None
        if T is not None:
            samp = np.zeros(1, dtype=O.WALK_SAMPLING_DTYPE)
            samp[0] = (0, 5, T, 1.0, 0.0, 1, 0)
        t, _, _ = on_device(np.array([anchor], np.int32), np.array(cands, np.int32), np.array(unary, np.float32),
                            np.array(hidden, np.float32), True, cb(pred, rank), cb(succ, rank), samp)
        return list(host(t))

    z2 = lambda i: [0.0, 0.0]  # noqa: E731
    assert walk(1, [[10, 11], [20, 21]], [[0.0, 1.0], [2.0, 0.0]], [[1.0, 1.0], [1.0, 1.0]], z2, z2) == [11, 20]
    assert walk(1, [[10, 11], [20, 21]], [[0.0, 1.0], [2.0, 0.0]], [[1.0, 1.0], [1.0, 1.0]], z2, z2, T=1e-6) == [11, 20]
    assert walk(3, [[10, 11]], [[0.0, 0.5]], [[1.0, 1.0]], lambda i: [1.0, 1.0], lambda i: [1.0, 1.0] if i == 10 else [0.0, 0.0]) == [10]
    pred = lambda i: [1.0] if i == 1 else [-1.0]  # noqa: E731
    succ = lambda i: [1.0] if i == 10 else [0.0]  # noqa: E731
    assert walk(2, [[1, 2], [10, 11]], [[1.0, 0.0], [0.0, 0.0]], [[1.0], [1.0]], pred, succ) == [1, 10]
    assert walk(1, [[1, 2], [10, 11]], [[0.0, 1.0], [0.0, 0.0]], [[1.0], [1.0]], pred, succ) == [2, 11]
    assert walk(1, [[30, 12, 20]], [[1.0, 1.0, 0.5]], [[0.0, 0.0]], z2, z2, T=0.0) == [12]
    assert walk(1, [[30, 12, 20]], [[1.0, 1.0, 0.5]], [[0.0, 0.0]], z2, z2) == [30]
