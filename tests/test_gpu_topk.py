"""Exact top-k drop-ins on the GPU against the oracle's restatement of the device contracts (the stable sort by
(value desc, id asc) with the dtype's NaN / signed-zero rules). Cases follow crates/cuda/tests/glue.rs:934-1160 and
crates/cuda/tests/nemotron_glue.rs:520-720."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from rexl3_amd import sampling as S
from rexl3_amd import workloads as W
from tests.common import Rng
from tests.gpu_util import dev, host, log, need_gpu

pytestmark = pytest.mark.gpu


def f32_to_bf16(v):
    return W.to_bf16_bits(np.asarray(v, dtype=np.float32))


def check16(logits_bits, rows, stride, valid, count, f16=False, what=""):
    t = dev(logits_bits.reshape(rows, stride).astype(np.uint16), torch.bfloat16 if not f16 else torch.float16)
    ids, vals = S.topk(t, count, valid=valid)
    ids, vals = host(ids), host(vals)
    for r in range(rows):
        wi, wv = O.topk_row(logits_bits.reshape(rows, stride)[r, :valid], count, O.DTYPE_F16 if f16 else O.DTYPE_BF16)
        assert np.array_equal(ids[r], wi), f"{what}: row {r} ids"
        assert np.array_equal(vals[r].view(np.uint32), wv.view(np.uint32)), f"{what}: row {r} vals"
        assert (ids[r] < valid).all()


def test_bf16_ties_nan_inf_chunk_edges():
    need_gpu()
    rng = Rng(11)
    vocab, rows = 248320, 4
    pool = f32_to_bf16([-2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0, 2.0])
    sel = np.array([rng.next() % 8 for _ in range(rows * vocab)])
    l = pool[sel].reshape(rows, vocab)
    for r in range(rows):
        l[r, 5], l[r, 12], l[r, 99], l[r, 100] = 0x8000, 0x7FC1, 0xFF80, 0x7F80
        for c in range(1, 4):
            l[r, c * 16384 - 1] = l[r, c * 16384] = 0x7F80
        l[r, vocab - 1] = 0x7F80
    for count in [1, 16, 28, 64]:
        log(f"bf16 ties count={count}")
        check16(l, rows, vocab, vocab, count, what=f"ties {count}")
    eq = np.full(vocab, f32_to_bf16([1.5])[0], dtype=np.uint16)
    for count in [1, 16, 28, 64]:
        ids, _ = S.topk(dev(eq.reshape(1, -1), torch.bfloat16), count)
        assert list(host(ids)[0]) == list(range(count))
    zz = np.where(np.arange(vocab) % 3 == 0, 0x8000, 0).astype(np.uint16)
    zz[vocab - 7] = f32_to_bf16([1e-30])[0]
    check16(zz, 1, vocab, vocab, 16, what="signed zeros")


def test_bf16_random_bits_sorted_and_odd_vocabs():
    need_gpu()
    rng = np.random.default_rng(12)
    vocab = 248320
    anyb = rng.integers(0, 1 << 16, 3 * vocab, dtype=np.uint64).astype(np.uint16)
    for count in [1, 16, 28, 64]:
        log(f"bf16 any-bits count={count}")
        check16(anyb, 3, vocab, vocab, count, what="any bits")
    asc = f32_to_bf16(np.arange(vocab, dtype=np.float32) * 1e-3)
    check16(asc, 1, vocab, vocab, 64, what="ascending")
    check16(asc[::-1].copy(), 1, vocab, vocab, 64, what="descending")
    for v, count in [(64, 64), (100, 64), (1001, 28), (16384, 16), (16385, 16), (2 * 16384 + 3, 64), (24576 + 5, 64), (17, 1),
                     (1, 1), (16, 16)]:
        l = f32_to_bf16((rng.integers(0, 9, 2 * v) * 0.25).astype(np.float32))
        check16(l, 2, v, v, count, what=f"vocab {v}")


def test_bf16_valid_never_reads_the_pad():
    need_gpu()
    rng = np.random.default_rng(21)
    for rows, stride, valid in [(3, 248192, 248144), (2, 1000, 987), (2, 20000, 19999), (2, 2 * 16384 + 64, 2 * 16384 + 1),
                                (2, 4096, 17)]:
        for count in [1, 16, 28, 64]:
            if count > valid:
                continue
            l = f32_to_bf16(rng.uniform(-6, 6, rows * stride).astype(np.float32)).reshape(rows, stride)
            for r in range(rows):
                for c in [0, valid - 1, valid // 2, min(16384, valid - 1)]:
                    l[r, c] = f32_to_bf16([40.0])[0]
                l[r, valid:] = np.array([0x7F7F, 0x7F80, 0x7FC1], dtype=np.uint16)[(np.arange(stride - valid) + r) % 3]
            check16(l.reshape(-1), rows, stride, valid, count, what=f"valid {valid}")


def test_f16_contract():
    need_gpu()
    rng = np.random.default_rng(31)
    vocab = 70000
    anyb = rng.integers(0, 1 << 16, 2 * vocab, dtype=np.uint64).astype(np.uint16)
    for count in [1, 8, 40, 64]:
        check16(anyb, 2, vocab, vocab, count, f16=True, what="f16 any bits")


def nemo_kinds(rng, vocab):
    def nanp():
        r = int(rng.integers(0, 1 << 32))
        return np.array([((r & 1) << 31) | 0x7F800000 | ((r >> 1) & 0x7FFFFF) | 1], dtype=np.uint32).view(np.float32)[0]
    out = []
    out.append(rng.uniform(-8, 8, vocab).astype(np.float32))
    out.append(np.array([-1.0, -0.0, 0.0, 0.5, 2.0, 2.0, np.uint32(1).view(np.float32)], dtype=np.float32)[rng.integers(0, 7, vocab)])
    x = rng.uniform(-5, 5, vocab).astype(np.float32)
    x[rng.integers(0, 10, vocab) == 0] = nanp()
    out.append(x)
    out.append(np.full(vocab, nanp(), dtype=np.float32))
    out.append(np.array([-np.inf, np.inf, np.nan, 1.0, -1.0, 0.0, -np.inf], dtype=np.float32)[rng.integers(0, 7, vocab)])
    out.append(np.arange(vocab, dtype=np.float32))
    out.append(-np.arange(vocab, dtype=np.float32))
    out.append(np.full(vocab, 3.5, dtype=np.float32))
    z = np.zeros(vocab, dtype=np.float32)
    k = rng.integers(0, 4, vocab)
    z[k == 1] = -0.0
    z[k == 2] = np.uint32(3).view(np.float32)
    z[k == 3] = -np.uint32(2).view(np.float32)
    out.append(z)
    sp = (rng.uniform(-1, 1, vocab) * 1e-3).astype(np.float32)
    sp[rng.integers(0, vocab, max(3, vocab // 400))] = rng.uniform(10, 1e30, max(3, vocab // 400)).astype(np.float32)
    out.append(sp)
    return out


def check_f32(data, count, blocks=None, what=""):
    rows, vocab = data.shape
    ids, vals = S.topk(dev(data), count, blocks=blocks)
    ids, vals = host(ids), host(vals)
    for r in range(rows):
        wi, wv = O.topk_row(data[r], count, O.DTYPE_F32)
        assert np.array_equal(ids[r], wi), f"{what} row {r}"
        assert np.array_equal(vals[r].view(np.uint32), wv.view(np.uint32)), f"{what} row {r} value bits"
    return ids, vals


def test_f32_every_kind_and_shape():
    need_gpu()
    rng = np.random.default_rng(404)
    for rows, count in [(64, 40), (64, 64), (7, 1), (1, 64), (3, 17)]:
        kinds = nemo_kinds(rng, 131072)
        data = np.stack([kinds[r % len(kinds)] for r in range(rows)])
        log(f"f32 rows={rows} count={count}")
        check_f32(data, count, what=f"rows {rows} count {count}")
    for vocab in [1003, 5000, 4099, 2049, 70, 64, 33, 13]:
        kinds = nemo_kinds(rng, vocab)
        for count in [1, 2, 40, 63, 64]:
            if count > vocab:
                continue
            data = np.stack([kinds[r % len(kinds)] for r in range(7)])
            check_f32(data, count, what=f"vocab {vocab} count {count}")


def test_f32_rows_are_invariant_and_blocks_do_not_matter():
    need_gpu()
    rng = np.random.default_rng(505)
    kinds = nemo_kinds(rng, 131072)
    data = np.stack([kinds[r % len(kinds)] for r in range(64)])
    ids, vals = check_f32(data, 40)
    for b in [1, 3, 16]:
        i2, v2 = check_f32(data[:7], 40, blocks=b)
        assert np.array_equal(i2, ids[:7]) and np.array_equal(v2.view(np.uint32), vals[:7].view(np.uint32))


def test_refusals():
    need_gpu()
    from rexl3_amd import _lib
    l = dev(np.zeros(200, dtype=np.float32))
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    ids = torch.zeros(128, dtype=torch.int32, device="cuda")
    vals = torch.zeros(128, dtype=torch.float32, device="cuda")
    lib = _lib.load()
    P = lambda t: t.data_ptr()  # noqa: E731
    for vocab, count in [(100, 0), (100, 65), (10, 11)]:
        assert lib.gb_nemo_glue_topk(P(l), 1, vocab, count, 1, P(ws), 1 << 20, P(ids), P(vals), None) == 1
    assert lib.gb_nemo_glue_topk(P(l), 0, 100, 5, 1, P(ws), 1 << 20, P(ids), P(vals), None) == 0
    need = 1 * 1 * 8 * 5 * 8
    assert lib.gb_nemo_glue_topk(P(l), 1, 100, 5, 1, P(ws), need - 1, P(ids), P(vals), None) == 1
    assert lib.gb_nemo_glue_topk(P(l), 1, 100, 5, 1, P(ws), need, P(ids), P(vals), None) == 0
    torch.cuda.synchronize()
    assert list(ids.cpu().numpy()[:5]) == [0, 1, 2, 3, 4]
    b = dev(np.zeros(200, dtype=np.uint16), torch.bfloat16)
    assert lib.gb_topk_valid(P(b), 2, 100, 101, 10, P(ids), P(vals), P(ws), 1 << 20, None) == 1
    assert lib.gb_topk_valid(P(b), 2, 100, 10, 11, P(ids), P(vals), P(ws), 1 << 20, None) == 1
    assert lib.gb_topk_valid(P(b), 2, 100, 100, 65, P(ids), P(vals), P(ws), 1 << 20, None) == 1
    assert lib.gb_topk_valid(P(b), 2, 100, 0, 1, P(ids), P(vals), P(ws), 1 << 20, None) == 1
    assert lib.gb_topk_valid(P(b), 2, 100, 100, 10, P(ids), P(vals), P(ws), 8, None) == 1
    assert lib.gb_topk_valid_workspace_bytes(1, 100, 65) == 0
    assert lib.gb_topk_valid(P(b), 2, 100, 100, 10, P(ids), P(vals), P(ws), 1 << 20, None) == 0
    torch.cuda.synchronize()


def test_ling_single_launch_f16_matches_two_launch_and_oracle():
    """gb_ling_topk_f16 (one launch, the last chunk block merges) gives gb_glm_topk_f16's ids and values; its counters
    reset themselves across calls of varying row counts on one workspace (crates/cuda/tests/ling_kda_proj_fused_ab.rs:
    3404-3470 checks the same two properties); more than 64 rows is refused."""
    need_gpu()
    rng = np.random.default_rng(41)
    ws = torch.zeros(S._lib.load().gb_ling_topk_f16_workspace_bytes(64, 151_936, 64), dtype=torch.uint8, device="cuda")
    for rows, stride, valid, count in [(1, 151_936, 151_936, 64), (7, 32_768, 32_000, 40), (64, 151_936, 151_900, 50),
                                       (3, 100, 97, 16), (33, 16_384, 16_384, 1), (64, 65_540, 65_540, 32), (2, 5, 5, 5)]:
        bits = rng.integers(0, 1 << 16, rows * stride, dtype=np.uint64).astype(np.uint16)
        bits[rng.choice(rows * stride, rows * stride // 50, replace=False)] = 0x3C00  # ties at 1.0
        bits = bits.reshape(rows, stride)
        bits[:, valid:] = 0x7C00  # +inf past valid: never read
        t = dev(bits, torch.float16)
        log(f"ling topk rows={rows} stride={stride} valid={valid} count={count}")
        gi, gv = S.topk_f16_single_launch(t, count, valid=valid, workspace=ws)
        wi, wv = S.topk(t, count, valid=valid)
        gi, gv, wi, wv = host(gi), host(gv), host(wi), host(wv)
        assert np.array_equal(gi, wi)
        assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32))
        for r in range(0, rows, max(1, rows // 4)):
            oi, ov = O.topk_row(bits[r, :valid], count, O.DTYPE_F16)
            assert np.array_equal(gi[r], oi) and np.array_equal(gv[r].view(np.uint32), ov.view(np.uint32))
    assert int(host(ws[:256]).astype(np.uint8).sum()) == 0  # every call left its counters at zero
    big = dev(np.zeros((65, 64), dtype=np.uint16), torch.float16)
    with pytest.raises(S._lib.GbsError):
        S.topk_f16_single_launch(big, 8, workspace=torch.zeros(1 << 16, dtype=torch.uint8, device="cuda"))
