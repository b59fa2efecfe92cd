"""The extended pipeline (gbs_sample_rows) on the GPU against the oracle: token ids, greedy ids and statuses bit-exact;
probabilities within 1e-5 relative; log-probabilities within 1e-5 absolute, i.e. the probability they stand for within 1e-5
relative (the oracle computes them in double, the device sums the softmax denominator in f32)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from rexl3_amd import sampling as S
from rexl3_amd import workloads as W
from tests.gpu_util import dev, host, log, need_gpu

pytestmark = pytest.mark.gpu
RTOL = 1e-5
LOGPROB_ATOL = 1e-5


def run_both(cfg, kmax=64, logprobs=True):
    x = cfg["logits"]
    is_bf16 = cfg["dtype"] == "bf16"
    t = dev(x, torch.bfloat16) if is_bf16 else dev(x)
    counts = None if cfg["counts"] is None else dev(cfg["counts"])
    mask = None if cfg["mask"] is None else dev(cfg["mask"])
    u = dev(cfg["uniforms"])
    g = S.sample_rows(t, cfg["params"], u, counts, mask, kmax=kmax, logprobs=logprobs)
    g = {k: host(v) for k, v in g.items()}
    w = O.sample_rows(x, O.DTYPE_BF16 if is_bf16 else O.DTYPE_F32, cfg["counts"], cfg["mask"], cfg["params"], cfg["uniforms"],
                      threads=8)
    return g, w


def compare(g, w, what):
    assert np.array_equal(g["status"], w["status"]), f"{what}: status {np.nonzero(g['status'] != w['status'])[0][:10]}"
    bad = np.nonzero(g["ids"] != w["ids"])[0]
    assert bad.size == 0, f"{what}: ids differ at rows {bad[:10]} got {g['ids'][bad[:5]]} want {w['ids'][bad[:5]]}"
    ok = w["status"] == 0
    assert np.array_equal(g["greedy"][ok], w["greedy"][ok]), what
    np.testing.assert_allclose(g["probs"][ok], w["probs"][ok], rtol=RTOL, atol=0, err_msg=what)
    if "logprobs" in g:
        fin = ok & np.isfinite(w["logprobs"])
        # an absolute error of 1e-5 in a log-probability is a relative error of 1e-5 in the probability it stands for
        np.testing.assert_allclose(g["logprobs"][fin], w["logprobs"][fin], rtol=0, atol=LOGPROB_ATOL, err_msg=what)


def test_config1_single_row():
    need_gpu()
    for seed in range(1, 6):
        cfg = W.config1(seed)
        g, w = run_both(cfg)
        compare(g, w, f"config1 seed {seed}")


def test_config2_bf16_batched():
    need_gpu()
    cfg = W.config2()
    g, w = run_both(cfg)
    compare(g, w, "config2")
    t0 = cfg["params"]["temperature"] == 0
    assert np.array_equal(g["ids"][t0], g["greedy"][t0])


def test_config4_grammar_masks():
    need_gpu()
    cfg = W.config4(rows=64)
    g, w = run_both(cfg)
    compare(g, w, "config4")
    # rows that allow exactly one token return it for any uniform
    m = cfg["mask"]
    for r in range(8):
        bits = np.unpackbits(m[r].view(np.uint8), bitorder="little")
        assert g["ids"][r] == int(np.nonzero(bits)[0][0])
        assert g["probs"][r] == 1.0


def test_northstar_pipeline_penalties_and_mask():
    need_gpu()
    cfg = W.northstar(rows=32)
    log("northstar rows=32")
    g, w = run_both(cfg)
    compare(g, w, "northstar")


def test_edge_rows():
    need_gpu()
    rng = np.random.default_rng(9)
    V, B = 5000, 16
    x = rng.standard_normal((B, V)).astype(np.float32)
    words = (V + 31) // 32
    mask = np.full((B, words), 0xFFFFFFFF, dtype=np.uint32)
    p = S.row_params(B, temperature=0.9, top_p=0.8, min_p=0.1, top_k=30, repetition=1.2, presence=0.2, frequency=0.1)
    u = W.uniforms_f32(5, B)
    counts = rng.integers(0, 3, (B, V)).astype(np.int32)
    mask[0] = 0                       # nothing allowed
    x[1, 77] = np.nan                 # NaN allowed -> NanLogit
    x[2, 77] = np.nan
    mask[2, 77 // 32] &= ~np.uint32(1 << (77 % 32))  # NaN masked out -> fine
    p[3]["temperature"] = 0.0         # greedy
    p[4]["top_k"] = 65                # breaks kmax
    p[5]["temperature"] = -1.0        # invalid
    u[6] = 1.0                        # invalid uniform
    x[7, 100] = np.inf                # +inf maximum
    x[7, 4000] = np.inf
    mask[8] = 0
    mask[8, 3] = 0b1011               # three allowed tokens < top_k
    x[9, :] = 1.25                    # all equal
    counts[9] = 0
    p[10]["top_p"] = 1.0
    p[10]["min_p"] = 0.0
    u[11] = np.float32(0.99999994)    # largest uniform
    u[12] = 0.0
    x[13] = -x[13] * 1e-3             # tiny spread
    x[14, :] = -0.0
    x[14, 10] = 0.0
    p[15]["top_k"] = 1
    cfg = dict(logits=x, dtype="f32", params=p, uniforms=u, counts=counts, mask=mask)
    g, w = run_both(cfg)
    # row 4 breaks the kmax promise (top_k 65 > 64): the single-pass path refuses it; the oracle has no such limit
    assert g["status"][4] == 3 and g["ids"][4] == -1 and w["status"][4] == 0
    for k in ("status", "ids", "greedy", "probs", "logprobs"):
        g[k] = np.delete(g[k], 4)
        w[k] = np.delete(w[k], 4)
    compare(g, w, "edges")
    assert list(g["status"][:6]) == [1, 2, 0, 0, 3, 3]


def test_kmax_and_rows_invariance():
    need_gpu()
    cfg = W.config4(rows=24)
    g1, w = run_both(cfg, kmax=64)
    compare(g1, w, "kmax 64")
    x, u = dev(cfg["logits"]), dev(cfg["uniforms"])
    m = dev(cfg["mask"])
    for r in [0, 9, 23]:
        one = S.sample_rows(x[r:r + 1].contiguous(), cfg["params"][r:r + 1], u[r:r + 1].contiguous(), None, m[r:r + 1].contiguous())
        assert host(one["ids"])[0] == g1["ids"][r]


# ---------------------------------------------------------------- the full-distribution path (kmax == 0)

def test_full_path_config3_penalties_top_p_over_the_whole_vocabulary():
    need_gpu()
    cfg = W.config3(rows=16)
    log("config3 rows=16 full path")
    g, w = run_both(cfg, kmax=0)
    compare(g, w, "config3")


def test_full_path_equals_fast_path_and_oracle():
    need_gpu()
    for cfg, what in [(W.config1(3), "c1"), (W.config2(), "c2"), (W.config4(rows=32), "c4"), (W.northstar(rows=16), "ns")]:
        g0, w = run_both(cfg, kmax=0)
        compare(g0, w, what + " full")
        g1, _ = run_both(cfg, kmax=64)
        assert np.array_equal(g0["ids"], g1["ids"]), what


def test_full_path_large_top_k_ties_and_min_p():
    need_gpu()
    rng = np.random.default_rng(17)
    B, V = 24, 70001
    x = (rng.integers(0, 12, (B, V)) * 0.25).astype(np.float32)  # massive exact ties
    x[3] = 1.0                                                      # one value everywhere
    x[4] = rng.standard_normal(V).astype(np.float32) * 4
    x[5, ::7] = -np.inf
    p = S.row_params(B, temperature=0.9, top_p=0.7, min_p=0.0, top_k=0)
    p["top_k"][:8] = [100, 1000, 5000, 70001, 70000, 3, 65, 256]
    p["min_p"][8:12] = [0.1, 0.5, 1.0, 0.01]
    p["top_p"][12:16] = [1.0, 0.0, 0.999, 0.01]
    p["temperature"][16:18] = [0.05, 3.0]
    u = W.uniforms_f32(77, B)
    cfg = dict(logits=x, dtype="f32", params=p, uniforms=u, counts=None, mask=None)
    g, w = run_both(cfg, kmax=0)
    compare(g, w, "ties")



def test_log_probabilities_at_huge_magnitudes():
    """Logits around 1e6 and -1e5: the log-sum-exp takes each difference to the running maximum before scaling by 1/T,
    which is exact near the maximum at any magnitude (both paths, one block per row and split)."""
    need_gpu()
    rng = np.random.default_rng(31)
    for rows in (4, 300):
        V = 20_000
        x = (rng.standard_normal((rows, V)) * 1.5).astype(np.float32)
        x[0::4] *= 1e6
        x[1::4] -= 1e5
        x[2::4] += 3e4
        p = S.row_params(rows, temperature=0.8, top_p=0.9, top_k=40)
        cfg = dict(logits=x, dtype="f32", params=p, uniforms=W.uniforms_f32(31, rows), counts=None, mask=None)
        for kmax in (64, 0):
            log(f"huge magnitudes rows={rows} kmax={kmax}")
            g, w = run_both(cfg, kmax=kmax)
            compare(g, w, f"huge magnitudes rows={rows} kmax={kmax}")


def test_full_path_split_rows_with_extreme_shapes():
    """The split full path (19 blocks per row) on rows with extreme shapes: a maximum far above the rest, leading tiles
    and a whole block without an allowed token, a crossing bin of far more than 2048 tokens (the single-block path
    takes the row inside the collection launch), one allowed token, huge magnitudes, sharp and flat temperatures."""
    need_gpu()
    rng = np.random.default_rng(23)
    B, V = 12, 154_880                         # 19 blocks of 2 tiles per row
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    words = (V + 31) // 32
    mask = np.full((B, words), 0xFFFFFFFF, dtype=np.uint32)
    counts = rng.integers(0, 2, (B, V)).astype(np.int32)
    p = S.row_params(B, temperature=0.8, top_p=0.9, min_p=0.0, top_k=0, repetition=1.1, presence=0.5, frequency=0.3)
    x[1, 8191] = 60.0                           # a maximum far above every other value
    mask[2, : 8192 // 32] = 0                   # block 0 of row 2: no allowed token
    mask[2, 8192 // 32: (8192 + 4096) // 32] = 0  # block 1: its first tile without an allowed token
    x[3] = (rng.standard_normal(V) * 1e-4).astype(np.float32)  # flat: far more than 2048 tokens in the crossing bin
    counts[3] = 0
    p[4]["top_p"] = 0.01
    p[5]["top_p"] = 0.999
    p[6]["min_p"] = 0.2
    mask[7] = 0
    mask[7, 4000] = 1 << 5                      # one allowed token
    x[8] = x[8] * 1e6                           # huge magnitudes
    x[9] = x[9] - 1e5
    p[10]["temperature"] = 0.05                 # sharp
    p[11]["temperature"] = 5.0                  # flat-ish
    cfg = dict(logits=x, dtype="f32", params=p, uniforms=W.uniforms_f32(29, B), counts=counts, mask=mask)
    log("full path extreme rows: 12 x 154880")
    g, w = run_both(cfg, kmax=0)
    compare(g, w, "extreme rows")


# ---------------------------------------------------------------- full batches (one block per row)

def test_northstar_full_size_and_repeated_launches():
    """The north star at its full size (256 rows x 151,936); every launch leaves the workspace's counters at zero, so
    repeated launches give the same results."""
    need_gpu()
    cfg = W.northstar()
    log("northstar 256 x 151936")
    g, w = run_both(cfg)
    compare(g, w, "northstar full")
    t = dev(cfg["logits"])
    c, m, u = dev(cfg["counts"]), dev(cfg["mask"]), dev(cfg["uniforms"])
    for rep in range(3):
        again = S.sample_rows(t, cfg["params"], u, c, m, kmax=64, logprobs=True)
        assert np.array_equal(host(again["ids"]), g["ids"]), rep
        assert np.array_equal(host(again["status"]), g["status"]), rep
        np.testing.assert_allclose(host(again["probs"]), g["probs"], rtol=0, atol=0)


def test_more_rows_than_cus_and_short_rows():
    """More rows than CUs, and rows of few wave-steps (fewer than a block has waves, a ragged last wave-step)."""
    need_gpu()
    for rows, vocab in [(300, 151_936), (600, 40_000), (512, 5_000), (257, 36_868)]:
        cfg = W.northstar(seed=rows, rows=rows, vocab=vocab)
        log(f"northstar rows={rows} vocab={vocab}")
        g, w = run_both(cfg)
        compare(g, w, f"rows {rows} vocab {vocab}")


def test_full_batches_bf16_masks_and_edge_rows():
    """bf16 logits and the grammar-mask workload at full batch sizes, plus the edge rows of test_edge_rows placed inside a
    full batch."""
    need_gpu()
    cfg = W.config2(rows=320)
    log("config2 bf16 rows=320")
    g, w = run_both(cfg)
    compare(g, w, "config2 320 rows")
    cfg = W.config4(rows=256)
    log("config4 rows=256")
    g, w = run_both(cfg)
    compare(g, w, "config4 256 rows")
    # edge rows: nothing allowed, NaN, T=0, invalid parameters, +inf, ties, extreme uniforms, among ordinary rows
    rng = np.random.default_rng(19)
    B, V = 272, 20_000
    x = rng.standard_normal((B, V)).astype(np.float32)
    mask = np.full((B, (V + 31) // 32), 0xFFFFFFFF, dtype=np.uint32)
    counts = rng.integers(0, 3, (B, V)).astype(np.int32)
    p = S.row_params(B, temperature=0.9, top_p=0.8, min_p=0.1, top_k=30, repetition=1.2, presence=0.2, frequency=0.1)
    u = W.uniforms_f32(7, B)
    mask[0] = 0
    x[1, 77] = np.nan
    x[2, 19_999] = np.nan
    mask[2, 19_999 // 32] &= ~np.uint32(1 << (19_999 % 32))
    p[3]["temperature"] = 0.0
    p[5]["temperature"] = -1.0
    u[6] = 1.0
    x[7, 100] = np.inf
    x[7, 15_000] = np.inf
    x[9, :] = 1.25
    counts[9] = 0
    u[11] = np.float32(0.99999994)
    u[12] = 0.0
    x[14, :] = -0.0
    x[14, 10] = 0.0
    p[15]["top_k"] = 1
    p[200]["top_k"] = 64
    cfg = dict(logits=x, dtype="f32", params=p, uniforms=u, counts=counts, mask=mask)
    g, w = run_both(cfg)
    compare(g, w, "edge rows in a full batch")
    assert list(g["status"][:3]) == [1, 2, 0] and g["status"][5] == 3 and g["status"][6] == 3


def test_workspace_reused_across_row_counts():
    """One workspace serves launches of different row counts: the counters that must be zero between launches sit at
    fixed per-row offsets, so partial lists written by one shape never land where another shape counts."""
    need_gpu()
    big = W.northstar(seed=31, rows=300, vocab=30_000)
    small = W.northstar(seed=32, rows=8, vocab=30_000)
    for cfg, what in [(big, "300 rows"), (small, "8 rows (split kernel)"), (big, "300 rows again"),
                      (W.config4(rows=3), "3 rows"), (big, "300 rows a third time")]:
        log(what)
        g, w = run_both(cfg)
        compare(g, w, what)


def test_full_path_binned_cut_edges():
    """The full path's binned top-p cut and its fallbacks: a crossing bin of exactly 2048 tokens (collected) and of 2049
    (the radix path), +inf in a row and a temperature whose 1/T overflows (the radix path), top-k with top-p (the
    radix path), min-p with top-p, and config 3 at its full size."""
    need_gpu()
    rng = np.random.default_rng(23)
    B, V = 12, 50_000
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    for r, n in [(0, 2048), (1, 2049), (2, 2047)]:
        x[r] = -30.0
        x[r, rng.choice(V, n, replace=False)] = 3.0
    x[3, rng.choice(V, 4000, replace=False)] = 5.0 + rng.uniform(0, 1e-3, 4000).astype(np.float32)
    x[4, 123] = np.inf
    p = S.row_params(B, temperature=0.9, top_p=0.6, min_p=0.0, top_k=0)
    p["temperature"][5] = 1e-39
    p["top_k"][6] = 40
    p["min_p"][7] = 0.05
    p["top_p"][8] = 0.999999
    p["top_p"][9] = 1e-7
    u = W.uniforms_f32(29, B)
    cfg = dict(logits=x, dtype="f32", params=p, uniforms=u, counts=None, mask=None)
    g, w = run_both(cfg, kmax=0)
    compare(g, w, "binned edges")
    cfg = W.config3()
    log("config3 full size, full path")
    g, w = run_both(cfg, kmax=0)
    compare(g, w, "config3 full size")


def test_full_path_collection_window_edges():
    """The split full path's collection window, made from pass 0's counts on a grid set by the row's first tile: a first
    tile far below the row's maximum (the grid's top bin holds most of the row), a first tile with no allowed token, a
    maximum in the first tile far above the rest (the cut at the top), a flat row (the window overflows: the single-block
    path), min-p with a floor, penalties and masks, f32 and bf16."""
    need_gpu()
    rng = np.random.default_rng(41)
    B, V = 10, 61_440
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    x[0, :4096] -= 30.0
    x[1, :4096] = -np.inf
    x[2, 17] = 40.0
    x[3] = 0.25
    x[4, 5000:5100] = 9.0
    counts = np.zeros((B, V), dtype=np.int32)
    counts[5:8, rng.choice(V, 3000, replace=False)] = rng.integers(1, 5, 3000)
    mask = np.full((B, (V + 31) // 32), 0xFFFFFFFF, dtype=np.uint32)
    mask[6, :128] = 0          # the first tile masked
    mask[7, ::3] = 0x0F0F0F0F
    p = S.row_params(B, temperature=0.8, top_p=0.9, min_p=0.0, top_k=0, repetition=1.1, presence=0.5, frequency=0.3)
    p["min_p"][8] = 0.02
    p["top_p"][9] = 0.3
    u = W.uniforms_f32(43, B)
    for dtype in ("f32", "bf16"):
        xx = x if dtype == "f32" else (x.view(np.uint32) >> 16).astype(np.uint16)
        cfg = dict(logits=xx, dtype=dtype, params=p, uniforms=u, counts=counts, mask=mask)
        log(f"window edges {dtype}")
        g, w = run_both(cfg, kmax=0)
        compare(g, w, f"window edges {dtype}")


def test_full_and_fast_paths_alternate_on_one_workspace():
    """The fast path (kmax 64) and the split full path (kmax 0, fewer rows than CUs: several blocks per row, three
    launches with last-block hand-offs) share one workspace; their counters sit in one control region and every
    launch leaves them zero, so alternating launches stay exact. Also the split path at one row (38 blocks)."""
    need_gpu()
    cases = [(W.config3(rows=16), 0, "c3 16 rows full"), (W.northstar(seed=3, rows=40, vocab=60_000), 64, "ns 40 rows fast"),
             (W.config1(5), 0, "c1 one row full"), (W.config4(rows=16), 64, "c4 16 rows fast"),
             (W.northstar(seed=4, rows=40, vocab=60_000), 0, "ns 40 rows full"), (W.config3(rows=16), 0, "c3 16 rows full again")]
    for cfg, kmax, what in cases:
        log(what)
        g, w = run_both(cfg, kmax=kmax)
        compare(g, w, what)


@pytest.mark.parametrize("kmax", [64, 0])
@pytest.mark.parametrize("vocab,pad", [(151_936, 64), (50_001, 7)])
@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_padded_rows_stride_above_vocab(dtype, vocab, pad, kmax):
    """The lm_head's padded layout (crates/cuda/csrc/glue.cu:1084-1098 reads columns [0, valid) of rows `stride` apart):
    logits [rows, vocab + pad] whose pad columns hold NaN or +inf. A kernel that read one of them would report NanLogit
    or pick it; the results must equal the oracle's on the unpadded rows."""
    need_gpu()
    rows = 16
    cfg = W.northstar(seed=31 + pad, rows=rows, vocab=vocab)
    if kmax == 0:
        cfg["params"]["top_k"][::2] = 0  # the full-distribution path serves any top_k
    x = cfg["logits"]
    if dtype == "bf16":
        x = W.to_bf16_bits(x)
        full = np.empty((rows, vocab + pad), np.uint16)
        full[:, vocab:] = np.where(np.arange(rows)[:, None] % 2 == 0, 0x7FC0, 0x7F80)
    elif dtype == "f16":
        x = x.astype(np.float16).view(np.uint16)
        full = np.empty((rows, vocab + pad), np.uint16)
        full[:, vocab:] = np.where(np.arange(rows)[:, None] % 2 == 0, 0x7E00, 0x7C00)
    else:
        full = np.empty((rows, vocab + pad), np.float32)
        full[:, vocab:] = np.where(np.arange(rows)[:, None] % 2 == 0, np.nan, np.inf)
    full[:, :vocab] = x
    log(f"padded rows dtype={dtype} vocab={vocab} pad={pad} kmax={kmax}")
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}.get(dtype)
    t = dev(full, tdt) if tdt is not None else dev(full)
    g = S.sample_rows(t, cfg["params"], dev(cfg["uniforms"]), dev(cfg["counts"]), dev(cfg["mask"]), kmax=kmax, logprobs=True,
                      vocab=vocab)
    g = {k: host(v) for k, v in g.items()}
    w = O.sample_rows(x, {"bf16": O.DTYPE_BF16, "f16": O.DTYPE_F16}.get(dtype, O.DTYPE_F32), cfg["counts"], cfg["mask"],
                      cfg["params"], cfg["uniforms"], threads=8)
    assert (w["status"] == 0).all()
    compare(g, w, f"padded {dtype} {vocab}+{pad} kmax {kmax}")


def test_wrapper_rejects_mis_shaped_operands():
    """The host mirror checks operand shapes before any launch: a short uniforms vector or a mask of the wrong width
    would make the kernel read past its allocation."""
    need_gpu()
    cfg = W.northstar(seed=2, rows=4, vocab=4096)
    x, c, m, u = dev(cfg["logits"]), dev(cfg["counts"]), dev(cfg["mask"]), dev(cfg["uniforms"])
    with pytest.raises(ValueError):
        S.sample_rows(x, cfg["params"], u[:3], c, m)
    with pytest.raises(ValueError):
        S.sample_rows(x, cfg["params"], u, c, m[:, :-1].contiguous())
    with pytest.raises(ValueError):
        S.sample_rows(x, cfg["params"], u, c.to(torch.int64), m)
    with pytest.raises(ValueError):
        S.sample_rows(x, cfg["params"][:3], u, c, m)


def test_workspaces_are_per_stream():
    """Two streams get two workspaces (their arrival counters must not be shared by overlapping calls), and both give
    the oracle's results."""
    need_gpu()
    cfg = W.northstar(seed=4, rows=8, vocab=8192)
    x, c, m, u = dev(cfg["logits"]), dev(cfg["counts"]), dev(cfg["mask"]), dev(cfg["uniforms"])
    w = O.sample_rows(cfg["logits"], O.DTYPE_F32, cfg["counts"], cfg["mask"], cfg["params"], cfg["uniforms"])
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for s in (s1, s2):
        with torch.cuda.stream(s):
            outs.append(S.sample_rows(x, cfg["params"], u, c, m))
    torch.cuda.synchronize()
    keys = [k for k in S.WORKSPACE.keys() if k[2] == "sample"]
    assert {s1.cuda_stream, s2.cuda_stream} <= {k[1] for k in keys}
    for o in outs:
        assert np.array_equal(host(o["ids"]), w["ids"])


@pytest.mark.parametrize("kmax", [64, 0])
def test_f16_logits_edge_values(kmax):
    """fp16 logits (the lm_head's half-precision output) widened exactly: subnormals, +-0 ties, the largest finite
    values, -inf (a banned token), and a row with a NaN (status NanLogit), against the oracle."""
    need_gpu()
    rows, vocab = 12, 20_000
    cfg = W.northstar(seed=17, rows=rows, vocab=vocab)
    x = cfg["logits"].astype(np.float16)
    x[0, :50] = np.float16(6.0e-8)                    # subnormals
    x[1, :] = np.float16(0.0)
    x[1, ::3] = np.float16(-0.0)                      # ties of +0 and -0 everywhere
    x[2, 123] = np.float16(65504.0)                   # the largest finite value
    x[3, 77] = np.float16(-np.inf)
    x[4, 5] = np.float16(np.nan)
    cfg["mask"][4, 0] |= np.uint32(1 << 5)             # allowed: a NaN at a banned position is ignored
    if kmax == 0:
        cfg["params"]["top_k"][::3] = 0
    bits = x.view(np.uint16)
    g = S.sample_rows(dev(bits, torch.float16), cfg["params"], dev(cfg["uniforms"]), dev(cfg["counts"]), dev(cfg["mask"]), kmax=kmax,
                      logprobs=True)
    g = {k: host(v) for k, v in g.items()}
    w = O.sample_rows(bits, O.DTYPE_F16, cfg["counts"], cfg["mask"], cfg["params"], cfg["uniforms"], threads=8)
    assert w["status"][4] == O.ROW_NAN_LOGIT
    compare(g, w, f"f16 kmax {kmax}")


DEFER_OFFSET = 3 * 65536 * 4  # the per-row dispatch flags in the workspace's control region


def mixed_batch(rows, vocab, seed=23):
    """A north-star batch whose rows mix top-k settings as an engine's decode round does: most rows top_k 50, some
    top_k 0 (top-p over the whole vocabulary) on peaked rows, some top_k 100, and some top_k 0 rows whose logits are
    flat (config 3's N(0, 1.5^2)), where the top-p cut lies far beyond any 64 candidates."""
    cfg = W.northstar(seed=seed, rows=rows, vocab=vocab)
    p = cfg["params"]
    peaked0 = np.arange(1, rows, 10)
    k100 = np.setdiff1d(np.arange(4, rows, 16), peaked0)
    flat = np.setdiff1d(np.setdiff1d(np.arange(7, rows, 21), peaked0), k100)
    p["top_k"][peaked0] = 0
    p["top_k"][k100] = 100
    p["top_k"][flat] = 0
    p["min_p"][k100[::2]] = 0.02
    x = cfg["logits"]
    x[flat] = (W.normals(seed + 1, len(flat) * vocab) * 1.5).astype(np.float32).reshape(len(flat), vocab)
    # the peaked rows: five dominant tokens (allowed, no history) that hold nearly all the mass, the top-p cut among them
    rng = np.random.default_rng(seed)
    for r in peaked0:
        ids = rng.choice(vocab, 5, replace=False)
        x[r, ids] = [24.0, 23.6, 23.3, 23.0, 22.8]
        cfg["counts"][r, ids] = 0
        cfg["mask"][r, ids // 32] |= (np.uint32(1) << (ids % 32).astype(np.uint32))
    return cfg, peaked0, k100, flat


@pytest.mark.parametrize("rows", [256, 40])  # one block per row; split rows
def test_per_row_dispatch_mixed_batch(rows):
    need_gpu()
    vocab = 151_936 if rows == 256 else 60_000
    cfg, peaked0, k100, flat = mixed_batch(rows, vocab)
    log(f"mixed batch rows={rows}")
    g, w = run_both(cfg, kmax=S.KMAX_MIXED)
    compare(g, w, f"mixed {rows}")
    # the same ids as the full-distribution path
    g0, _ = run_both(cfg, kmax=0)
    assert np.array_equal(g["ids"], g0["ids"]) and np.array_equal(g["status"], g0["status"])
    # which rows the single pass left over: the flat ones, not the peaked top_k 0 rows nor the top-k rows
    ws = S.WORKSPACE.get(torch.device("cuda", torch.cuda.current_device()), "sample", 0)
    flags = host(ws[DEFER_OFFSET:DEFER_OFFSET + 4 * rows].view(torch.int32))
    allowed = np.unpackbits(cfg["mask"].view(np.uint8), axis=1, bitorder="little")[:, :vocab].sum(axis=1)
    wide = flat[allowed[flat] >= 1000]  # a flat row with a handful of allowed tokens is exact in the single pass
    assert len(wide) > 0 and flags[wide].all(), (wide, flags[wide])
    assert not flags[peaked0].any(), (peaked0, flags[peaked0])
    in_range = np.setdiff1d(np.arange(rows), np.concatenate([peaked0, k100, flat]))
    assert not flags[in_range].any()
    log(f"deferred rows {np.nonzero(flags)[0].tolist()}; top_k 100 rows deferred {int(flags[k100].sum())} of {len(k100)}")


def test_per_row_dispatch_edge_rows():
    """Open rows at the edges: fewer allowed tokens than the list holds (the list is the whole row, exact), min-p alone
    (no top-p) cutting inside the list or not, T = 0, and an open row with NaN."""
    need_gpu()
    rows, vocab = 16, 30_000
    cfg = W.northstar(seed=29, rows=rows, vocab=vocab)
    p = cfg["params"]
    p["top_k"][:] = 0
    m = cfg["mask"]
    m[0] = 0
    m[0, 0] = 0xFFFFFFFF
    m[0, 1] = 0x7FFFFFFF            # 63 allowed tokens: the list holds them all
    m[1] = 0
    m[1, 0] = 0x0000FFFF            # 16 allowed
    p["top_p"][2:6] = 1.0           # min-p alone
    p["min_p"][2:4] = 0.2           # cuts inside the list on a peaked row
    p["min_p"][4:6] = 1e-9          # keeps far more than 64: the full path
    p["temperature"][6] = 0.0
    cfg["logits"][7, 11] = np.nan
    m[7, 0] |= np.uint32(1 << 11)   # allowed: status NanLogit
    g, w = run_both(cfg, kmax=S.KMAX_MIXED)
    assert w["status"][7] == O.ROW_NAN_LOGIT
    compare(g, w, "open edge rows")
    ws = S.WORKSPACE.get(torch.device("cuda", torch.cuda.current_device()), "sample", 0)
    flags = host(ws[DEFER_OFFSET:DEFER_OFFSET + 4 * rows].view(torch.int32))
    assert not flags[[0, 1, 2, 3, 6, 7]].any() and flags[[4, 5]].all(), flags


def test_per_row_dispatch_more_deferred_rows_than_the_workspace_holds():
    """Every row flat with top_k 0: all of them are left over, more than the follow-up's 32 workspace rows, so the rest
    are taken whole by single blocks; the results are the oracle's."""
    need_gpu()
    rows, vocab = 100, 30_000
    cfg = W.config3(seed=41, rows=rows)
    cfg["logits"] = np.ascontiguousarray(cfg["logits"][:, :vocab])
    cfg["counts"] = np.ascontiguousarray(cfg["counts"][:, :vocab])
    g, w = run_both(cfg, kmax=S.KMAX_MIXED)
    compare(g, w, "all rows left over")
    ws = S.WORKSPACE.get(torch.device("cuda", torch.cuda.current_device()), "sample", 0)
    flags = host(ws[DEFER_OFFSET:DEFER_OFFSET + 4 * rows].view(torch.int32))
    assert flags.all()
