"""gbs_sample_rows_noalloc (the allocation-free form of gbs_sample_rows, workspace in a static device array) through the
C ABI against gbs_sample_rows on the same inputs: every output identical, on consecutive calls whose second input is
smaller (ids, greedy ids, probabilities and statuses bit-exact; log-probabilities within 1e-5 absolute, because the
single-pass kernel hands wave-steps to whichever wave asks first, so its f32 log-sum-exp order varies between runs),
for the single-pass path and the full-distribution path; a call too large for the array is refused with
nothing launched."""
import ctypes as C

import numpy as np
import pytest
import torch

from rexl3_amd import _lib
from rexl3_amd import sampling as S
from rexl3_amd import workloads as W
from tests.gpu_util import dev, host, log, need_gpu

pytestmark = pytest.mark.gpu
NOALLOC_MAX = 32 << 20  # GBS_NOALLOC_SCRATCH_BYTES
TOO_LARGE = 2           # GBS_ERR_NOALLOC_TOO_LARGE
LOGPROB_ATOL = 1e-5


def operands(cfg):
    rows, vocab = cfg["logits"].shape
    d = dict(x=dev(cfg["logits"]), c=None if cfg["counts"] is None else dev(cfg["counts"]),
             m=None if cfg["mask"] is None else dev(cfg["mask"]), u=dev(cfg["uniforms"]),
             p=dev(np.ascontiguousarray(cfg["params"]).view(np.uint8)))
    outs = [dict(ids=torch.full((rows,), -7, dtype=torch.int32, device="cuda"),
                 greedy=torch.full((rows,), -7, dtype=torch.int32, device="cuda"),
                 probs=torch.full((rows,), -7.0, device="cuda"), logprobs=torch.full((rows,), -7.0, device="cuda"),
                 status=torch.full((rows,), -7, dtype=torch.int32, device="cuda")) for _ in range(2)]
    return rows, vocab, d, outs


def args(rows, vocab, d, o, kmax):
    P = S._ptr
    return [P(d["x"]), 0, rows, vocab, vocab, P(d["c"]), P(d["m"]), P(d["p"]), P(d["u"]), kmax, P(o["ids"]), P(o["greedy"]),
            P(o["probs"]), P(o["logprobs"]), P(o["status"])]


def both(cfg, kmax):
    rows, vocab, d, (o_ref, o_na) = operands(cfg)
    wsb = _lib.load().gbs_sample_workspace_bytes(rows, vocab, kmax)
    assert 0 < wsb <= NOALLOC_MAX
    ws = torch.zeros(wsb, dtype=torch.uint8, device="cuda")
    st = S._stream(torch.device("cuda"))
    log(f"noalloc rows={rows} vocab={vocab} kmax={kmax}")
    _lib.call("gbs_sample_rows", *args(rows, vocab, d, o_ref, kmax), S._ptr(ws), wsb, st)
    _lib.call("gbs_sample_rows_noalloc", *args(rows, vocab, d, o_na, kmax), st)
    torch.cuda.synchronize()
    for k in ("ids", "greedy", "probs", "status"):
        a, b = host(o_ref[k]), host(o_na[k])
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (k, rows, vocab, kmax)
    np.testing.assert_allclose(host(o_na["logprobs"]), host(o_ref["logprobs"]), rtol=0, atol=LOGPROB_ATOL)
    assert (host(o_ref["status"]) == 0).all() and (host(o_ref["ids"]) >= 0).all()


def test_noalloc_single_pass_twice_second_smaller():
    need_gpu()
    both(W.northstar(seed=12, rows=64, vocab=151_936), 64)
    both(W.northstar(seed=13, rows=5, vocab=50_001), 64)


def test_noalloc_full_path_twice_second_smaller():
    need_gpu()
    both(W.config3(seed=14, rows=16), 0)
    both(W.config3(seed=15, rows=3), 0)


def test_noalloc_refuses_a_call_beyond_its_scratch():
    need_gpu()
    rows, vocab = 200, 154_880
    assert _lib.load().gbs_sample_workspace_bytes(rows, vocab, 0) > NOALLOC_MAX
    cfg = dict(logits=np.zeros((rows, vocab), np.float32), counts=None, mask=None, uniforms=np.zeros(rows, np.float32),
               params=W.row_params(rows, top_p=0.9))
    rows, vocab, d, (o, _) = operands(cfg)
    rc = _lib.load().gbs_sample_rows_noalloc(*args(rows, vocab, d, o, 0), S._stream(torch.device("cuda")))
    torch.cuda.synchronize()
    assert rc == TOO_LARGE
    assert (host(o["ids"]) == -7).all() and (host(o["status"]) == -7).all()
