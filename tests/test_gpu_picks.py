"""gb_dsv4_mtp_argmax and gb_mtp_pick on the device against the oracle (tests/test_oracle_picks.py pins it): ids bit
exact; the pick's probability within 2e-5 relative (the device sums fast-exp float terms, the oracle float64)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from rexl3_amd import sampling as S

pytestmark = pytest.mark.gpu


def _bf16(a):
    return (np.asarray(a, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("rows,vocab", [(1, 129280), (8, 129280), (3, 1001), (5, 4)])
def test_dsv4_argmax_matches_oracle(rows, vocab):
    rng = np.random.default_rng(rows * 7 + vocab)
    x = rng.integers(-50, 50, size=(rows, vocab)).astype(np.float32)  # ties at the maximum across the row
    if vocab > 100:
        x[0, :] = -np.inf
        x[0, 99] = np.nan
        if rows > 1:
            x[1, 40] = np.inf
            x[1, 30] = np.nan
            x[1, 77] = np.inf
    if rows > 2:
        x[2, :] = 0.0
        x[2, 1::2] = -0.0
    print(f"dsv4_argmax rows={rows} vocab={vocab}", flush=True)
    got = S.dsv4_argmax(torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(got, O.row_argmax(x))


def test_dsv4_argmax_unaligned_rows():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(4, 1003)).astype(np.float32)
    print("dsv4_argmax unaligned", flush=True)
    got = S.dsv4_argmax(torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(got, O.row_argmax(x))


@pytest.mark.parametrize("n", [1, 9, 4096, 129280, 151936])
def test_mtp_pick_matches_oracle(n):
    rng = np.random.default_rng(n)
    bits = _bf16(rng.normal(scale=2.0, size=n))
    if n > 100:
        bits[17] = bits[n - 3] = _bf16([9.5])[0]
    t = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
    out_id = torch.full((4,), -7, dtype=torch.int32, device="cuda")
    out_p = torch.zeros(4, dtype=torch.float32, device="cuda")
    print(f"mtp_pick n={n}", flush=True)
    S.mtp_pick(t, out_id, out_p, 2)
    i, p = O.mtp_pick(bits)
    oi, op = out_id.cpu().numpy(), out_p.cpu().numpy()
    assert oi[2] == i and oi[0] == -7 and oi[3] == -7
    assert op[2] == pytest.approx(p, rel=2e-5)


def test_mtp_pick_nan_and_empty():
    out_id = torch.zeros(1, dtype=torch.int32, device="cuda")
    out_p = torch.zeros(1, dtype=torch.float32, device="cuda")
    for vals, want in (([1.0, float("nan"), 3.0, 0.5, 0.0, 0.0, 0.0, 0.0], 2), ([float("-inf")] * 16, 0)):
        bits = _bf16(np.array(vals, np.float32))
        print(f"mtp_pick edge {want}", flush=True)
        S.mtp_pick(torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16), out_id, out_p, 0)
        assert out_id.item() == want and np.isnan(out_p.item())
