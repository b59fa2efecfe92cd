"""The DSV4 Markov walk drop-ins (gb_dsv4_mtp_markov_walk_fast_bf16 / _keyed_bf16) on the GPU against the oracle: ids
and the in-place biased logits bit-exact, the keyed walk's conf within 1e-6 relative."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from rexl3_amd import sampling as S
from tests.gpu_util import host, log, need_gpu
from tests.test_oracle_markov import bf16_bits

pytestmark = pytest.mark.gpu


def run(logits, first, embed, head, rows, **kw):
    V = logits.shape[1]
    assert logits.shape == (rows, V) and embed.shape == (V, 256) and head.shape == (V, 256) and V >= 1024
    lg = torch.from_numpy(logits.copy()).cuda()
    ids = torch.zeros(rows + 1, dtype=torch.int32, device="cuda")
    ids[0] = first
    emb = torch.from_numpy(embed.view(np.int16)).cuda().view(torch.bfloat16)
    hed = torch.from_numpy(head.view(np.int16)).cuda().view(torch.bfloat16)
    conf = S.markov_walk(lg, ids, emb, hed, **kw)
    torch.cuda.synchronize()
    return host(ids), (None if conf is None else host(conf)), host(lg)


@pytest.mark.parametrize("V", [1024, 5000, 151_936])
def test_fast_walk(V):
    need_gpu()
    rng = np.random.default_rng(V)
    rows = 6
    logits = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    embed = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    head = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    log(f"markov fast V={V}")
    g_ids, _, g_lg = run(logits, 11, embed, head, rows)
    w_ids, _, w_lg = O.markov_walk(logits, 11, embed, head, rows)
    assert np.array_equal(g_ids, w_ids)
    assert np.array_equal(g_lg, w_lg)


@pytest.mark.parametrize("cand_k,t,p,mp", [(1, 0.7, 1.0, 0.0), (8, 0.7, 0.9, 0.0), (64, 1.3, 0.95, 0.05), (20, 0.0, 1.0, 0.0),
                                           (64, 0.5, 0.5, 0.2)])
def test_keyed_walk(cand_k, t, p, mp):
    need_gpu()
    rng = np.random.default_rng(cand_k + 7)
    V, rows = 4096, 8
    logits = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    embed = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    head = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    log(f"markov keyed cand_k={cand_k} T={t} top_p={p} min_p={mp}")
    kw = dict(keyed=True, cand_k=cand_k, seed=1234, temperature=t, top_p=p, min_p=mp, base_pos=77)
    g_ids, g_conf, g_lg = run(logits, 5, embed, head, rows, **kw)
    w_ids, w_conf, w_lg = O.markov_walk(logits, 5, embed, head, rows, True, cand_k, 1234, t, p, mp, 77)
    assert np.array_equal(g_ids, w_ids)
    assert np.array_equal(g_lg, w_lg)
    np.testing.assert_allclose(g_conf, w_conf, rtol=1e-6)


def test_walk_from_an_out_of_range_token_and_ties():
    """ids[0] outside the vocabulary adds a zero bias; equal logits keep the lowest id first."""
    need_gpu()
    rng = np.random.default_rng(3)
    V, rows = 2048, 3
    logits = np.round(rng.standard_normal((rows, V)) * 4).astype(np.float32)  # many exact ties
    embed = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    head = bf16_bits(np.zeros((V, 256)))  # zero bias: the candidates keep their (tied) logits
    for keyed in (False, True):
        log(f"markov ties keyed={keyed}")
        kw = dict(keyed=keyed, cand_k=16, seed=5, temperature=0.0 if keyed else 1.0)
        g_ids, _, g_lg = run(logits, V + 5, embed, head, rows, **kw)
        w_ids, _, w_lg = O.markov_walk(logits, V + 5, embed, head, rows, keyed, 16, 5, 0.0 if keyed else 1.0, 1.0, 0.0, 0)
        assert np.array_equal(g_ids, w_ids) and np.array_equal(g_lg, w_lg)


def test_keyed_walk_with_device_params_equals_the_scalar_form():
    """gb_dsv4_mtp_markov_walk_keyed_bf16_params reads cand_k and the sampling fields from a 72-byte device record."""
    need_gpu()
    rng = np.random.default_rng(41)
    V, rows = 3000, 5
    logits = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    embed = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    head = bf16_bits(rng.standard_normal((V, 256)) * 0.1)
    rec = np.zeros(1, dtype=S.DSV4_ROUND_PARAMS_DTYPE)
    rec[0]["cand_k"], rec[0]["seed"], rec[0]["base_pos"] = 24, 2024, 500
    rec[0]["temperature"], rec[0]["top_p"], rec[0]["min_p"] = 0.9, 0.8, 0.02
    params = torch.from_numpy(rec.view(np.uint8).copy()).cuda()
    log("markov keyed, device params")
    g_ids, g_conf, g_lg = run(logits, 9, embed, head, rows, keyed=True, params=params)
    w_ids, w_conf, w_lg = O.markov_walk(logits, 9, embed, head, rows, True, 24, 2024, 0.9, 0.8, 0.02, 500)
    assert np.array_equal(g_ids, w_ids) and np.array_equal(g_lg, w_lg)
    np.testing.assert_allclose(g_conf, w_conf, rtol=1e-6)
