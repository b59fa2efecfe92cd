"""Seeded synthetic inputs of the benchmark configurations (splitmix64 streams; normals by Box-Muller in double,
rounded to the logit dtype). Used by bench.py and the tests; numpy only."""
from __future__ import annotations

import numpy as np

GOLDEN = 0x9E3779B97F4A7C15


def splitmix(seed: int, n: int) -> np.ndarray:
    """n outputs of the splitmix64 stream started at `seed`."""
    idx = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed % (1 << 64)) + idx * np.uint64(GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def unit(seed: int, n: int) -> np.ndarray:
    """uniform doubles in [0, 1): the top 53 bits."""
    return (splitmix(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normals(seed: int, n: int) -> np.ndarray:
    m = (n + 1) // 2
    u = unit(seed, 2 * m)
    u1 = 1.0 - u[:m]  # (0, 1]
    u2 = u[m:]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])
    return z[:n]


def uniforms_f32(seed: int, n: int) -> np.ndarray:
    """f32 uniforms in [0, 1): 24 random bits."""
    return ((splitmix(seed, n) >> np.uint64(40)).astype(np.float32) * np.float32(1.0 / 16777216.0)).astype(np.float32)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def peaked_logits(seed: int, rows: int, vocab: int, sigma: float, n_peaks, lo: float, hi: float) -> np.ndarray:
    x = (normals(seed, rows * vocab) * sigma).astype(np.float32).reshape(rows, vocab)
    k = splitmix(seed ^ 0x5EED, rows * 64)
    u = unit(seed ^ 0xBEEF, rows * 64)
    for r in range(rows):
        npk = n_peaks if isinstance(n_peaks, int) else int(n_peaks[0] + k[r * 64] % (n_peaks[1] - n_peaks[0] + 1))
        for j in range(npk):
            x[r, int(k[r * 64 + 1 + j] % vocab)] = np.float32(lo + (hi - lo) * u[r * 64 + j])
    return x


def zipf_counts(seed: int, rows: int, vocab: int, history: int = 4096, s: float = 1.1) -> np.ndarray:
    """Per row: `history` tokens drawn Zipf(s) over a seeded permutation of the vocabulary (rank k -> token
    (a * k + b_row) mod vocab, a coprime to vocab), reduced to int32 counts."""
    import math
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    a = 1_000_003
    while math.gcd(a, vocab) != 1:
        a += 2
    offs = splitmix(seed, rows) % np.uint64(vocab)
    out = np.zeros((rows, vocab), dtype=np.int32)
    for r in range(rows):
        k = np.minimum(np.searchsorted(cdf, unit(seed + 104729 * r + 1, history), side="right"), vocab - 1)
        tok = (k.astype(np.int64) * a + int(offs[r])) % vocab
        out[r] = np.bincount(tok, minlength=vocab).astype(np.int32)
    return out


def grammar_masks(seed: int, rows: int, vocab: int, lo_frac: float = 1e-3, hi_frac: float = 0.5, singles: int = 8,
                  pairs: int = 2) -> np.ndarray:
    """u32 bitmasks [rows, ceil(vocab/32)]: allowed fraction log-uniform in [lo_frac, hi_frac], built as contiguous runs
    plus scattered bits; the first `singles` rows allow exactly one token, the next `pairs` rows exactly two."""
    words = (vocab + 31) // 32
    allowed = np.zeros((rows, vocab), dtype=bool)
    for r in range(rows):
        u = unit(seed + 31 * r, 64)
        ids = splitmix(seed + 31 * r + 17, 4096)
        if r < singles:
            allowed[r, int(ids[0] % vocab)] = True
            continue
        if r < singles + pairs:
            a, b = int(ids[0] % vocab), int(ids[1] % vocab)
            if a == b:
                b = (a + 1) % vocab
            allowed[r, a] = allowed[r, b] = True
            continue
        frac = np.exp(np.log(lo_frac) + (np.log(hi_frac) - np.log(lo_frac)) * u[0])
        target = max(1, int(frac * vocab))
        runs = 1 + int(u[1] * 8)
        run_len = max(1, int(target * 0.7) // runs)
        for j in range(runs):
            start = int(ids[j] % vocab)
            allowed[r, start:start + run_len] = True
        n_scatter = max(0, target - int(allowed[r].sum()))
        sc = splitmix(seed + 31 * r + 99, n_scatter) % np.uint64(vocab)
        allowed[r, sc.astype(np.int64)] = True
    padded = np.zeros((rows, words * 32), dtype=bool)
    padded[:, :vocab] = allowed
    bits = padded.reshape(rows, words, 32).astype(np.uint64) << np.arange(32, dtype=np.uint64)
    return bits.sum(axis=2).astype(np.uint32)


def row_params(rows: int, temperature=1.0, top_p=1.0, min_p=0.0, repetition=1.0, presence=0.0, frequency=0.0, top_k=0):
    from .sampling import ROW_PARAMS_DTYPE
    p = np.zeros(rows, dtype=ROW_PARAMS_DTYPE)
    p["temperature"], p["top_p"], p["min_p"] = temperature, top_p, min_p
    p["repetition"], p["presence"], p["frequency"], p["top_k"] = repetition, presence, frequency, top_k
    return p


# ---------------------------------------------------------------- the BASELINE configurations

def config1(seed: int = 1):
    V = 151_936
    x = peaked_logits(seed, 1, V, 2.0, 8, 8.0, 14.0)
    p = row_params(1, temperature=0.7, top_p=0.9, top_k=50)
    return dict(logits=x, dtype="f32", params=p, uniforms=uniforms_f32(seed + 2, 1), counts=None, mask=None)


def config2(seed: int = 2, rows: int = 64):
    B, V = rows, 151_936
    x = peaked_logits(seed, B, V, 1.0, (4, 16), 6.0, 14.0)
    t = (0.5 + 0.7 * unit(seed + 3, B)).astype(np.float32)
    t[[i for i in (5, 17, 33, 60) if i < B]] = 0.0
    p = row_params(B, temperature=t, top_p=0.95, min_p=0.05, top_k=40)
    return dict(logits=to_bf16_bits(x), dtype="bf16", params=p, uniforms=uniforms_f32(seed + 4, B), counts=None, mask=None)


def config3(seed: int = 3, rows: int = 128):
    V = 154_880
    x = (normals(seed, rows * V) * 1.5).astype(np.float32).reshape(rows, V)
    c = zipf_counts(seed + 5, rows, V)
    p = row_params(rows, temperature=0.8, top_p=0.9, repetition=1.1, presence=0.5, frequency=0.3, top_k=0)
    return dict(logits=x, dtype="f32", params=p, uniforms=uniforms_f32(seed + 6, rows), counts=c, mask=None)


def config4(seed: int = 4, rows: int = 256):
    V = 129_280
    x = (normals(seed, rows * V) * 2.0).astype(np.float32).reshape(rows, V)
    m = grammar_masks(seed + 7, rows, V)
    p = row_params(rows, temperature=1.0, top_p=0.95, top_k=64)
    return dict(logits=x, dtype="f32", params=p, uniforms=uniforms_f32(seed + 8, rows), counts=None, mask=m)


def northstar(seed: int = 9, rows: int = 256, vocab: int = 151_936):
    """B=256, V=151,936 fp32: penalties over dense counts + grammar mask + temperature + top-k/top-p."""
    x = peaked_logits(seed, rows, vocab, 2.0, (4, 16), 6.0, 14.0)
    c = zipf_counts(seed + 5, rows, vocab)
    m = grammar_masks(seed + 7, rows, vocab, lo_frac=0.05, hi_frac=0.9, singles=2, pairs=2)
    p = row_params(rows, temperature=0.8, top_p=0.9, top_k=50, repetition=1.1, presence=0.5, frequency=0.3)
    return dict(logits=x, dtype="f32", params=p, uniforms=uniforms_f32(seed + 8, rows), counts=c, mask=m)


def config5(seed: int = 5, n_seq: int = 32, width: int = 7, vocab: int = 151_936, temperature: float = 1.0):
    R = n_seq * (width + 1)
    target = peaked_logits(seed, R, vocab, 2.0, 8, 8.0, 14.0)
    draft = (target + (normals(seed + 11, R * vocab) * 0.5).astype(np.float32).reshape(R, vocab)).astype(np.float32)
    temps = np.full(R, temperature, dtype=np.float32)
    # draft tokens from q (softmax of the draft rows at T) by inverse CDF on seeded uniforms, float64
    u = unit(seed + 12, R)
    ids = np.zeros((n_seq, width), dtype=np.int32)
    for s in range(n_seq):
        for j in range(width):
            row = draft[s * (width + 1) + j].astype(np.float64) / temperature
            q = np.exp(row - row.max())
            cdf = np.cumsum(q)
            ids[s, j] = min(int(np.searchsorted(cdf, u[s * (width + 1) + j] * cdf[-1], side="right")), vocab - 1)
    return dict(target=target, draft=draft, draft_ids=ids, temperatures=temps, u_accept=uniforms_f32(seed + 13, n_seq * width).reshape(n_seq, width),
                u_resample=uniforms_f32(seed + 14, n_seq), n_seq=n_seq, width=width)
