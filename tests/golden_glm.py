"""Input generator of crates/cuda/tests/glm_keyed.rs:24-74 and 266-296 (the golden keyed-pick hashes)."""
from __future__ import annotations

import numpy as np

from tests.common import Rng


def f16_round(v: float) -> np.float32:
    """gb_exl3::f16 round trip (crates/exl3/src/f16.rs:6-49): f64 -> fp16 ties to even -> f64, then to f32."""
    return np.float32(np.float64(np.float16(np.float64(v))))


def candidates(rng: Rng, count: int):
    ids = []
    while len(ids) < count:
        i = rng.next() % 154_856
        if i not in ids:
            ids.append(i)
    pairs = []
    for i, tid in enumerate(ids):
        base = rng.uniform(-3.0, 3.0)
        if i % 7 == 3:
            v = np.float32(1.0)
        elif i % 11 == 0:
            v = np.float32(base + np.float32(4.0))
        else:
            v = base
        pairs.append((tid, f16_round(float(v))))
    pairs.sort(key=lambda p: (-float(p[1]), p[0]))
    return [p[0] for p in pairs], [p[1] for p in pairs]


def settings(rng: Rng, count: int):
    pick = lambda n: rng.next() % n  # noqa: E731
    top_k = min([1, 2, 8, 20, 40, 56][pick(6)], count)
    seed = rng.next() & ((1 << 63) - 1)
    temperature = [0.3, 0.7, 1.0, 1.3][pick(4)]
    top_p = [1.0, 0.95, 0.8, 0.5][pick(4)]
    min_p = [0.0, 0.05, 0.2][pick(3)]
    return dict(seed=seed, temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p)


def golden_case(count: int, rows: int, depth: int, keyed_row_dtype):
    """(ids [rows, count], vals [rows, count], params [rows]) of one golden line."""
    rng = Rng(9000 + count * 1000 + rows * 10 + depth)
    lists = [candidates(rng, count) for _ in range(rows)]
    recs = np.zeros(rows, dtype=keyed_row_dtype)
    for r in range(rows):
        s = settings(rng, count)
        pos = rng.next() % 8000
        recs[r] = (s["seed"], pos, 0.0 if r % 9 == 4 else s["temperature"], s["top_p"], s["min_p"], s["top_k"], int(r % 6 != 5))
    ids = np.array([l[0] for l in lists], dtype=np.int32)
    vals = np.array([l[1] for l in lists], dtype=np.float32)
    return ids, vals, recs


def golden_lines(path: str):
    out = []
    for line in open(path):
        parts = line.split()
        if not parts:
            continue
        kv = dict(p.split("=") for p in parts[:3])
        out.append((int(kv["count"]), int(kv["rows"]), int(kv["depth"]), int(parts[4], 16), int(parts[6], 16)))
    return out
