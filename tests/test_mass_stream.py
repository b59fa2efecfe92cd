"""The branchless per-token mass the streaming kernels use (mass_fast) equals the definition (the oracle's gbo_mass)
bit for bit wherever its preconditions hold (c2 and M finite, l <= M): random and edge-case (l, M, c2) triples, built for the host from the same header."""
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


def triples(rng, n):
    out = []
    # typical rows: M the max of normals and peaks, temperatures 0.05 .. 4
    M = rng.uniform(-30, 30, n).astype(np.float32)
    l = (M - np.abs(rng.normal(0, 1, n)) * rng.choice([0.01, 1, 10, 40, 100], n)).astype(np.float32)
    l = np.minimum(l, M)
    c2 = (np.float32(1.4426950408889634) / rng.uniform(0.05, 4, n).astype(np.float32)).astype(np.float32)
    out.append((l, M, c2))
    # the boundaries of the shift range: y near every integer and half-integer in [-70, 1]
    k = np.repeat(np.arange(-140, 2) / 2.0, 64)
    m = len(k)
    M2 = rng.uniform(-5, 5, m).astype(np.float32)
    c22 = np.full(m, 1.0, np.float32)
    l2 = (M2 + (k + rng.uniform(-1e-3, 1e-3, m))).astype(np.float32)
    l2 = np.minimum(l2, M2)
    out.append((l2, M2, c22))
    # l == M, l = -inf, -0 / +0, huge c2 and tiny differences
    e = np.array([(0.0, 0.0, 1.0), (-0.0, 0.0, 1.0), (0.0, -0.0, 3.0), (-np.inf, 1.0, 1.0), (-np.inf, -5.0, 1e30), (1.0, 1.0, np.inf),
                  (np.nextafter(np.float32(1), np.float32(0)), 1.0, 1e6), (-3e38, 3e38, 1.0), (-1e-30, 0.0, 1e31)], dtype=np.float32)
    out.append((e[:, 0], e[:, 1], e[:, 2]))
    return [np.concatenate(z).astype(np.float32) for z in zip(*out)]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not present")
def test_mass_fast_matches_definition():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    tmp = tempfile.mkdtemp()
    try:
        exe = os.path.join(tmp, "mass_check")
        subprocess.run([HIPCC, "-O2", "-std=c++20", "-ffp-contract=off", "-fno-fast-math", "-x", "hip", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        os.path.join(ROOT, "tests", "mass_stream_check.cpp"), "-x", "none",
                        os.path.join(ROOT, "oracle", "build", "libgbs_oracle.so"),
                        "-Wl,-rpath," + os.path.join(ROOT, "oracle", "build"), "-o", exe], check=True)
        l, M, c2 = triples(np.random.default_rng(7), 200_000)
        inp = "\n".join(f"{a:x} {b:x} {c:x}" for a, b, c in zip(l.view(np.uint32), M.view(np.uint32), c2.view(np.uint32)))
        res = subprocess.run([exe], input=inp, capture_output=True, text=True, check=True).stdout.split()
        got = np.array(res[0::2], dtype=np.uint64)
        want = np.array(res[1::2], dtype=np.uint64)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, [(float(l[i]), float(M[i]), float(c2[i]), int(got[i]), int(want[i])) for i in bad[:5]]
        assert len(got) == len(l) and (want > 0).sum() > len(l) // 2
    finally:
        shutil.rmtree(tmp)
