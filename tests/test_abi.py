"""The C ABI without a GPU: libgbsample_hip.so loads and exports exactly the functions include/gbs_sample.h declares,
the struct layouts match the reference's, and the workspace-size queries follow their contracts."""
import ctypes as C
import os
import re
import subprocess

import numpy as np

from rexl3_amd import _lib
from rexl3_amd import sampling as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gbs_sample.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w]*\s*\**\s+\**([A-Za-z_]\w*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n.startswith(("gb_", "gbs_"))))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = declared()
    assert len(names) >= 19
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, n
    assert set(_lib.SIGNATURES) == set(names)


def test_no_other_symbols_are_exported():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = sorted({l.split()[-1] for l in out.splitlines() if " T " in l})
    ours = [s for s in exported if s.startswith(("gb_", "gbs_"))]
    assert sorted(ours) == declared()


def test_struct_layouts():
    assert S.KEYED_ROW_DTYPE.itemsize == 48  # crates/cuda/csrc/glm_mtp.cu:258-264
    assert [S.KEYED_ROW_DTYPE.fields[f][1] for f in S.KEYED_ROW_DTYPE.names] == [0, 8, 16, 24, 32, 40, 44]
    assert S.ROW_PARAMS_DTYPE.itemsize == 32


def test_workspace_queries():
    lib = _lib.load()
    # the reference's bf16 plan: rows * ceil(valid / 16384) * P(count) * 8 (crates/cuda/csrc/glue.cu:1078-1081)
    assert lib.gb_topk_valid_workspace_bytes(4, 248320, 28) == 4 * 16 * 32 * 8
    assert lib.gb_topk_valid_workspace_bytes(1, 100, 16) == 1 * 1 * 16 * 8
    assert lib.gb_topk_valid_workspace_bytes(1, 100, 65) == 0
    assert lib.gb_topk_valid_workspace_bytes(0, 100, 5) == 0
    assert lib.gb_topk_workspace_bytes(3, 5000, 64) == lib.gb_topk_valid_workspace_bytes(3, 5000, 64)
    assert lib.gb_glm_topk_f16_workspace_bytes(2, 70000, 40) == 2 * 5 * 64 * 8
    assert lib.gbs_sample_workspace_bytes(256, 151936, 64) > 0
    assert lib.gbs_sample_workspace_bytes(256, 151936, 65) == 0
    assert lib.gbs_sample_workspace_bytes(4, S.ROW_PARAMS_DTYPE.itemsize * 0 + 524289, 8) == 0  # vocab above the maximum
    assert lib.gbs_keyed_sample_workspace_bytes(64, 151936) > 0
    assert lib.gbs_spec_verify_workspace_bytes(32, 7, 151936) > 0
    assert lib.gbs_version().startswith(b"gbsample-hip")


def test_argument_checks_refuse_before_touching_memory():
    """Shapes outside the contract return 1 (hipErrorInvalidValue) with null pointers, so nothing is dereferenced or
    launched; an empty batch is a successful no-op."""
    lib = _lib.load()
    n = None
    assert lib.gb_topk_valid(n, 1, 100, 101, 10, n, n, n, 0, n) == 1
    assert lib.gb_topk_valid(n, 0, 100, 100, 10, n, n, n, 0, n) == 0
    assert lib.gb_nemo_glue_topk(n, 1, 100, 65, 1, n, 0, n, n, n) == 1
    assert lib.gb_glm_keyed_pick(n, n, 65, 1, n, 0, n, n, n) == 1
    assert lib.gb_glm_keyed_pick(n, n, 8, 0, n, 0, n, n, n) == 0
    assert lib.gb_qfn_greedy_gather(n, n, 8, 1, n, n, n) == 1
    assert lib.gb_dsv4_mtp_argmax(n, n, 1, 100, n) == 1
    assert lib.gb_mtp_pick(n, 0, n, n, 0, n) == 1
    assert lib.gbs_keyed_sample_rows(n, 0, 1, 100, 101, n, 0, n, n, n, n, 0, n) == 1
    assert lib.gbs_keyed_sample_rows(n, 7, 1, 100, 100, n, 0, n, n, n, n, 0, n) == 1
    assert lib.gbs_sample_rows(n, 0, 1, 100, 100, n, n, n, n, 65, n, n, n, n, n, n, 0, n) == 1
    assert lib.gbs_sample_rows(n, 3, 1, 100, 100, n, n, n, n, 8, n, n, n, n, n, n, 0, n) == 1  # no dtype 3
    assert lib.gbs_sample_rows(n, 0, 1, 100, 100, n, n, n, n, -2, n, n, n, n, n, n, 0, n) == 1  # kmax below GBS_KMAX_MIXED
    assert lib.gbs_sample_rows(n, 0, 0, 100, 100, n, n, n, n, 8, n, n, n, n, n, n, 0, n) == 0
    assert lib.gbs_spec_verify(n, n, 1, 7, 524289, 524289, n, n, n, n, n, n, n, n, 0, n) == 1
    assert lib.gbs_spec_verify(n, n, 1, 7, 1000, 999, n, n, n, n, n, n, n, n, 0, n) == 1  # stride below vocab
    assert lib.gbs_accept(n, n, -1, 3, n, n) == 1
    assert lib.gbs_accept_tree(n, n, n, 1, 0, n, n, n) == 1
    assert lib.gbs_workspace_clear(n, 0, n) == 0


def test_product_never_imports_the_oracle():
    """The oracle is the checker only: nothing under rexl3_amd/ imports, links or loads it."""
    pat = re.compile(r"from\s+oracle|import\s+oracle|gbs_oracle|libgbs_oracle|oracle/")
    for dirpath, _, files in os.walk(os.path.join(ROOT, "rexl3_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".h")):
                assert not pat.search(open(os.path.join(dirpath, f)).read()), f
