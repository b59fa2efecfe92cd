"""Loads libgbsample_hip.so (built in-tree by rexl3_amd/build.py) and declares its C ABI (include/gbs_sample.h).

There is no fallback: if the library is missing or does not load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libgbsample_hip.so")

P = C.c_void_p
I = C.c_int
Z = C.c_size_t

# name -> (restype, argtypes), exactly the declarations of include/gbs_sample.h
SIGNATURES = {
    "gb_topk_valid_workspace_bytes": (Z, [I, I, I]),
    "gb_topk_workspace_bytes": (Z, [I, I, I]),
    "gb_topk_valid": (I, [P, I, I, I, I, P, P, P, Z, P]),
    "gb_topk": (I, [P, I, I, I, P, P, P, Z, P]),
    "gb_nemo_glue_topk": (I, [P, I, I, I, I, P, Z, P, P, P]),
    "gb_glm_topk_f16_workspace_bytes": (Z, [I, I, I]),
    "gb_glm_topk_f16": (I, [P, I, I, I, I, P, P, P, Z, P]),
    "gb_ling_topk_f16_workspace_bytes": (Z, [I, I, I]),
    "gb_ling_topk_f16": (I, [P, I, I, I, I, P, P, P, Z, P]),
    "gb_dflash_selector_walk_keyed": (I, [P, P, P, P, I, P, P, I, I, I, I, P, P, P, P]),
    "gb_dflash_selector_walk_ragged": (I, [P, P, P, P, I, P, P, I, I, I, P, P, P, P, P, P]),
    "gb_dflash_selector_walk": (I, [P, P, P, P, I, P, P, I, I, I, I, P, P, P]),
    "gb_dsv4_mtp_markov_walk_fast_bf16": (I, [P, P, P, P, P, P, I, I, I, P]),
    "gb_dsv4_mtp_markov_walk_keyed_bf16": (I, [P, P, P, P, P, P, P, I, I, I, I, C.c_ulonglong, C.c_double, C.c_double, C.c_double,
                                                C.c_ulonglong, P]),
    "gb_dsv4_mtp_markov_walk_keyed_bf16_params": (I, [P, P, P, P, P, P, P, I, I, I, P, P]),
    "gb_glm_keyed_pick": (I, [P, P, I, I, P, I, P, P, P]),
    "gb_qfn_greedy_gather": (I, [P, P, I, I, P, P, P]),
    "gb_dsv4_mtp_argmax": (I, [P, P, I, I, P]),
    "gb_mtp_pick": (I, [P, I, P, P, I, P]),
    "gbs_workspace_clear": (I, [P, Z, P]),
    "gbs_keyed_sample_workspace_bytes": (Z, [I, I]),
    "gbs_keyed_sample_rows": (I, [P, I, I, I, I, P, I, P, P, P, P, Z, P]),
    "gbs_accept": (I, [P, P, I, I, P, P]),
    "gbs_accept_tree": (I, [P, P, P, I, I, P, P, P]),
    "gbs_tree_verify_workspace_bytes": (Z, [I, I, I]),
    "gbs_tree_verify": (I, [P, I, I, I, I, I, P, P, P, P, P, P, P, P, Z, P]),
    "gbs_sample_workspace_bytes": (Z, [I, I, I]),
    "gbs_sample_rows": (I, [P, I, I, I, I, P, P, P, P, I, P, P, P, P, P, P, Z, P]),
    "gbs_sample_rows_noalloc": (I, [P, I, I, I, I, P, P, P, P, I, P, P, P, P, P, P]),
    "gbs_spec_verify_workspace_bytes": (Z, [I, I, I]),
    "gbs_spec_verify": (I, [P, P, I, I, I, I, P, P, P, P, P, P, P, P, Z, P]),
    "gbs_spec_set_fuse_wait": (C.c_longlong, [C.c_longlong]),
    "gbs_version": (C.c_char_p, []),
}

_lib = None


class GbsError(RuntimeError):
    """A non-zero return code of a C entry point (1 = hipErrorInvalidValue: outside the contract, nothing launched)."""

    def __init__(self, name: str, code: int):
        super().__init__(f"{name} returned {code}")
        self.code = code


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python rexl3_amd/build.py` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise GbsError(name, rc)
