"""ctypes binding of the CPU oracle (oracle/build/libgbs_oracle.so) -- TEST INFRASTRUCTURE ONLY.

Only the tests, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg import this module, and only as the
checker. The product library (``rexl3_amd``) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libgbs_oracle.so")

ROW_OK, ROW_NO_CANDIDATES, ROW_NAN_LOGIT, ROW_INVALID_PARAMS = 0, 1, 2, 3
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2


class Sampling(C.Structure):
    """gb_sampling::Sampling (crates/sampling/src/lib.rs:28-36)."""

    _fields_ = [("seed", C.c_uint64), ("temperature", C.c_double), ("top_k", C.c_uint64), ("top_p", C.c_double),
                ("min_p", C.c_double)]


class KeyedRow(C.Structure):
    """KeyedRow (crates/cuda/csrc/glm_mtp.cu:258-264), 48 bytes."""

    _fields_ = [("seed", C.c_uint64), ("first_position", C.c_uint64), ("temperature", C.c_double), ("top_p", C.c_double),
                ("min_p", C.c_double), ("top_k", C.c_int32), ("keyed", C.c_int32)]


class RowParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("min_p", C.c_float), ("repetition", C.c_float),
                ("presence", C.c_float), ("frequency", C.c_float), ("top_k", C.c_int32), ("reserved", C.c_int32)]


class SampleOut(C.Structure):
    _fields_ = [("id", C.c_int32), ("greedy", C.c_int32), ("prob", C.c_float), ("logprob", C.c_double),
                ("status", C.c_int32), ("kept", C.c_int32), ("z_kept", C.c_uint64)]


class SpecOut(C.Structure):
    _fields_ = [("accepted", C.c_int32), ("status", C.c_int32)]


KEYED_ROW_DTYPE = np.dtype([("seed", "<u8"), ("first_position", "<u8"), ("temperature", "<f8"), ("top_p", "<f8"),
                            ("min_p", "<f8"), ("top_k", "<i4"), ("keyed", "<i4")])
ROW_PARAMS_DTYPE = np.dtype([("temperature", "<f4"), ("top_p", "<f4"), ("min_p", "<f4"), ("repetition", "<f4"),
                             ("presence", "<f4"), ("frequency", "<f4"), ("top_k", "<i4"), ("reserved", "<i4")])
assert KEYED_ROW_DTYPE.itemsize == 48 and ROW_PARAMS_DTYPE.itemsize == 32

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        L.gbo_mix.restype = C.c_uint64
        L.gbo_mix.argtypes = [C.c_uint64]
        L.gbo_unit_open.restype = C.c_double
        L.gbo_unit_open.argtypes = [C.c_uint64]
        L.gbo_uniform.restype = C.c_double
        L.gbo_uniform.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.gbo_pairwise_sum.restype = C.c_double
        L.gbo_pairwise_sum.argtypes = [P, C.c_size_t]
        L.gbo_seed_for.restype = C.c_uint64
        L.gbo_seed_for.argtypes = [P, C.c_size_t, C.c_uint64]
        L.gbo_sha256.argtypes = [P, C.c_size_t, P]
        L.gbo_try_choose.restype = C.c_int
        L.gbo_try_choose.argtypes = [P, P, C.c_size_t, C.c_uint64, C.POINTER(Sampling), C.POINTER(C.c_uint32)]
        L.gbo_try_top_candidates.restype = C.c_int
        L.gbo_try_top_candidates.argtypes = [P, C.c_size_t, C.c_size_t, P, P]
        L.gbo_accept.restype = C.c_size_t
        L.gbo_accept.argtypes = [P, C.c_size_t, P, C.c_size_t]
        L.gbo_accept_tree.restype = C.c_size_t
        L.gbo_accept_tree.argtypes = [P, P, P, C.c_size_t, P]
        for f in ("gbo_topk_f32_row", "gbo_topk_bf16_row", "gbo_topk_f16_row"):
            getattr(L, f).argtypes = [P, C.c_int, C.c_int, P, P]
        L.gbo_keyed_pick_row.argtypes = [P, P, C.c_int, P, C.c_int, P, P]
        L.gbo_keyed_sample_row.restype = C.c_int
        L.gbo_keyed_sample_row.argtypes = [P, C.c_int, C.c_int, P, C.c_int, P, P]
        L.gbo_mass.restype = C.c_uint64
        L.gbo_mass.argtypes = [C.c_float, C.c_float, C.c_float]
        L.gbo_temp_scale.restype = C.c_float
        L.gbo_temp_scale.argtypes = [C.c_float]
        L.gbo_mul_floor.restype = C.c_uint64
        L.gbo_mul_floor.argtypes = [C.c_float, C.c_uint64, C.POINTER(C.c_int)]
        L.gbo_order_key_f32.restype = C.c_uint32
        L.gbo_order_key_f32.argtypes = [C.c_float]
        L.gbo_penalized_logit.restype = C.c_float
        L.gbo_penalized_logit.argtypes = [C.c_float, C.c_int32, C.POINTER(RowParams), C.c_float]
        L.gbo_sample_row.argtypes = [P, C.c_int, C.c_int, P, P, C.POINTER(RowParams), C.c_float, C.POINTER(SampleOut)]
        L.gbo_spec_verify_seq.argtypes = [P, P, C.c_int, C.c_int, P, P, P, C.c_float, P, C.POINTER(SpecOut)]
        L.gbo_batch_keyed_sample.restype = C.c_int
        L.gbo_batch_keyed_sample.argtypes = [P, C.c_int, C.c_int, C.c_int, C.c_int, P, C.c_int, P, C.c_int]
        L.gbo_batch_sample.restype = C.c_int
        L.gbo_batch_sample.argtypes = [P, C.c_int, C.c_int, C.c_int, C.c_int, P, P, P, P, P, P, P, P, P, C.c_int]
        L.gbo_keyed_choose.restype = C.c_int
        L.gbo_keyed_choose.argtypes = [P, P, C.c_int, C.c_uint64, C.c_double, C.c_double, C.c_double, C.c_uint64, C.POINTER(C.c_float)]
        L.gbo_selector_walk.argtypes = [P, P, P, P, C.c_int, P, P, C.c_int, C.c_int, C.c_int, C.c_int, P, P, P, P, P]
        L.gbo_markov_walk.restype = None
        L.gbo_markov_walk.argtypes = [P, P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint64, C.c_double, C.c_double,
                                      C.c_double, C.c_uint64]
        L.gbo_row_argmax.restype = None
        L.gbo_row_argmax.argtypes = [P, C.c_int, C.c_int, P]
        L.gbo_mtp_pick.restype = None
        L.gbo_mtp_pick.argtypes = [P, C.c_int, P, P]
        L.gbo_batch_spec_verify.restype = C.c_int
        L.gbo_batch_spec_verify.argtypes = [P, P, C.c_int, C.c_int, C.c_int, P, P, P, P, P, P, P, C.c_int]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- Mode K

def mix(x: int) -> int:
    return lib().gbo_mix(x)


def uniform(seed: int, position: int, tid: int) -> float:
    return lib().gbo_uniform(seed, position, tid)


def unit_open(x: int) -> float:
    return lib().gbo_unit_open(x)


def pairwise_sum(a) -> float:
    a = np.ascontiguousarray(a, dtype=np.float64)
    return lib().gbo_pairwise_sum(_p(a), a.size)


def seed_for(tokens, salt: int) -> int:
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    return lib().gbo_seed_for(_p(t), t.size, salt)


def sha256(data: bytes) -> bytes:
    out = (C.c_uint8 * 32)()
    buf = C.create_string_buffer(data, len(data))
    lib().gbo_sha256(buf, len(data), out)
    return bytes(out)


def try_choose(values, ids, position: int, s: Sampling):
    """(status, token id) of try_choose (crates/sampling/src/lib.rs:210)."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    i = np.ascontiguousarray(ids, dtype=np.uint32)
    if v.size != i.size:
        return ("LengthMismatch", None)
    out = C.c_uint32(0)
    st = lib().gbo_try_choose(_p(v), _p(i), v.size, position, C.byref(s), C.byref(out))
    return (st, out.value if st == ROW_OK else None)


def try_top_candidates(logits, count: int):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    take = min(count, lg.size)
    ids = np.zeros(max(take, 1), dtype=np.uint32)
    vals = np.zeros(max(take, 1), dtype=np.float32)
    st = lib().gbo_try_top_candidates(_p(lg), lg.size, count, _p(ids), _p(vals))
    return st, ids[:take], vals[:take]


def accept(drafts, samples) -> int:
    d = np.ascontiguousarray(drafts, dtype=np.uint32)
    s = np.ascontiguousarray(samples, dtype=np.uint32)
    return lib().gbo_accept(_p(d), d.size, _p(s), s.size)


def accept_tree(tokens, parents, samples):
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    p = np.ascontiguousarray(parents, dtype=np.int32)
    s = np.ascontiguousarray(samples, dtype=np.uint32)
    path = np.zeros(t.size, dtype=np.uint64)
    n = lib().gbo_accept_tree(_p(t), _p(p), _p(s), t.size, _p(path))
    return [int(x) for x in path[:n]]


def topk_row(row, count: int, dtype: int):
    """The device top-k contract for one row (dtype f32 / bf16 bits / f16 bits)."""
    ids = np.zeros(count, dtype=np.int32)
    vals = np.zeros(count, dtype=np.float32)
    if dtype == DTYPE_F32:
        r = np.ascontiguousarray(row, dtype=np.float32)
        lib().gbo_topk_f32_row(_p(r), r.size, count, _p(ids), _p(vals))
    else:
        r = np.ascontiguousarray(row, dtype=np.uint16)
        f = lib().gbo_topk_bf16_row if dtype == DTYPE_BF16 else lib().gbo_topk_f16_row
        f(_p(r), r.size, count, _p(ids), _p(vals))
    return ids, vals


def keyed_pick_rows(ids, vals, params, depth: int):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    vals = np.ascontiguousarray(vals, dtype=np.float32)
    params = np.ascontiguousarray(params, dtype=KEYED_ROW_DTYPE)
    rows, count = ids.shape
    oi = np.zeros(rows, dtype=np.int32)
    ov = np.zeros(rows, dtype=np.float32)
    for r in range(rows):
        lib().gbo_keyed_pick_row(_p(ids[r]), _p(vals[r]), count, _p(params[r:r + 1]), depth, _p(oi[r:r + 1]), _p(ov[r:r + 1]))
    return oi, ov


def keyed_sample_rows(logits, dtype: int, valid: int, params, depth: int):
    """gbs_keyed_sample_rows per row: (ids, vals, status)."""
    logits = np.ascontiguousarray(logits)
    params = np.ascontiguousarray(params, dtype=KEYED_ROW_DTYPE)
    rows = logits.shape[0]
    oi = np.zeros(rows, dtype=np.int32)
    ov = np.zeros(rows, dtype=np.float32)
    st = np.zeros(rows, dtype=np.int32)
    for r in range(rows):
        st[r] = lib().gbo_keyed_sample_row(_p(logits[r]), dtype, valid, _p(params[r:r + 1]), depth, _p(oi[r:r + 1]),
                                           _p(ov[r:r + 1]))
    return oi, ov, st


def batch_keyed_sample(logits, dtype: int, valid: int, params, depth: int, threads: int = 1):
    logits = np.ascontiguousarray(logits)
    params = np.ascontiguousarray(params, dtype=KEYED_ROW_DTYPE)
    rows, stride = logits.shape
    oi = np.zeros(rows, dtype=np.int32)
    lib().gbo_batch_keyed_sample(_p(logits), dtype, rows, stride, valid, _p(params), depth, _p(oi), threads)
    return oi


# ---------------------------------------------------------------- Mode U

def mass(l: float, lmax: float, c2: float) -> int:
    return lib().gbo_mass(l, lmax, c2)


def temp_scale(t: float) -> float:
    return lib().gbo_temp_scale(t)


def mul_floor(x: float, z: int):
    ex = C.c_int(0)
    f = lib().gbo_mul_floor(x, z, C.byref(ex))
    return f, bool(ex.value)


def order_key(v: float) -> int:
    return lib().gbo_order_key_f32(v)


def sample_rows(logits, dtype: int, counts, mask, params, uniforms, threads: int = 1):
    """The extended pipeline over a batch: dict of ids, greedy, probs, logprobs, status."""
    logits = np.ascontiguousarray(logits)
    rows, stride = logits.shape
    vocab = stride
    counts = None if counts is None else np.ascontiguousarray(counts, dtype=np.int32)
    mask = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    params = np.ascontiguousarray(params, dtype=ROW_PARAMS_DTYPE)
    uniforms = np.ascontiguousarray(uniforms, dtype=np.float32)
    out = dict(ids=np.zeros(rows, np.int32), greedy=np.zeros(rows, np.int32), probs=np.zeros(rows, np.float32),
               logprobs=np.zeros(rows, np.float64), status=np.zeros(rows, np.int32))
    lib().gbo_batch_sample(_p(logits), dtype, rows, stride, vocab, _p(counts), _p(mask), _p(params), _p(uniforms),
                           _p(out["ids"]), _p(out["greedy"]), _p(out["probs"]), _p(out["logprobs"]), _p(out["status"]),
                           threads)
    return out


def sample_row_detail(logits_row, dtype: int, counts_row, mask_row, params_row, u: float) -> SampleOut:
    r = np.ascontiguousarray(logits_row)
    c = None if counts_row is None else np.ascontiguousarray(counts_row, dtype=np.int32)
    m = None if mask_row is None else np.ascontiguousarray(mask_row, dtype=np.uint32)
    p = RowParams(*[params_row[f] for f in ROW_PARAMS_DTYPE.names])
    o = SampleOut()
    lib().gbo_sample_row(_p(r), dtype, r.size, _p(c), _p(m), C.byref(p), u, C.byref(o))
    return o


def spec_verify(target, draft, n_seq: int, width: int, draft_ids, temperatures, u_accept, u_resample, threads: int = 1):
    target = np.ascontiguousarray(target, dtype=np.float32)
    draft = np.ascontiguousarray(draft, dtype=np.float32)
    vocab = target.shape[-1]
    draft_ids = np.ascontiguousarray(draft_ids, dtype=np.int32)
    temperatures = np.ascontiguousarray(temperatures, dtype=np.float32)
    u_accept = np.ascontiguousarray(u_accept, dtype=np.float32)
    u_resample = np.ascontiguousarray(u_resample, dtype=np.float32)
    acc = np.zeros(n_seq, np.int32)
    toks = np.full((n_seq, width + 1), -1, np.int32)
    st = np.zeros(n_seq, np.int32)
    lib().gbo_batch_spec_verify(_p(target), _p(draft), n_seq, width, vocab, _p(draft_ids), _p(temperatures), _p(u_accept),
                                _p(u_resample), _p(acc), _p(toks), _p(st), threads)
    return acc, toks, st


WALK_SAMPLING_DTYPE = np.dtype([("seed", "<u8"), ("first_position", "<u8"), ("temperature", "<f8"), ("top_p", "<f8"),
                                ("min_p", "<f8"), ("keyed", "<i4"), ("pad", "<i4")])


def keyed_choose(scores, ids, seed: int, temperature: float, top_p: float, min_p: float, position: int):
    """crates/cuda/csrc/keyed.cuh:50-112 over k <= 64 scored candidates: (chosen index, margin)."""
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    m = C.c_float(0.0)
    i = lib().gbo_keyed_choose(_p(scores), _p(ids), scores.size, seed, temperature, top_p, min_p, position, C.byref(m))
    return i, m.value


def markov_walk(logits, first_id: int, embed, head, walk_rows: int, keyed: bool = False, cand_k: int = 1, seed: int = 0,
                temperature: float = 1.0, top_p: float = 1.0, min_p: float = 0.0, base_pos: int = 0):
    """crates/cuda/csrc/dsv4_mtp_gpu.cu:1233-1480 / 1662-1718: the DSV4 draft head's Markov walk. logits f32
    [walk_rows, vocab]; embed / head bf16 bits (u16) [vocab, 256]. Returns (ids [walk_rows + 1], conf [walk_rows],
    logits after the in-place bias)."""
    lg = np.array(logits, dtype=np.float32, order="C", copy=True)
    embed = np.ascontiguousarray(embed, dtype=np.uint16)
    head = np.ascontiguousarray(head, dtype=np.uint16)
    ids = np.zeros(walk_rows + 1, np.int32)
    ids[0] = first_id
    conf = np.zeros(walk_rows, np.float32)
    lib().gbo_markov_walk(_p(lg), _p(ids), _p(conf), _p(embed), _p(head), walk_rows, lg.shape[1], 1 if keyed else 0, cand_k, seed,
                          temperature, top_p, min_p, base_pos)
    return ids, conf, lg


def selector_walk(anchor, ids, vals, gate, gate_f32: bool, pred_cb, succ_cb, n_seq: int, rows: int, sampling=None, row_off=None):
    """crates/cuda/csrc/dflash2.cu:436-519 (walk_kernel). ids / vals [rows total, k]; gate [rows total, rank] as f32 or
    as bf16 bits (u16); codebooks as f16 bits (u16) [V, rank]. Returns (tokens, conf, margin) per row."""
    anchor = np.ascontiguousarray(anchor, dtype=np.int32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    vals = np.ascontiguousarray(vals, dtype=np.float32)
    gate = np.ascontiguousarray(gate, dtype=np.float32 if gate_f32 else np.uint16)
    pred_cb = np.ascontiguousarray(pred_cb, dtype=np.uint16)
    succ_cb = np.ascontiguousarray(succ_cb, dtype=np.uint16)
    total, k = ids.shape
    rank = gate.shape[-1]
    ws = None if sampling is None else np.ascontiguousarray(sampling, dtype=WALK_SAMPLING_DTYPE)
    ro = None if row_off is None else np.ascontiguousarray(row_off, dtype=np.int32)
    out = np.zeros(total, np.int32)
    conf = np.zeros(total, np.float32)
    margin = np.zeros(total, np.float32)
    lib().gbo_selector_walk(_p(anchor), _p(ids), _p(vals), _p(gate), 1 if gate_f32 else 0, _p(pred_cb), _p(succ_cb), n_seq, rows, k,
                            rank, _p(ws), _p(ro), _p(out), _p(conf), _p(margin))
    return out, conf, margin



def row_argmax(logits):
    """crates/cuda/csrc/dsv4_mtp_gpu.cu:503-539: per row, the first index of the largest value above -inf (0 if none)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    rows, vocab = x.shape
    out = np.zeros(rows, dtype=np.int32)
    lib().gbo_row_argmax(_p(x), rows, vocab, _p(out))
    return out


def mtp_pick(bf16_bits):
    """crates/cuda/csrc/mtp.cu:78-117: (argmax, 1 / sum exp(x - max)) of one bf16 row given as uint16 bits."""
    x = np.ascontiguousarray(bf16_bits, dtype=np.uint16)
    i = np.zeros(1, dtype=np.int32)
    p = np.zeros(1, dtype=np.float32)
    lib().gbo_mtp_pick(_p(x), x.shape[0], _p(i), _p(p))
    return int(i[0]), float(p[0])
