"""Host-side mirror of REXL3's sampler API over the MI355X library (include/gbs_sample.h).

Names and argument meanings follow `gb_sampling` (crates/sampling/src/lib.rs:26-305) and `gb_spec`
(crates/spec/src/lib.rs:30-35, crates/spec/src/tree.rs:417-438); every call runs on the GPU through the C ABI.
PyTorch only provides device memory and the current stream.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

MARGIN = 8  # crates/sampling/src/lib.rs:26
TOP_K_CAP = 56  # crates/server/src/api.rs:43-44
ROW_OK, ROW_NO_CANDIDATES, ROW_NAN_LOGIT, ROW_INVALID_PARAMS = 0, 1, 2, 3
KMAX_MIXED = -1  # sample_rows: per-row dispatch for a batch that mixes rows of any top_k (GBS_KMAX_MIXED)
STATUS_NAMES = {0: "ok", 1: "NoCandidates", 2: "NanLogit", 3: "InvalidParams"}
DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

KEYED_ROW_DTYPE = np.dtype([("seed", "<u8"), ("first_position", "<u8"), ("temperature", "<f8"), ("top_p", "<f8"),
                            ("min_p", "<f8"), ("top_k", "<i4"), ("keyed", "<i4")])
ROW_PARAMS_DTYPE = np.dtype([("temperature", "<f4"), ("top_p", "<f4"), ("min_p", "<f4"), ("repetition", "<f4"),
                             ("presence", "<f4"), ("frequency", "<f4"), ("top_k", "<i4"), ("reserved", "<i4")])


class SamplingError(Exception):
    """crates/sampling/src/lib.rs:70-76."""


@dataclass(frozen=True)
class Sampling:
    """crates/sampling/src/lib.rs:28-68."""

    seed: int = 0
    temperature: float = 1.0
    top_k: int = 20
    top_p: float = 0.95
    min_p: float = 0.0

    def candidate_count(self, vocab: int) -> int:
        return vocab if self.top_k == 0 else min(self.top_k + MARGIN, vocab)

    def validate(self) -> None:
        if not math.isfinite(self.temperature) or self.temperature < 0.0:
            raise SamplingError("invalid sampling parameters: temperature must be finite and >= 0")
        if not math.isfinite(self.top_p) or not 0.0 <= self.top_p <= 1.0:
            raise SamplingError("invalid sampling parameters: top_p must be in [0, 1]")
        if not math.isfinite(self.min_p) or not 0.0 <= self.min_p <= 1.0:
            raise SamplingError("invalid sampling parameters: min_p must be in [0, 1]")


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(device) -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_cuda(t: torch.Tensor, name: str):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")


class Workspace:
    """Zero-initialised device workspaces, one per (device, stream, purpose), grown on demand. The gbs_* entry points
    leave their arrival counters at zero after every call, so a workspace is cleared once when it is allocated.

    Calls that share a workspace must not overlap; keying on the stream gives calls on different streams different
    buffers. A buffer is allocated while its stream is current, so the caching allocator hands a replaced buffer's
    memory only to later work on that same stream: the kernels still using it finish first."""

    def __init__(self):
        self._bufs = {}

    def get(self, device: torch.device, purpose: str, nbytes: int) -> torch.Tensor:
        stream = torch.cuda.current_stream(device)
        key = (str(device), stream.cuda_stream, purpose)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            with torch.cuda.stream(stream):
                buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            _lib.call("gbs_workspace_clear", _ptr(buf), buf.numel(), C.c_void_p(stream.cuda_stream))
            self._bufs[key] = buf
        return buf

    def keys(self):
        return list(self._bufs)


WORKSPACE = Workspace()


# ------------------------------------------------------------------------------------------------ top-k drop-ins

def topk_workspace_bytes(rows: int, valid: int, count: int, dtype: torch.dtype = torch.bfloat16, blocks: int = 1) -> int:
    lib = _lib.load()
    if dtype == torch.float32:
        return rows * blocks * 8 * count * 8
    if dtype == torch.float16:
        return lib.gb_glm_topk_f16_workspace_bytes(rows, valid, count)
    return lib.gb_topk_valid_workspace_bytes(rows, valid, count)


def topk(logits: torch.Tensor, count: int, valid: int | None = None, blocks: int | None = None):
    """Exact top-`count` per row by (value desc, id asc) (gb_topk_valid / gb_nemo_glue_topk / gb_glm_topk_f16).
    Returns (ids int32 [rows, count], vals float32 [rows, count])."""
    _require_cuda(logits, "logits")
    rows, stride = logits.shape
    valid = stride if valid is None else valid
    dev = logits.device
    ids = torch.empty((rows, count), dtype=torch.int32, device=dev)
    vals = torch.empty((rows, count), dtype=torch.float32, device=dev)
    st = _stream(dev)
    if logits.dtype == torch.float32:
        if valid != stride:
            raise ValueError("the f32 top-k reads whole rows (valid == stride)")
        if blocks is None:  # the reference's plan, crates/cuda/src/nemotron_glue.rs:172-176
            blocks = max(1, min(48 // max(rows, 1), 16, -(-stride // 2048)))
        wsb = rows * blocks * 8 * count * 8
        ws = torch.empty(max(wsb, 8), dtype=torch.uint8, device=dev)
        _lib.call("gb_nemo_glue_topk", _ptr(logits), rows, stride, count, blocks, _ptr(ws), wsb, _ptr(ids), _ptr(vals), st)
    else:
        lib = _lib.load()
        f16 = logits.dtype == torch.float16
        wsb = (lib.gb_glm_topk_f16_workspace_bytes if f16 else lib.gb_topk_valid_workspace_bytes)(rows, valid, count)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
        name = "gb_glm_topk_f16" if f16 else "gb_topk_valid"
        _lib.call(name, _ptr(logits), rows, stride, valid, count, _ptr(ids), _ptr(vals), _ptr(ws), wsb, st)
    return ids, vals


def topk_f16_single_launch(logits: torch.Tensor, count: int, valid: int | None = None, workspace: torch.Tensor | None = None):
    """gb_ling_topk_f16 (crates/cuda/src/ling_kda_proj_fused.rs:1409-1452, `topk_f16`): gb_glm_topk_f16's exact per-row
    top-`count` of fp16 logits in one launch. The workspace's first 256 bytes are self-resetting arrival counters: a
    caller-owned workspace must be cleared once before its first use (the default one is). Returns (ids, vals)."""
    _require_cuda(logits, "logits")
    if logits.dtype != torch.float16:
        raise ValueError("gb_ling_topk_f16 takes fp16 logits")
    rows, stride = logits.shape
    valid = stride if valid is None else valid
    dev = logits.device
    ids = torch.empty((rows, count), dtype=torch.int32, device=dev)
    vals = torch.empty((rows, count), dtype=torch.float32, device=dev)
    wsb = _lib.load().gb_ling_topk_f16_workspace_bytes(rows, valid, count)
    ws = WORKSPACE.get(dev, "ling_topk", wsb) if workspace is None else workspace
    _lib.call("gb_ling_topk_f16", _ptr(logits), rows, stride, valid, count, _ptr(ids), _ptr(vals), _ptr(ws), ws.numel(), _stream(dev))
    return ids, vals


WALK_SAMPLING_DTYPE = np.dtype([("seed", "<u8"), ("first_position", "<u8"), ("temperature", "<f8"), ("top_p", "<f8"),
                                ("min_p", "<f8"), ("keyed", "<i4"), ("pad", "<i4")])


def selector_walk(anchor: torch.Tensor, topk_ids: torch.Tensor, topk_vals: torch.Tensor, gate: torch.Tensor,
                  pred_codebook: torch.Tensor, succ_codebook: torch.Tensor, sampling: np.ndarray | None = None,
                  row_off: torch.Tensor | None = None):
    """The draft head's selector walk (gb_dflash_selector_walk_keyed, or _ragged when row_off is given;
    crates/cuda/src/dflash2.rs). topk_ids / topk_vals [rows total, k]; gate [rows total, rank] bf16 or f32; codebooks
    f16 [V, rank]; sampling: WALK_SAMPLING_DTYPE per sequence or None. Returns (tokens, conf, margin or None)."""
    dev = topk_ids.device
    n_seq = anchor.shape[0]
    rows_total, k = topk_ids.shape
    rank = gate.shape[-1]
    out = torch.empty(rows_total, dtype=torch.int32, device=dev)
    conf = torch.empty(rows_total, dtype=torch.float32, device=dev)
    ws = None
    if sampling is not None:
        ws = torch.from_numpy(np.ascontiguousarray(sampling, dtype=WALK_SAMPLING_DTYPE).view(np.uint8)).to(dev)
    g32 = 1 if gate.dtype == torch.float32 else 0
    if row_off is None:
        _lib.call("gb_dflash_selector_walk_keyed", _ptr(anchor), _ptr(topk_ids), _ptr(topk_vals), _ptr(gate), g32, _ptr(pred_codebook),
                  _ptr(succ_codebook), n_seq, rows_total // n_seq, k, rank, _ptr(ws), _ptr(out), _ptr(conf), _stream(dev))
        return out, conf, None
    margin = torch.empty(rows_total, dtype=torch.float32, device=dev)
    _lib.call("gb_dflash_selector_walk_ragged", _ptr(anchor), _ptr(topk_ids), _ptr(topk_vals), _ptr(gate), g32, _ptr(pred_codebook),
              _ptr(succ_codebook), n_seq, k, rank, _ptr(ws), _ptr(row_off), _ptr(out), _ptr(conf), _ptr(margin), _stream(dev))
    return out, conf, margin


DSV4_ROUND_PARAMS_DTYPE = np.dtype([("anchor", "<i4"), ("start_pos", "<i4"), ("reach", "<i4"), ("n_kv", "<i4"), ("window", "<i4"),
                                    ("block_size", "<i4"), ("cand_k", "<i4"), ("pad", "<i4"), ("seed", "<u8"), ("base_pos", "<u8"),
                                    ("temperature", "<f8"), ("top_p", "<f8"), ("min_p", "<f8")])


def markov_walk(logits: torch.Tensor, ids: torch.Tensor, embed: torch.Tensor, head: torch.Tensor, keyed: bool = False,
                cand_k: int = 1, seed: int = 0, temperature: float = 1.0, top_p: float = 1.0, min_p: float = 0.0,
                base_pos: int = 0, params: torch.Tensor | None = None):
    """The DSV4 draft head's Markov walk (gb_dsv4_mtp_markov_walk_fast_bf16 / _keyed_bf16 / _keyed_bf16_params;
    crates/cuda/src/dsv4_mtp_gpu.rs).
    logits f32 [walk_rows, vocab], biased in place; ids i32 [walk_rows + 1] (ids[0] in, the rest written); embed / head
    bf16 [vocab, 256]. Returns conf f32 [walk_rows] for the keyed walk, else None."""
    walk_rows, vocab = logits.shape
    rank = embed.shape[-1]
    dev = logits.device
    if ids.shape[0] != walk_rows + 1 or embed.shape[0] < vocab or head.shape[0] < vocab or head.shape[-1] != rank:
        raise ValueError("markov_walk: shapes")
    cand = torch.empty((walk_rows, 1024), dtype=torch.int32, device=dev)
    scores = torch.empty(1024, dtype=torch.float32, device=dev)
    if not keyed:
        _lib.call("gb_dsv4_mtp_markov_walk_fast_bf16", _ptr(logits), _ptr(ids), _ptr(embed), _ptr(head), _ptr(cand), _ptr(scores),
                  walk_rows, vocab, rank, _stream(dev))
        return None
    conf = torch.empty(walk_rows, dtype=torch.float32, device=dev)
    if params is not None:  # the device-params form: a 72-byte DSV4_ROUND_PARAMS_DTYPE record in device memory
        if params.numel() * params.element_size() != 72:
            raise ValueError("markov_walk: params must be one 72-byte record")
        _lib.call("gb_dsv4_mtp_markov_walk_keyed_bf16_params", _ptr(logits), _ptr(ids), _ptr(conf), _ptr(embed), _ptr(head), _ptr(cand),
                  _ptr(scores), walk_rows, vocab, rank, _ptr(params), _stream(dev))
        return conf
    _lib.call("gb_dsv4_mtp_markov_walk_keyed_bf16", _ptr(logits), _ptr(ids), _ptr(conf), _ptr(embed), _ptr(head), _ptr(cand),
              _ptr(scores), walk_rows, vocab, rank, cand_k, seed, temperature, top_p, min_p, base_pos, _stream(dev))
    return conf


def keyed_rows(samplings, positions) -> np.ndarray:
    """KeyedRow records (crates/cuda/csrc/glm_mtp.cu:258-264) for a list of Sampling and absolute positions."""
    recs = np.zeros(len(samplings), dtype=KEYED_ROW_DTYPE)
    for r, (s, p) in enumerate(zip(samplings, positions)):
        recs[r] = (s.seed, p, s.temperature, s.top_p, s.min_p, s.top_k, 1)
    return recs


def keyed_pick(ids: torch.Tensor, vals: torch.Tensor, params: np.ndarray, depth: int = 0):
    """gb_glm_keyed_pick: the keyed draw over each row's sorted candidates. Returns (ids [rows], vals [rows])."""
    rows, count = ids.shape
    dev = ids.device
    p = torch.from_numpy(np.ascontiguousarray(params, dtype=KEYED_ROW_DTYPE).view(np.uint8)).to(dev)
    oi = torch.empty(rows, dtype=torch.int32, device=dev)
    ov = torch.empty(rows, dtype=torch.float32, device=dev)
    _lib.call("gb_glm_keyed_pick", _ptr(ids), _ptr(vals), count, rows, _ptr(p), depth, _ptr(oi), _ptr(ov), _stream(dev))
    return oi, ov


def greedy_gather(ids: torch.Tensor, vals: torch.Tensor):
    rows, count = ids.shape
    dev = ids.device
    oi = torch.empty(rows, dtype=torch.int32, device=dev)
    ov = torch.empty(rows, dtype=torch.float32, device=dev)
    _lib.call("gb_qfn_greedy_gather", _ptr(ids), _ptr(vals), count, rows, _ptr(oi), _ptr(ov), _stream(dev))
    return oi, ov


def dsv4_argmax(logits: torch.Tensor) -> torch.Tensor:
    """gb_dsv4_mtp_argmax over f32 logits [rows, vocab]: per row the lowest id of the largest value above -inf (0 if
    none), int32 [rows]."""
    _require_cuda(logits, "logits")
    if logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous float32 [rows, vocab] tensor")
    rows, vocab = logits.shape
    out = torch.empty(rows, dtype=torch.int32, device=logits.device)
    _lib.call("gb_dsv4_mtp_argmax", _ptr(logits), _ptr(out), rows, vocab, _stream(logits.device))
    return out


def mtp_pick(logits: torch.Tensor, out_id: torch.Tensor, out_p: torch.Tensor, j: int) -> None:
    """gb_mtp_pick over one bf16 row [n]: out_id[j] = its argmax (lowest id on ties), out_p[j] = the maximum's softmax
    probability."""
    _require_cuda(logits, "logits")
    if logits.dtype != torch.bfloat16 or logits.dim() != 1 or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous bfloat16 [n] tensor")
    if out_id.dtype != torch.int32 or out_p.dtype != torch.float32 or out_id.numel() <= j or out_p.numel() <= j or j < 0:
        raise ValueError("out_id int32 / out_p float32 must hold index j")
    _lib.call("gb_mtp_pick", _ptr(logits), logits.shape[0], _ptr(out_id), _ptr(out_p), j, _stream(logits.device))


# ------------------------------------------------------------------------------------------------ fused keyed sampler

def keyed_sample_rows(logits: torch.Tensor, params: np.ndarray | torch.Tensor, depth: int = 0, valid: int | None = None,
                      out_vals: bool = False):
    """gbs_keyed_sample_rows: per row, top-(top_k + 8) of the full row then `try_choose` at first_position + depth.
    Returns (ids int32 [rows], status int32 [rows], vals float32 [rows] or None)."""
    _require_cuda(logits, "logits")
    rows, stride = logits.shape
    valid = stride if valid is None else valid
    dev = logits.device
    if isinstance(params, np.ndarray):
        params = torch.from_numpy(np.ascontiguousarray(params, dtype=KEYED_ROW_DTYPE).view(np.uint8)).to(dev)
    oi = torch.empty(rows, dtype=torch.int32, device=dev)
    os_ = torch.empty(rows, dtype=torch.int32, device=dev)
    ov = torch.empty(rows, dtype=torch.float32, device=dev) if out_vals else None
    wsb = _lib.load().gbs_keyed_sample_workspace_bytes(rows, valid)
    ws = WORKSPACE.get(dev, "keyed", wsb)
    _lib.call("gbs_keyed_sample_rows", _ptr(logits), DTYPE_CODE[logits.dtype], rows, stride, valid, _ptr(params), depth, _ptr(oi),
              _ptr(ov), _ptr(os_), _ptr(ws), ws.numel(), _stream(dev))
    return oi, os_, ov


def choose_rows(logits: torch.Tensor, positions, s: Sampling, valid: int | None = None) -> list[int]:
    """`choose_rows` (crates/sampling/src/lib.rs:269-280) over full logits rows: row r sampled at positions[r].
    Raises SamplingError on a failed row, as `choose` panics."""
    s.validate()
    rows = logits.shape[0]
    if len(positions) != rows:
        raise SamplingError("choose_rows: values, ids and positions differ in length")
    ids, st, _ = keyed_sample_rows(logits, keyed_rows([s] * rows, positions), 0, valid)
    st = st.cpu().numpy()
    bad = np.nonzero(st)[0]
    if bad.size:
        raise SamplingError(f"sampling failed: {STATUS_NAMES[int(st[bad[0]])]} (row {int(bad[0])})")
    return [int(x) for x in ids.cpu().numpy()]


# ------------------------------------------------------------------------------------------------ accept steps

def accept(drafts: torch.Tensor, samples: torch.Tensor) -> torch.Tensor:
    """Longest prefix with drafts == samples per sequence (crates/spec/src/lib.rs:30-35).
    drafts int32 [n_seq, width], samples int32 [n_seq, width + 1] -> int32 [n_seq]."""
    n_seq, width = drafts.shape
    dev = samples.device
    out = torch.empty(n_seq, dtype=torch.int32, device=dev)
    _lib.call("gbs_accept", _ptr(drafts), _ptr(samples), n_seq, width, _ptr(out), _stream(dev))
    return out


def accept_tree(tokens: torch.Tensor, parents: torch.Tensor, samples: torch.Tensor):
    """crates/spec/src/tree.rs:417-438 per tree: (path int32 [n_tree, nodes] padded with -1, path_len int32 [n_tree])."""
    n_tree, nodes = tokens.shape
    dev = tokens.device
    path = torch.empty((n_tree, nodes), dtype=torch.int32, device=dev)
    plen = torch.empty(n_tree, dtype=torch.int32, device=dev)
    _lib.call("gbs_accept_tree", _ptr(tokens), _ptr(parents), _ptr(samples), n_tree, nodes, _ptr(path), _ptr(plen), _stream(dev))
    return path, plen


def tree_verify(logits: torch.Tensor, params: np.ndarray | torch.Tensor, tokens: torch.Tensor, parents: torch.Tensor,
                valid: int | None = None):
    """gbs_tree_verify: a speculative tree round committed on the device (crates/engine/src/lib.rs:2376-2410). logits
    [n_tree * nodes, stride]; params KeyedRow per row with first_position = the node's position; tokens / parents
    [n_tree, nodes]. Returns (samples [n_tree * nodes], path [n_tree, nodes], path_len [n_tree], status [n_tree])."""
    _require_cuda(logits, "logits")
    rows, stride = logits.shape
    n_tree, nodes = tokens.shape
    if rows != n_tree * nodes:
        raise ValueError("tree_verify: logits rows != n_tree * nodes")
    valid = stride if valid is None else valid
    dev = logits.device
    if isinstance(params, np.ndarray):
        params = torch.from_numpy(np.ascontiguousarray(params, dtype=KEYED_ROW_DTYPE).view(np.uint8)).to(dev)
    samples = torch.empty(rows, dtype=torch.int32, device=dev)
    path = torch.empty((n_tree, nodes), dtype=torch.int32, device=dev)
    plen = torch.empty(n_tree, dtype=torch.int32, device=dev)
    st = torch.empty(n_tree, dtype=torch.int32, device=dev)
    wsb = _lib.load().gbs_tree_verify_workspace_bytes(n_tree, nodes, valid)
    ws = WORKSPACE.get(dev, "tree", wsb)
    _lib.call("gbs_tree_verify", _ptr(logits), DTYPE_CODE[logits.dtype], n_tree, nodes, stride, valid, _ptr(params), _ptr(tokens),
              _ptr(parents), _ptr(samples), _ptr(path), _ptr(plen), _ptr(st), _ptr(ws), ws.numel(), _stream(dev))
    return samples, path, plen, st


# ------------------------------------------------------------------------------------------------ extended pipeline

def row_params(rows: int, temperature=1.0, top_p=1.0, min_p=0.0, repetition=1.0, presence=0.0, frequency=0.0,
               top_k=0) -> np.ndarray:
    p = np.zeros(rows, dtype=ROW_PARAMS_DTYPE)
    p["temperature"], p["top_p"], p["min_p"] = temperature, top_p, min_p
    p["repetition"], p["presence"], p["frequency"], p["top_k"] = repetition, presence, frequency, top_k
    return p


def _check(t, name: str, dtype, shape: tuple, device):
    if t is None:
        return
    dtypes = dtype if isinstance(dtype, tuple) else (dtype,)
    if t.dtype not in dtypes or tuple(t.shape) != shape or not t.is_contiguous() or t.device != device:
        raise ValueError(f"{name} must be a contiguous {dtype} tensor of shape {shape} on {device}, got {t.dtype} "
                         f"{tuple(t.shape)} on {t.device}")


def sample_rows(logits: torch.Tensor, params: np.ndarray | torch.Tensor, uniforms: torch.Tensor, counts: torch.Tensor | None = None,
                mask: torch.Tensor | None = None, kmax: int = 64, logprobs: bool = False, probs: bool = True,
                vocab: int | None = None):
    """gbs_sample_rows over logits [rows, stride] (f32 / bf16 / f16, row stride may exceed `vocab`: the lm_head's padded
    layout; columns past `vocab` are never read). counts int32 [rows, vocab], mask uint32 [rows, ceil(vocab / 32)],
    uniforms float32 [rows]. Returns a dict of device tensors: ids, greedy, status, and probs / logprobs when asked."""
    _require_cuda(logits, "logits")
    rows, stride = logits.shape
    vocab = stride if vocab is None else vocab
    dev = logits.device
    if logits.dtype not in DTYPE_CODE or logits.stride(1) != 1 or not 0 < vocab <= stride:
        raise ValueError("logits must be f32, bf16 or f16 rows with unit column stride and vocab <= stride")
    _check(counts, "counts", torch.int32, (rows, vocab), dev)
    _check(mask, "mask", (torch.uint32, torch.int32), (rows, -(-vocab // 32)), dev)
    _check(uniforms, "uniforms", torch.float32, (rows,), dev)
    if isinstance(params, np.ndarray):
        params = torch.from_numpy(np.ascontiguousarray(params, dtype=ROW_PARAMS_DTYPE).view(np.uint8)).to(dev)
    if params.numel() * params.element_size() != rows * ROW_PARAMS_DTYPE.itemsize:
        raise ValueError("params must hold one 32-byte record per row")
    out = dict(ids=torch.empty(rows, dtype=torch.int32, device=dev), greedy=torch.empty(rows, dtype=torch.int32, device=dev),
               status=torch.empty(rows, dtype=torch.int32, device=dev))
    if probs:
        out["probs"] = torch.empty(rows, dtype=torch.float32, device=dev)
    if logprobs:
        out["logprobs"] = torch.empty(rows, dtype=torch.float32, device=dev)
    wsb = _lib.load().gbs_sample_workspace_bytes(rows, vocab, kmax)
    ws = WORKSPACE.get(dev, "sample", wsb)
    _lib.call("gbs_sample_rows", _ptr(logits), DTYPE_CODE[logits.dtype], rows, logits.stride(0), vocab, _ptr(counts), _ptr(mask),
              _ptr(params), _ptr(uniforms), kmax, _ptr(out["ids"]), _ptr(out["greedy"]), _ptr(out.get("probs")),
              _ptr(out.get("logprobs")), _ptr(out["status"]), _ptr(ws), ws.numel(), _stream(dev))
    return out


def spec_verify(target: torch.Tensor, draft: torch.Tensor, draft_ids: torch.Tensor, temperatures: torch.Tensor,
                u_accept: torch.Tensor, u_resample: torch.Tensor, vocab: int | None = None):
    """gbs_spec_verify over f32 target / draft rows [n_seq * (width + 1), stride] (the same row stride for both, which may
    exceed `vocab`: columns past it are never read): (accepted int32 [n_seq], tokens int32 [n_seq, width + 1], status
    int32 [n_seq])."""
    _require_cuda(target, "target")
    n_seq, width = draft_ids.shape
    rows, stride = target.shape
    vocab = stride if vocab is None else vocab
    dev = target.device
    if (target.dtype != torch.float32 or draft.dtype != torch.float32 or target.stride(1) != 1 or draft.stride(1) != 1
            or tuple(draft.shape) != (rows, stride) or draft.stride(0) != target.stride(0) or not 0 < vocab <= stride
            or rows != n_seq * (width + 1)):
        raise ValueError("target and draft must be f32 [n_seq * (width + 1), stride] rows with one row stride and vocab <= stride")
    _check(draft_ids, "draft_ids", torch.int32, (n_seq, width), dev)
    _check(temperatures, "temperatures", torch.float32, (rows,), dev)
    _check(u_accept, "u_accept", torch.float32, (n_seq, width), dev)
    _check(u_resample, "u_resample", torch.float32, (n_seq,), dev)
    acc = torch.empty(n_seq, dtype=torch.int32, device=dev)
    toks = torch.empty((n_seq, width + 1), dtype=torch.int32, device=dev)
    st = torch.empty(n_seq, dtype=torch.int32, device=dev)
    wsb = _lib.load().gbs_spec_verify_workspace_bytes(n_seq, width, vocab)
    ws = WORKSPACE.get(dev, "spec", wsb)
    _lib.call("gbs_spec_verify", _ptr(target), _ptr(draft), n_seq, width, vocab, target.stride(0), _ptr(draft_ids), _ptr(temperatures),
              _ptr(u_accept), _ptr(u_resample), _ptr(acc), _ptr(toks), _ptr(st), _ptr(ws), ws.numel(), _stream(dev))
    return acc, toks, st
