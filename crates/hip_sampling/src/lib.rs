//! The token-sampling path of REXL3 on AMD MI355X (gfx950), as a thin FFI over `libgbsample_hip.so`.
//!
//! `ffi` declares every function of `include/gbs_sample.h` exactly. The reference drop-ins (`gb_topk`,
//! `gb_topk_valid`, `gb_nemo_glue_topk`, `gb_glm_topk_f16`, `gb_ling_topk_f16`, `gb_glm_keyed_pick`,
//! `gb_qfn_greedy_gather`, the draft heads' walks) keep the names, arguments and return codes of `crates/cuda`
//! (`crates/cuda/src/glue.rs:494-558` and its sibling modules), so REXL3's existing wrappers link against this library
//! unchanged. The safe-signature wrappers below cover the entry points the reference has no launcher for: the fused
//! keyed sampler, the device accept steps and tree round, and the extended pipeline with its speculative verification.
//!
//! Conventions (every entry point): raw device pointers; the stream is a `hipStream_t` passed as `*mut c_void` (null =
//! the default stream); launches are asynchronous; 0 is success, 1 an argument outside the contract with nothing
//! launched, anything else the HIP launch error. The caller owns every buffer and workspace and keeps them alive until
//! the stream has drained them.

#![allow(clippy::too_many_arguments)]

use std::ffi::{c_void, CStr};

/// Per-row status, in the order of `gb_sampling::SamplingError` (crates/sampling/src/lib.rs:70-76).
pub const ROW_OK: i32 = 0;
pub const ROW_NO_CANDIDATES: i32 = 1;
pub const ROW_NAN_LOGIT: i32 = 2;
pub const ROW_INVALID_PARAMS: i32 = 3;

/// Logit element types.
pub const DTYPE_F32: i32 = 0;
pub const DTYPE_BF16: i32 = 1;
pub const DTYPE_F16: i32 = 2;

/// Largest vocabulary of the extended pipeline (integer mass sums stay below 2^63).
pub const MAX_VOCAB: usize = 524_288;
/// Candidates per row of the exact top-count kernels.
pub const MAX_COUNT: usize = 64;
/// `sample_rows`'s `kmax` for a batch that mixes rows of any top_k (per-row dispatch).
pub const KMAX_MIXED: i32 = -1;
/// Workspace bytes the allocation-free `sample_rows_noalloc` holds per GPU.
pub const NOALLOC_SCRATCH_BYTES: usize = 32 << 20;

/// The device keyed sampler's per-row record (crates/cuda/csrc/glm_mtp.cu:258-264), 48 bytes.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct KeyedRow {
    pub seed: u64,
    pub first_position: u64,
    pub temperature: f64,
    pub top_p: f64,
    pub min_p: f64,
    pub top_k: i32,
    pub keyed: i32,
}

/// The extended pipeline's per-row parameters, 32 bytes (no reference counterpart: REXL3 refuses penalties and grammar
/// masks, crates/server/src/api.rs:196-206). `top_k` 0 means no top-k.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct RowParams {
    pub temperature: f32,
    pub top_p: f32,
    pub min_p: f32,
    pub repetition: f32,
    pub presence: f32,
    pub frequency: f32,
    pub top_k: i32,
    pub reserved: i32,
}

const _: () = assert!(std::mem::size_of::<KeyedRow>() == 48);
const _: () = assert!(std::mem::size_of::<RowParams>() == 32);

/// A non-zero return code of an entry point (1: outside the contract, nothing launched; otherwise a HIP error).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct GbsError(pub i32);

impl GbsError {
    pub fn check(code: i32) -> Result<(), GbsError> {
        if code == 0 {
            Ok(())
        } else {
            Err(GbsError(code))
        }
    }
}

impl std::fmt::Display for GbsError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        match self.0 {
            1 => write!(f, "gbsample: invalid argument (nothing launched)"),
            2 => write!(f, "gbsample: the allocation-free call needs more than its static scratch"),
            c => write!(f, "gbsample: HIP error {c}"),
        }
    }
}

impl std::error::Error for GbsError {}

fn i(v: usize) -> Result<i32, GbsError> {
    i32::try_from(v).map_err(|_| GbsError(1))
}

/// The C declarations of include/gbs_sample.h, one for one.
pub mod ffi {
    use super::{KeyedRow, RowParams};
    use std::ffi::{c_char, c_void};

    extern "C" {
        // ---- 1. reference drop-ins
        pub fn gb_topk_valid_workspace_bytes(rows: i32, valid: i32, count: i32) -> usize;
        pub fn gb_topk_workspace_bytes(rows: i32, vocab: i32, count: i32) -> usize;
        pub fn gb_topk_valid(logits: *const c_void, rows: i32, stride: i32, valid: i32, count: i32, ids: *mut i32, vals: *mut f32,
                             workspace: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> i32;
        pub fn gb_topk(logits: *const c_void, rows: i32, vocab: i32, count: i32, ids: *mut i32, vals: *mut f32, workspace: *mut c_void,
                       ws_bytes: usize, stream: *mut c_void) -> i32;
        pub fn gb_nemo_glue_topk(logits: *const c_void, rows: i32, vocab: i32, count: i32, blocks: i32, ws: *mut c_void, ws_bytes: usize,
                                 ids: *mut c_void, vals: *mut c_void, stream: *mut c_void) -> i32;
        pub fn gb_glm_topk_f16_workspace_bytes(rows: i32, valid: i32, count: i32) -> usize;
        pub fn gb_glm_topk_f16(logits: *const c_void, rows: i32, stride: i32, valid: i32, count: i32, ids: *mut i32, vals: *mut f32,
                               workspace: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> i32;
        pub fn gb_ling_topk_f16_workspace_bytes(rows: i32, valid: i32, count: i32) -> usize;
        pub fn gb_ling_topk_f16(logits: *const c_void, rows: i32, stride: i32, valid: i32, count: i32, ids: *mut i32, vals: *mut f32,
                                workspace: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> i32;
        pub fn gb_dflash_selector_walk_keyed(anchor: *const c_void, topk_ids: *const c_void, topk_vals: *const c_void, gate: *const c_void,
                                             gate_is_f32: i32, pred_codebook: *const c_void, succ_codebook: *const c_void, n_seq: i32,
                                             rows: i32, k: i32, rank: i32, sampling: *const c_void, out_tokens: *mut c_void,
                                             conf: *mut c_void, stream: *mut c_void) -> i32;
        pub fn gb_dflash_selector_walk_ragged(anchor: *const c_void, topk_ids: *const c_void, topk_vals: *const c_void,
                                              gate: *const c_void, gate_is_f32: i32, pred_codebook: *const c_void,
                                              succ_codebook: *const c_void, n_seq: i32, k: i32, rank: i32, sampling: *const c_void,
                                              row_off: *const c_void, out_tokens: *mut c_void, conf: *mut c_void, margin: *mut c_void,
                                              stream: *mut c_void) -> i32;
        pub fn gb_dflash_selector_walk(anchor: *const c_void, topk_ids: *const c_void, topk_vals: *const c_void, gate: *const c_void,
                                       gate_is_f32: i32, pred_codebook: *const c_void, succ_codebook: *const c_void, n_seq: i32, rows: i32,
                                       k: i32, rank: i32, out_tokens: *mut c_void, conf: *mut c_void, stream: *mut c_void) -> i32;
        pub fn gb_dsv4_mtp_markov_walk_fast_bf16(logits: *mut c_void, ids: *mut i32, embed: *const c_void, head: *const c_void,
                                                 cand_ids_ws: *mut c_void, cand_scores_ws: *mut c_void, walk_rows: i32, vocab: i32,
                                                 rank: i32, stream: *mut c_void) -> i32;
        pub fn gb_dsv4_mtp_markov_walk_keyed_bf16(logits: *mut c_void, ids: *mut i32, conf: *mut f32, embed: *const c_void,
                                                  head: *const c_void, cand_ids_ws: *mut c_void, cand_scores_ws: *mut c_void,
                                                  walk_rows: i32, vocab: i32, rank: i32, cand_k: i32, seed: u64, temperature: f64,
                                                  top_p: f64, min_p: f64, base_pos: u64, stream: *mut c_void) -> i32;
        pub fn gb_dsv4_mtp_markov_walk_keyed_bf16_params(logits: *mut c_void, ids: *mut i32, conf: *mut f32, embed: *const c_void,
                                                         head: *const c_void, cand_ids_ws: *mut c_void, cand_scores_ws: *mut c_void,
                                                         walk_rows: i32, vocab: i32, rank: i32, params: *const c_void,
                                                         stream: *mut c_void) -> i32;
        pub fn gb_glm_keyed_pick(ids: *const i32, vals: *const f32, count: i32, rows: i32, params: *const c_void, depth: i32,
                                 out_ids: *mut i32, out_vals: *mut f32, stream: *mut c_void) -> i32;
        pub fn gb_qfn_greedy_gather(ids: *const c_void, vals: *const c_void, count: i32, rows: i32, out_ids: *mut c_void,
                                    out_vals: *mut c_void, stream: *mut c_void) -> i32;
        pub fn gb_dsv4_mtp_argmax(logits: *const f32, out: *mut i32, rows: i32, vocab: i32, stream: *mut c_void) -> i32;
        pub fn gb_mtp_pick(logits: *const c_void, n: i32, out_id: *mut c_void, out_p: *mut c_void, j: i32, stream: *mut c_void) -> i32;
        // ---- 2. fused and extended entry points
        pub fn gbs_workspace_clear(ws: *mut c_void, bytes: usize, stream: *mut c_void) -> i32;
        pub fn gbs_keyed_sample_workspace_bytes(rows: i32, valid: i32) -> usize;
        pub fn gbs_keyed_sample_rows(logits: *const c_void, dtype: i32, rows: i32, stride: i32, valid: i32, params: *const KeyedRow,
                                     depth: i32, out_ids: *mut i32, out_vals: *mut f32, out_status: *mut i32, ws: *mut c_void,
                                     ws_bytes: usize, stream: *mut c_void) -> i32;
        pub fn gbs_accept(drafts: *const i32, samples: *const i32, n_seq: i32, width: i32, accepted: *mut i32, stream: *mut c_void) -> i32;
        pub fn gbs_accept_tree(tokens: *const i32, parents: *const i32, samples: *const i32, n_tree: i32, nodes: i32, path: *mut i32,
                               path_len: *mut i32, stream: *mut c_void) -> i32;
        pub fn gbs_tree_verify_workspace_bytes(n_tree: i32, nodes: i32, valid: i32) -> usize;
        pub fn gbs_tree_verify(logits: *const c_void, dtype: i32, n_tree: i32, nodes: i32, stride: i32, valid: i32, params: *const KeyedRow,
                               tokens: *const i32, parents: *const i32, out_samples: *mut i32, out_path: *mut i32, out_path_len: *mut i32,
                               out_status: *mut i32, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> i32;
        pub fn gbs_sample_workspace_bytes(rows: i32, vocab: i32, kmax: i32) -> usize;
        pub fn gbs_sample_rows(logits: *const c_void, dtype: i32, rows: i32, stride: i32, vocab: i32, counts: *const i32, mask: *const u32,
                               params: *const RowParams, uniforms: *const f32, kmax: i32, out_ids: *mut i32, out_greedy: *mut i32,
                               out_probs: *mut f32, out_logprobs: *mut f32, out_status: *mut i32, ws: *mut c_void, ws_bytes: usize,
                               stream: *mut c_void) -> i32;
        pub fn gbs_sample_rows_noalloc(logits: *const c_void, dtype: i32, rows: i32, stride: i32, vocab: i32, counts: *const i32,
                                       mask: *const u32, params: *const RowParams, uniforms: *const f32, kmax: i32, out_ids: *mut i32,
                                       out_greedy: *mut i32, out_probs: *mut f32, out_logprobs: *mut f32, out_status: *mut i32,
                                       stream: *mut c_void) -> i32;
        pub fn gbs_spec_verify_workspace_bytes(n_seq: i32, width: i32, vocab: i32) -> usize;
        pub fn gbs_spec_verify(target: *const f32, draft: *const f32, n_seq: i32, width: i32, vocab: i32, stride: i32, draft_ids: *const i32,
                               temperatures: *const f32, u_accept: *const f32, u_resample: *const f32, out_accepted: *mut i32,
                               out_tokens: *mut i32, out_status: *mut i32, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> i32;
        pub fn gbs_spec_set_fuse_wait(ticks: i64) -> i64;
        pub fn gbs_version() -> *const c_char;
    }
}

/// The library's version string.
pub fn version() -> String {
    unsafe { CStr::from_ptr(ffi::gbs_version()) }.to_string_lossy().into_owned()
}

/// Zero a workspace by a kernel (capturable in a HIP graph). The gbs_* workspaces must be zero before their first use;
/// every call leaves their counters zero again.
pub unsafe fn workspace_clear(ws: *mut c_void, bytes: usize, stream: *mut c_void) -> Result<(), GbsError> {
    GbsError::check(ffi::gbs_workspace_clear(ws, bytes, stream))
}

/// Workspace bytes of [`keyed_sample_rows`].
pub fn keyed_sample_workspace_bytes(rows: usize, valid: usize) -> usize {
    unsafe { ffi::gbs_keyed_sample_workspace_bytes(rows as i32, valid as i32) }
}

/// Per row: the exact top-(top_k + 8) of `logits[row, 0..valid)` and `try_choose` (crates/sampling/src/lib.rs:210-267) at
/// `params[row].first_position + depth`, in one launch: `Engine::decode_round`'s gb_topk + download_candidates +
/// try_choose (crates/engine/src/lib.rs:2089-2117) with only ids leaving the device. `out_ids` -1 on a failed row,
/// whose status (`out_status`, may be null) says why.
pub unsafe fn keyed_sample_rows(logits: *const c_void, dtype: i32, rows: usize, stride: usize, valid: usize, params: *const KeyedRow,
                                depth: usize, out_ids: *mut i32, out_vals: *mut f32, out_status: *mut i32, ws: *mut c_void,
                                ws_bytes: usize, stream: *mut c_void) -> Result<(), GbsError> {
    GbsError::check(ffi::gbs_keyed_sample_rows(logits, dtype, i(rows)?, i(stride)?, i(valid)?, params, i(depth)?, out_ids, out_vals,
                                               out_status, ws, ws_bytes, stream))
}

/// `gb_spec::accept` (crates/spec/src/lib.rs:30-35) per sequence on the device: drafts i32 `[n_seq, width]`, samples
/// i32 `[n_seq, width + 1]`, accepted i32 `[n_seq]`.
pub unsafe fn accept(drafts: *const i32, samples: *const i32, n_seq: usize, width: usize, accepted: *mut i32,
                     stream: *mut c_void) -> Result<(), GbsError> {
    GbsError::check(ffi::gbs_accept(drafts, samples, i(n_seq)?, i(width)?, accepted, stream))
}

/// `gb_spec::tree::accept_tree` (crates/spec/src/tree.rs:417-438) per tree on the device.
pub unsafe fn accept_tree(tokens: *const i32, parents: *const i32, samples: *const i32, n_tree: usize, nodes: usize, path: *mut i32,
                          path_len: *mut i32, stream: *mut c_void) -> Result<(), GbsError> {
    GbsError::check(ffi::gbs_accept_tree(tokens, parents, samples, i(n_tree)?, i(nodes)?, path, path_len, stream))
}

/// Workspace bytes of [`tree_verify`].
pub fn tree_verify_workspace_bytes(n_tree: usize, nodes: usize, valid: usize) -> usize {
    unsafe { ffi::gbs_tree_verify_workspace_bytes(n_tree as i32, nodes as i32, valid as i32) }
}

/// A speculative tree round committed on the device (crates/engine/src/lib.rs:2376-2410): every node keyed-sampled at
/// its own position, then the accept walk.
pub unsafe fn tree_verify(logits: *const c_void, dtype: i32, n_tree: usize, nodes: usize, stride: usize, valid: usize,
                          params: *const KeyedRow, tokens: *const i32, parents: *const i32, out_samples: *mut i32, out_path: *mut i32,
                          out_path_len: *mut i32, out_status: *mut i32, ws: *mut c_void, ws_bytes: usize,
                          stream: *mut c_void) -> Result<(), GbsError> {
    GbsError::check(ffi::gbs_tree_verify(logits, dtype, i(n_tree)?, i(nodes)?, i(stride)?, i(valid)?, params, tokens, parents,
                                         out_samples, out_path, out_path_len, out_status, ws, ws_bytes, stream))
}

/// Workspace bytes of [`sample_rows`] (`kmax` as there).
pub fn sample_workspace_bytes(rows: usize, vocab: usize, kmax: i32) -> usize {
    unsafe { ffi::gbs_sample_workspace_bytes(rows as i32, vocab as i32, kmax) }
}

/// The extended pipeline: penalties over `counts` (i32 `[rows, vocab]`, may be null), the grammar `mask` (u32
/// `[rows, ceil(vocab / 32)]`, may be null), temperature, top-k / top-p / min-p and the inverse-CDF draw from
/// `uniforms[row]`, exact in integer masses. `kmax` in [1, 64]: every row's top_k is in [1, kmax] (one pass); 0: the
/// full-distribution path; [`KMAX_MIXED`]: per-row dispatch. Outputs other than `out_ids` may be null.
pub unsafe fn sample_rows(logits: *const c_void, dtype: i32, rows: usize, stride: usize, vocab: usize, counts: *const i32, mask: *const u32,
                          params: *const RowParams, uniforms: *const f32, kmax: i32, out_ids: *mut i32, out_greedy: *mut i32,
                          out_probs: *mut f32, out_logprobs: *mut f32, out_status: *mut i32, ws: *mut c_void, ws_bytes: usize,
                          stream: *mut c_void) -> Result<(), GbsError> {
    GbsError::check(ffi::gbs_sample_rows(logits, dtype, i(rows)?, i(stride)?, i(vocab)?, counts, mask, params, uniforms, kmax, out_ids,
                                         out_greedy, out_probs, out_logprobs, out_status, ws, ws_bytes, stream))
}

/// [`sample_rows`] without a workspace argument, for callers that cannot allocate (graph capture, tight serving loops):
/// the library's static [`NOALLOC_SCRATCH_BYTES`] per GPU serves it. Calls on one GPU must not overlap.
pub unsafe fn sample_rows_noalloc(logits: *const c_void, dtype: i32, rows: usize, stride: usize, vocab: usize, counts: *const i32,
                                  mask: *const u32, params: *const RowParams, uniforms: *const f32, kmax: i32, out_ids: *mut i32,
                                  out_greedy: *mut i32, out_probs: *mut f32, out_logprobs: *mut f32, out_status: *mut i32,
                                  stream: *mut c_void) -> Result<(), GbsError> {
    GbsError::check(ffi::gbs_sample_rows_noalloc(logits, dtype, i(rows)?, i(stride)?, i(vocab)?, counts, mask, params, uniforms, kmax,
                                                 out_ids, out_greedy, out_probs, out_logprobs, out_status, stream))
}

/// Workspace bytes of [`spec_verify`].
pub fn spec_verify_workspace_bytes(n_seq: usize, width: usize, vocab: usize) -> usize {
    unsafe { ffi::gbs_spec_verify_workspace_bytes(n_seq as i32, width as i32, vocab as i32) }
}

/// Speculative verification by rejection, exact in integer masses: n_seq sequences of `width` drafts and one bonus row
/// (f32 target and draft logits `[n_seq * (width + 1), stride]`, columns `[0, vocab)` read).
pub unsafe fn spec_verify(target: *const f32, draft: *const f32, n_seq: usize, width: usize, vocab: usize, stride: usize,
                          draft_ids: *const i32,
                          temperatures: *const f32, u_accept: *const f32, u_resample: *const f32, out_accepted: *mut i32,
                          out_tokens: *mut i32, out_status: *mut i32, ws: *mut c_void, ws_bytes: usize,
                          stream: *mut c_void) -> Result<(), GbsError> {
    GbsError::check(ffi::gbs_spec_verify(target, draft, i(n_seq)?, i(width)?, i(vocab)?, i(stride)?, draft_ids, temperatures, u_accept, u_resample,
                                         out_accepted, out_tokens, out_status, ws, ws_bytes, stream))
}

/// A [`KeyedRow`] for one request: `gb_sampling::Sampling`'s fields (crates/sampling/src/lib.rs:28-68) at the absolute
/// position the engine samples.
pub fn keyed_row(seed: u64, temperature: f64, top_k: usize, top_p: f64, min_p: f64, position: u64) -> KeyedRow {
    KeyedRow { seed, first_position: position, temperature, top_p, min_p, top_k: top_k as i32, keyed: 1 }
}
