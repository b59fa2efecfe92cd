/*
 * gbs_sample.h -- C ABI of the MI355X (gfx950) token-sampling library `libgbsample_hip.so`.
 *
 * Two groups of entry points:
 *
 *  1. Drop-ins for the launchers REXL3's model runtime binds for this path (same names, same argument meaning, same
 *     return codes). Each declaration cites the reference launcher it replaces.
 *  2. `gbs_*` entry points with no single reference launcher: the fused keyed sampler (top-(k+8) plus the keyed draw of
 *     `crates/sampling::try_choose` in one launch), the device accept steps of `crates/spec`, and the extended pipeline
 *     (penalties, grammar mask, temperature, top-k/top-p/min-p, inverse-CDF draw from a caller uniform, speculative
 *     rejection acceptance).
 *
 * Conventions (all entry points; they follow crates/cuda/csrc/common.cuh:1-12 and crates/cuda/csrc/glue.cu:1076-1104):
 *  - raw device pointers; `stream` is a hipStream_t passed as void* (NULL = the default stream);
 *  - launches are asynchronous and never synchronise the stream;
 *  - return 0 on success, GBS_ERR_INVALID (1, the value of hipErrorInvalidValue and cudaErrorInvalidValue) for an
 *    argument outside the contract (nothing is launched), otherwise the HIP launch error;
 *  - rows == 0 is a successful no-op;
 *  - the caller owns every buffer and workspace and keeps them alive until the stream has drained them.
 *
 * Row status codes mirror `gb_sampling::SamplingError` (crates/sampling/src/lib.rs:70-76).
 */
#ifndef GBS_SAMPLE_H
#define GBS_SAMPLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GBS_OK 0
#define GBS_ERR_INVALID 1
/* gbs_sample_rows_noalloc: the call needs more workspace than its static scratch holds (2, hipErrorOutOfMemory) */
#define GBS_ERR_NOALLOC_TOO_LARGE 2

/* per-row status (crates/sampling/src/lib.rs:70-76) */
#define GBS_ROW_OK 0
#define GBS_ROW_NO_CANDIDATES 1
#define GBS_ROW_NAN_LOGIT 2
#define GBS_ROW_INVALID_PARAMS 3

/* logits element types */
#define GBS_DTYPE_F32 0
#define GBS_DTYPE_BF16 1
#define GBS_DTYPE_F16 2

/* Largest vocabulary the extended pipeline accepts: 2^19 tokens keeps every row's integer mass sum below 2^63. */
#define GBS_MAX_VOCAB 524288
/* Candidates per row of the exact top-count kernels (crates/cuda/csrc/glue.cu:1088). */
#define GBS_MAX_COUNT 64
/* gbs_sample_rows's `kmax` for a batch that mixes rows of any top_k (per-row dispatch). */
#define GBS_KMAX_MIXED (-1)

/*
 * The keyed sampling record of one row, 48 bytes, field for field the `KeyedRow` of crates/cuda/csrc/glm_mtp.cu:258-264:
 * the row samples `try_choose` at absolute position first_position + depth.
 */
typedef struct GbsKeyedRow {
    uint64_t seed;
    uint64_t first_position;
    double temperature;
    double top_p;
    double min_p;
    int32_t top_k;
    int32_t keyed;
} GbsKeyedRow;

/*
 * The extended pipeline's per-row parameters (32 bytes). No reference counterpart: REXL3 refuses penalties and grammar
 * masks (crates/server/src/api.rs:196-206). Per element, with c = counts[i]:
 *   l = x;  if c > 0: l = (l > 0 ? l * (1/repetition) : l * repetition);  l = l - ((float)c * frequency + presence);
 *   if the mask bit of i is clear: l = -inf.
 * temperature 0 is exact greedy. top_k 0 = off. top_p outside (0,1) = off. min_p 0 = off.
 */
typedef struct GbsRowParams {
    float temperature;
    float top_p;
    float min_p;
    float repetition;
    float presence;
    float frequency;
    int32_t top_k;
    int32_t reserved;
} GbsRowParams;

/* ------------------------------------------------------------------------------------------------------------------
 * 1. Reference drop-ins
 * ------------------------------------------------------------------------------------------------------------------ */

/* Replaces crates/cuda/csrc/glue.cu:1078-1081 (gb_topk_valid_workspace_bytes). 0 for a shape outside the contract. */
size_t gb_topk_valid_workspace_bytes(int rows, int valid, int count);
/* Replaces crates/cuda/csrc/glue.cu:1083 (gb_topk_workspace_bytes). */
size_t gb_topk_workspace_bytes(int rows, int vocab, int count);

/*
 * Replaces crates/cuda/csrc/glue.cu:1089-1100 (gb_topk_valid). bf16 logits [rows, stride]; per row the exact `count`
 * largest of columns [0, valid) by (value desc, id asc); NaN is ordered and reported as -inf, -0 ties +0 (and is
 * reported as +0). ids i32 [rows, count], vals f32 [rows, count]. 1 <= count <= min(64, valid), valid <= stride.
 * Workspace: gb_topk_valid_workspace_bytes(rows, valid, count) bytes, 16-byte aligned; contents on entry do not matter.
 */
int gb_topk_valid(const void* logits, int rows, int stride, int valid, int count, int* ids, float* vals, void* workspace,
                  size_t ws_bytes, void* stream);
/* Replaces crates/cuda/csrc/glue.cu:1103-1106 (gb_topk): gb_topk_valid with valid == stride == vocab. */
int gb_topk(const void* logits, int rows, int vocab, int count, int* ids, float* vals, void* workspace, size_t ws_bytes,
            void* stream);

/*
 * Replaces crates/cuda/csrc/nemotron_glue.cu:504-522 (gb_nemo_glue_topk). f32 logits [rows, vocab]; the exact `count`
 * largest by (value desc, id asc) with -0 == +0 and NaN below -inf (NaNs among themselves by id); values are returned
 * as stored (NaN payload and zero sign kept). `blocks` >= 1 is the caller's block plan (crates/cuda/src/nemotron_glue.rs:172-176);
 * the workspace must hold rows * blocks * 8 * count * 8 bytes, 8-byte aligned. The result does not depend on `blocks`.
 * 1 <= count <= min(64, vocab), rows <= 65535.
 */
int gb_nemo_glue_topk(const void* logits, int rows, int vocab, int count, int blocks, void* ws, size_t ws_bytes, void* ids,
                      void* vals, void* stream);

/* Replaces crates/cuda/csrc/glm_glue.cu:270-315 (gb_glm_topk_f16_workspace_bytes / gb_glm_topk_f16): gb_topk_valid on
 * fp16 logits (NaN ordered and reported as -inf, -0 ties +0 and is reported as +0). */
size_t gb_glm_topk_f16_workspace_bytes(int rows, int valid, int count);
int gb_glm_topk_f16(const void* logits, int rows, int stride, int valid, int count, int* ids, float* vals, void* workspace,
                    size_t ws_bytes, void* stream);

/* Replaces crates/cuda/csrc/ling_kda_proj_fused.cu:2735-2764 (gb_ling_topk_f16_workspace_bytes / gb_ling_topk_f16):
 * gb_glm_topk_f16's results in ONE launch (the row's last chunk block merges the row's lists). Workspace: 256 bytes of
 * per-row arrival counters, then gb_glm_topk_f16_workspace_bytes(rows, valid, count); 16-byte aligned; the counters
 * must be zero before the first call (clear the workspace once, e.g. gbs_workspace_clear) and every call leaves them
 * zero. rows <= 64 (the counter region's capacity; more rows return GBS_ERR_INVALID). */
size_t gb_ling_topk_f16_workspace_bytes(int rows, int valid, int count);
int gb_ling_topk_f16(const void* logits, int rows, int stride, int valid, int count, int* ids, float* vals, void* workspace,
                     size_t ws_bytes, void* stream);

/*
 * Replace crates/cuda/csrc/dflash2.cu:595-660 (gb_dflash_selector_walk_keyed / _ragged / gb_dflash_selector_walk): the
 * draft head's selector chain walk, one sequence per block. Row i of a sequence scores its k (<= 64) candidates as
 * topk_vals[c] + <pred_codebook[prev] * gate[row], succ_codebook[topk_ids[c]]> (f16 codebooks [V, rank]; gate bf16,
 * or f32 when gate_is_f32) with the reference kernel's float arithmetic, and picks with the sequence's WalkSampling
 * (48 bytes: u64 seed, u64 first_position, f64 temperature, top_p, min_p, i32 keyed; nullable = every sequence
 * unkeyed): keyed = the device try_choose over all k at first_position + i (NaN scores last); unkeyed = the first
 * maximum. anchor i32 [n_seq]; topk_ids i32 / topk_vals f32 [rows total, k]; out_tokens i32 and conf f32 (nullable,
 * the pick's score) per row; margin (nullable, ragged form) the pick's lead over the runner-up. The ragged form takes
 * row_off i32 [n_seq + 1] (sequence b owns rows row_off[b] .. row_off[b + 1]).
 */
int gb_dflash_selector_walk_keyed(const void* anchor, const void* topk_ids, const void* topk_vals, const void* gate, int gate_is_f32,
                                  const void* pred_codebook, const void* succ_codebook, int n_seq, int rows, int k, int rank,
                                  const void* sampling, void* out_tokens, void* conf, void* stream);
int gb_dflash_selector_walk_ragged(const void* anchor, const void* topk_ids, const void* topk_vals, const void* gate, int gate_is_f32,
                                   const void* pred_codebook, const void* succ_codebook, int n_seq, int k, int rank, const void* sampling,
                                   const void* row_off, void* out_tokens, void* conf, void* margin, void* stream);
int gb_dflash_selector_walk(const void* anchor, const void* topk_ids, const void* topk_vals, const void* gate, int gate_is_f32,
                            const void* pred_codebook, const void* succ_codebook, int n_seq, int rows, int k, int rank,
                            void* out_tokens, void* conf, void* stream);

/*
 * Replace crates/cuda/csrc/dsv4_mtp_gpu.cu:1662-1718 (gb_dsv4_mtp_markov_walk_fast_bf16 / _keyed_bf16; Rust bindings
 * crates/cuda/src/dsv4_mtp_gpu.rs:55-67): the DSV4 draft head's Markov walk over walk_rows rows of logits f32
 * [walk_rows, vocab] (vocab >= 1024). Row k's 1024 candidates are each of 256 threads' 4 largest logits of
 * v = t, t + 256, ...; each gains <embed[ids[k]], head[v]> (bf16 [vocab, 256], rank must be 256) in place, with the
 * reference kernel's float arithmetic; ids[k + 1] is their maximum (fast) or the keyed choose over their top cand_k
 * (1..64) at base_pos + k, conf[k] (nullable) = 1 / (1 + exp(-margin)). ids i32 [walk_rows + 1], ids[0] the input
 * token. Workspaces: cand_ids_ws i32 [walk_rows, 1024], cand_scores_ws f32 [1024] (16-byte aligned, like embed and
 * head). Two launches per row after one for the candidates; each row's pick sorts its 1024 keys in registers.
 */
int gb_dsv4_mtp_markov_walk_fast_bf16(void* logits, int* ids, const void* embed, const void* head, void* cand_ids_ws,
                                      void* cand_scores_ws, int walk_rows, int vocab, int rank, void* stream);
int gb_dsv4_mtp_markov_walk_keyed_bf16(void* logits, int* ids, float* conf, const void* embed, const void* head, void* cand_ids_ws,
                                       void* cand_scores_ws, int walk_rows, int vocab, int rank, int cand_k, unsigned long long seed,
                                       double temperature, double top_p, double min_p, unsigned long long base_pos, void* stream);
/* The same keyed walk with cand_k, seed, temperature, top_p, min_p and base_pos read on the device from params, a
 * DEVICE pointer to the 72-byte Dsv4MtpRoundParams (crates/cuda/src/dsv4_mtp_gpu.rs:2683-2701; the reference's
 * gb_dsv4_mtp_markov_walk_keyed_bf16_params, dsv4_mtp_gpu.cu:1720-1760). */
int gb_dsv4_mtp_markov_walk_keyed_bf16_params(void* logits, int* ids, float* conf, const void* embed, const void* head,
                                              void* cand_ids_ws, void* cand_scores_ws, int walk_rows, int vocab, int rank,
                                              const void* params, void* stream);

/*
 * Replaces crates/cuda/csrc/glm_mtp.cu:272-280 (gb_glm_keyed_pick). ids i32 / vals f32 [rows, count] sorted by
 * (value desc, id asc), count <= 64; params GbsKeyedRow[rows]. A keyed row with temperature > 0 takes
 * `try_choose` (crates/sampling/src/lib.rs:210-267) over its first min(top_k, count) candidates (top_k 0 = all) at
 * position first_position + depth; any other row takes the first candidate. out_ids i32 / out_vals f32 [rows].
 */
int gb_glm_keyed_pick(const int* ids, const float* vals, int count, int rows, const void* params, int depth, int* out_ids,
                      float* out_vals, void* stream);

/* Replaces crates/cuda/csrc/qfn_verify.cu:33-40 (gb_qfn_greedy_gather): column 0 of each candidate row; the value is
 * NaN when any of the row's `count` candidates is NaN. */
int gb_qfn_greedy_gather(const void* ids, const void* vals, int count, int rows, void* out_ids, void* out_vals, void* stream);

/* Replaces crates/cuda/csrc/dsv4_mtp_gpu.cu:981-985 (gb_dsv4_mtp_argmax; Rust binding crates/cuda/src/dsv4_mtp_gpu.rs:119):
 * out i32 [rows] = per row of logits f32 [rows, vocab] the lowest id of the largest value above -inf (NaN never
 * counts, +0 and -0 are equal), 0 when the row has none. */
int gb_dsv4_mtp_argmax(const float* logits, int* out, int rows, int vocab, void* stream);

/* Replaces crates/cuda/csrc/mtp.cu:162-166 (gb_mtp_pick; Rust binding crates/cuda/src/mtpk.rs:24, 119-127): one row of
 * bf16 logits [n]; out_id i32 [j] = its argmax as above, out_p f32 [j] = 1 / sum_i exp(x_i - max), the maximum's
 * softmax probability (NaN when the row holds a NaN or has no finite maximum). Returns 1 for n < 1. */
int gb_mtp_pick(const void* logits, int n, void* out_id, void* out_p, int j, void* stream);

/* ------------------------------------------------------------------------------------------------------------------
 * 2. Fused and extended entry points
 * ------------------------------------------------------------------------------------------------------------------ */

/*
 * Fills `bytes` bytes of a workspace with zeros by a kernel (not hipMemset, so it may be captured in a HIP graph).
 * The gbs_* workspaces hold per-row arrival counters that must be zero before the first call; every call leaves them
 * zero again. Calls that share one workspace must not overlap.
 */
int gbs_workspace_clear(void* ws, size_t bytes, void* stream);

/*
 * Fused keyed sampler: per row, the exact top-(top_k + 8) of logits[row, 0..valid) (dtype f32 / bf16 / f16 with the NaN
 * rules of the matching drop-in above) and then `try_choose` (crates/sampling/src/lib.rs:210-267) over those candidates
 * at position params[row].first_position + depth: what REXL3's decode round computes with gb_topk / gb_nemo_glue_topk,
 * download_candidates and try_choose (crates/engine/src/lib.rs:2089-2117), without the candidate readback.
 * params[row].top_k must be in [1, 56] (the API cap, crates/server/src/api.rs:43-44) -- otherwise the row's status is
 * GBS_ROW_INVALID_PARAMS, as it is for the parameter checks of Sampling::validate (crates/sampling/src/lib.rs:56-67).
 * `keyed` is ignored: every row is sampled.
 * out_ids i32 [rows] (-1 on error), out_vals f32 [rows] (the chosen candidate's value; may be NULL),
 * out_status i32 [rows] (may be NULL). Workspace: gbs_keyed_sample_workspace_bytes(rows, valid), 256-byte aligned,
 * zeroed once (gbs_workspace_clear).
 */
size_t gbs_keyed_sample_workspace_bytes(int rows, int valid);
int gbs_keyed_sample_rows(const void* logits, int dtype, int rows, int stride, int valid, const GbsKeyedRow* params, int depth,
                          int* out_ids, float* out_vals, int* out_status, void* ws, size_t ws_bytes, void* stream);

/*
 * Chain accept (crates/spec/src/lib.rs:30-35): for each of n_seq sequences, the longest prefix with
 * drafts[s, i] == samples[s, i], i < width. drafts i32 [n_seq, width], samples i32 [n_seq, width + 1],
 * accepted i32 [n_seq].
 */
int gbs_accept(const int* drafts, const int* samples, int n_seq, int width, int* accepted, void* stream);

/*
 * Tree accept (crates/spec/src/tree.rs:417-438): per tree, from row 0 follow the first child whose token equals the
 * node's sample. tokens / parents / samples i32 [n_tree, nodes] (parents[0] = -1, parents come first);
 * path i32 [n_tree, nodes] (the accepted rows root first, then -1), path_len i32 [n_tree].
 */
int gbs_accept_tree(const int* tokens, const int* parents, const int* samples, int n_tree, int nodes, int* path, int* path_len,
                    void* stream);

/*
 * A tree round committed on the device (crates/engine/src/lib.rs:2376-2410: every row keyed-sampled at its own
 * position, then crates/spec/src/tree.rs:417-438's accept walk). logits [n_tree * nodes, stride] (f32 / bf16 / f16, as
 * gbs_keyed_sample_rows; columns [0, valid)); params GbsKeyedRow[n_tree * nodes], row r's first_position = the
 * position the engine samples that node at (the sequence's length plus the node's depth); tokens / parents i32
 * [n_tree, nodes] as gbs_accept_tree. Outputs: out_samples i32 [n_tree * nodes] (the keyed samples, -1 for a failed
 * row), out_path i32 [n_tree, nodes] and out_path_len i32 [n_tree] (as gbs_accept_tree), out_status i32 [n_tree] (the
 * first failed row's status: a tree with a failed row has path_len 0 and an all -1 path, as the engine fails the
 * sequence). n_tree * nodes <= 65535. The committed tokens are out_samples at the path's rows.
 */
size_t gbs_tree_verify_workspace_bytes(int n_tree, int nodes, int valid);
int gbs_tree_verify(const void* logits, int dtype, int n_tree, int nodes, int stride, int valid, const GbsKeyedRow* params,
                    const int* tokens, const int* parents, int* out_samples, int* out_path, int* out_path_len, int* out_status,
                    void* ws, size_t ws_bytes, void* stream);

/*
 * Extended sampling pipeline. logits [rows, stride] (dtype f32, bf16 or f16; 16-bit values widened exactly), columns
 * [0, vocab);
 * counts i32 [rows, vocab] (NULL = all zero); mask u32 [rows, ceil(vocab/32)] (bit i%32 of word i/32 set = token
 * allowed; NULL = all allowed); params GbsRowParams[rows]; uniforms f32 [rows], each in [0, 1).
 * `kmax` in [1, 64] promises top_k in [1, kmax] on every row and selects the single-pass kernel (a row that breaks the
 * promise gets GBS_ROW_INVALID_PARAMS); kmax == 0 selects the multi-pass full-distribution path (any top_k, 0 = off).
 * kmax == GBS_KMAX_MIXED dispatches per row, for a batch that mixes them (as REXL3's engine sends its decode rounds,
 * crates/engine/src/lib.rs:2089-2117): every row takes the single-pass kernel, which finishes rows with top_k in
 * [1, 64] and, from its best 64 candidates and the row's log-sum-exp, the rows with top_k 0 or above 64 whose top-p /
 * min-p cut provably lies among those candidates; the other rows are finished by the full-distribution path in a
 * second launch. Results are the same as with kmax 0.
 * Outputs (any but out_ids may be NULL): out_ids i32 [rows] (-1 on error), out_greedy i32 [rows] (argmax, ties to the
 * lowest id), out_probs f32 [rows] (probability of the chosen token in the final kept distribution),
 * out_logprobs f32 [rows] (log-softmax of the chosen token over every allowed token at temperature T, or 1 when T == 0),
 * out_status i32 [rows].
 * Workspace: gbs_sample_workspace_bytes(rows, vocab, kmax), 256-byte aligned, zeroed once (gbs_workspace_clear).
 * vocab <= GBS_MAX_VOCAB.
 */
size_t gbs_sample_workspace_bytes(int rows, int vocab, int kmax);
int gbs_sample_rows(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts, const uint32_t* mask,
                    const GbsRowParams* params, const float* uniforms, int kmax, int* out_ids, int* out_greedy, float* out_probs,
                    float* out_logprobs, int* out_status, void* ws, size_t ws_bytes, void* stream);

/*
 * Allocation-free gbs_sample_rows. No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments, meaning
 * and results as gbs_sample_rows without `ws` / `ws_bytes`: the workspace is a static device array of
 * GBS_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends and cleared by the first call on each GPU. A call
 * whose gbs_sample_workspace_bytes(rows, vocab, kmax) exceeds it returns GBS_ERR_NOALLOC_TOO_LARGE with nothing
 * launched. No hipMalloc, hipFree or allocating library call is made. Every call on one GPU shares its array: calls
 * that overlap on one GPU (other streams, other host threads) race and must be serialised by the caller.
 */
#define GBS_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int gbs_sample_rows_noalloc(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts,
                            const uint32_t* mask, const GbsRowParams* params, const float* uniforms, int kmax, int* out_ids,
                            int* out_greedy, float* out_probs, float* out_logprobs, int* out_status, void* stream);

/*
 * Speculative verification by rejection (Leviathan et al. 2023 / Chen et al. 2023), exact in integer masses.
 * n_seq sequences of `width` drafts + 1 bonus row: target and draft f32 logits [n_seq * (width + 1), stride], columns
 * [0, vocab) read, stride >= vocab (row s * (width + 1) + j; draft rows j == width are not read); draft_ids i32
 * [n_seq, width]; temperatures f32
 * [n_seq * (width + 1)]; u_accept f32 [n_seq, width] and u_resample f32 [n_seq], all in [0, 1).
 * Draft j is accepted iff u_accept * q(x) < p(x), p and q the softmax at the row's temperature (temperature 0: x must be
 * the target's argmax). At the first rejection the token is drawn from max(p - q, 0) (the target's argmax at
 * temperature 0); after `width` acceptances the bonus token is drawn from the last row's p.
 * out_accepted i32 [n_seq]; out_tokens i32 [n_seq, width + 1] (accepted drafts, then the drawn token, then -1);
 * out_status i32 [n_seq] (may be NULL). Workspace: gbs_spec_verify_workspace_bytes(n_seq, width, vocab), zeroed once.
 */
size_t gbs_spec_verify_workspace_bytes(int n_seq, int width, int vocab);
int gbs_spec_verify(const float* target, const float* draft, int n_seq, int width, int vocab, int stride, const int* draft_ids,
                    const float* temperatures, const float* u_accept, const float* u_resample, int* out_accepted,
                    int* out_tokens, int* out_status, void* ws, size_t ws_bytes, void* stream);

/* Test hook (no counterpart in the reference). When the row pass's grid is resident at once, the row-pass blocks of
 * gbs_spec_verify sweep their sequence's draw row themselves once the sequence is decided. Each waits at most `ticks`
 * of the device's 100 MHz clock for the decision (default 10000, 100 us); a block that waits longer leaves the sweep
 * to the exact pass. Sets the limit for later calls from this process (ticks >= 0) and returns the previous one. A
 * limit of 0 forces the fallback on every sequence whose deciding block is not the first to look; the results are
 * the same either way. */
int64_t gbs_spec_set_fuse_wait(int64_t ticks);

/* Library version string. */
const char* gbs_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GBS_SAMPLE_H */
