/*
 * CPU oracle of the token-sampling path. TEST INFRASTRUCTURE ONLY: the tests, the smoke check and the bench's
 * cpu_baseline leg load it as the checker; the product library never links, loads or calls it.
 *
 * Two halves:
 *  - Mode K: a plain-C restatement of REXL3's keyed sampler and accept steps (crates/sampling/src/lib.rs,
 *    crates/spec/src/lib.rs:30-35, crates/spec/src/tree.rs:417-438, crates/spec/src/draft_pick.rs:58-64) and of the
 *    device top-k contracts (crates/cuda/csrc/glue.cu:509-534, crates/cuda/csrc/nemotron_glue.cu:22-34, 191-203,
 *    crates/cuda/csrc/glm_mtp.cu:266-297, crates/cuda/csrc/qfn_verify.cu:11-29).
 *  - Mode U: the definition of the extended pipeline (penalties, grammar mask, temperature, top-k/top-p/min-p, the
 *    inverse-CDF draw from one caller uniform, rejection acceptance). The reference has no code for it
 *    (crates/server/src/api.rs:196-206 refuses these features); this file is its specification.
 */
#ifndef GBS_ORACLE_H
#define GBS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/gbs_sample.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Sampling (crates/sampling/src/lib.rs:28-36). */
typedef struct GboSampling {
    uint64_t seed;
    double temperature;
    uint64_t top_k;
    double top_p;
    double min_p;
} GboSampling;

/* ---- Mode K: crates/sampling ---- */
uint64_t gbo_mix(uint64_t x);
double gbo_unit_open(uint64_t x);
double gbo_uniform(uint64_t seed, uint64_t position, uint64_t id);
double gbo_pairwise_sum(const double* a, size_t n);
uint64_t gbo_seed_for(const uint32_t* tokens, size_t n, uint64_t salt);
void gbo_sha256(const uint8_t* data, size_t n, uint8_t out[32]);
int gbo_validate(const GboSampling* s);
uint64_t gbo_candidate_count(const GboSampling* s, uint64_t vocab);
/* returns a GBS_ROW_* status; LengthMismatch cannot occur (one n for both arrays) */
int gbo_try_choose(const float* values, const uint32_t* ids, size_t n, uint64_t position, const GboSampling* s, uint32_t* out);
int gbo_try_top_candidates(const float* logits, size_t n, size_t count, uint32_t* ids, float* vals);
size_t gbo_accept(const uint32_t* drafts, size_t nd, const uint32_t* samples, size_t ns);
size_t gbo_accept_tree(const uint32_t* tokens, const int32_t* parents, const uint32_t* samples, size_t n, size_t* path);

/* ---- Mode K: device contracts ---- */
/* gb_nemo_glue_topk row contract: f32, NaN below -inf, -0 == +0, stable by id, values as stored */
void gbo_topk_f32_row(const float* row, int vocab, int count, int32_t* ids, float* vals);
/* gb_topk_valid row contract: bf16 bits, NaN -> -inf, -0 -> +0, values decoded from the order key */
void gbo_topk_bf16_row(const uint16_t* row, int valid, int count, int32_t* ids, float* vals);
/* gb_glm_topk_f16 row contract: fp16 bits, NaN -> -inf, -0 -> +0 */
void gbo_topk_f16_row(const uint16_t* row, int valid, int count, int32_t* ids, float* vals);
/* gb_glm_keyed_pick, one row */
void gbo_keyed_pick_row(const int32_t* ids, const float* vals, int count, const GbsKeyedRow* p, int depth, int32_t* out_id,
                        float* out_val);
/* gbs_keyed_sample_rows, one row: top-(top_k+8) under the dtype's contract, then try_choose */
int gbo_keyed_sample_row(const void* row, int dtype, int valid, const GbsKeyedRow* p, int depth, int32_t* out_id, float* out_val);

/* ---- Mode U ---- */
typedef struct GboSampleOut {
    int32_t id;
    int32_t greedy;
    float prob;
    double logprob;
    int32_t status;
    int32_t kept;     /* size of the final kept set */
    uint64_t z_kept;  /* integer mass of the kept set */
} GboSampleOut;

int gbo_row_params_invalid(const GbsRowParams* p, float u);
float gbo_penalized_logit(float x, int32_t count, const GbsRowParams* p, float rinv);
uint32_t gbo_order_key_f32(float v);
uint64_t gbo_mass(float l, float lmax, float c2);
float gbo_temp_scale(float temperature);
uint64_t gbo_mul_floor(float x, uint64_t z, int* exact);
void gbo_sample_row(const void* logits, int dtype, int vocab, const int32_t* counts, const uint32_t* mask, const GbsRowParams* p,
                    float u, GboSampleOut* out);

typedef struct GboSpecOut {
    int32_t accepted;
    int32_t status;
} GboSpecOut;
void gbo_spec_verify_seq(const float* target, const float* draft, int width, int vocab, const int32_t* draft_ids,
                         const float* temperatures, const float* u_accept, float u_resample, int32_t* tokens, GboSpecOut* out);

/* ---- batch drivers (CPU baseline; rows split over `threads` pthreads) ---- */
int gbo_batch_keyed_sample(const void* logits, int dtype, int rows, int stride, int valid, const GbsKeyedRow* params, int depth,
                           int32_t* out_ids, int threads);
int gbo_batch_sample(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts,
                     const uint32_t* mask, const GbsRowParams* params, const float* uniforms, int32_t* out_ids,
                     int32_t* out_greedy, float* out_probs, double* out_logprobs, int32_t* out_status, int threads);
int gbo_batch_spec_verify(const float* target, const float* draft, int n_seq, int width, int vocab, const int32_t* draft_ids,
                          const float* temperatures, const float* u_accept, const float* u_resample, int32_t* out_accepted,
                          int32_t* out_tokens, int32_t* out_status, int threads);


/* The draft head's selector walk (crates/cuda/csrc/dflash2.cu:436-519) and its keyed choice (crates/cuda/csrc/keyed.cuh:50-112).
 * GboWalkSampling is the 48-byte WalkSampling record (dflash2.cu:436-441). */
typedef struct {
    uint64_t seed, first_position;
    double temperature, top_p, min_p;
    int32_t keyed;
    int32_t pad;
} GboWalkSampling;
int gbo_keyed_choose(const float* scores, const int32_t* c_row, int k, uint64_t seed, double temperature, double top_p, double min_p,
                     uint64_t position, float* margin);
void gbo_selector_walk(const int32_t* anchor, const int32_t* ids, const float* vals, const void* gate, int gate_f32,
                       const uint16_t* pred_cb, const uint16_t* succ_cb, int n_seq, int rows, int k, int rank,
                       const GboWalkSampling* ws, const int32_t* row_off, int32_t* out, float* conf, float* margin);

/* The DSV4 draft head's Markov walk (crates/cuda/csrc/dsv4_mtp_gpu.cu:1233-1480, 1662-1718). logits f32
 * [walk_rows, vocab] (the candidates' logits gain their bias in place); ids i32 [walk_rows + 1] (ids[0] in, ids[1..]
 * out); embed / head bf16 bits [vocab, 256]; keyed = 0: argmax, 1: keyed choose over the top cand_k (conf: the
 * sigmoid of its margin, nullable). */
void gbo_markov_walk(float* logits, int32_t* ids, float* conf, const uint16_t* embed, const uint16_t* head, int walk_rows, int vocab,
                     int keyed, int cand_k, uint64_t seed, double temperature, double top_p, double min_p, uint64_t base_pos);
/* draft-head argmax picks: crates/cuda/csrc/dsv4_mtp_gpu.cu:503-539 and crates/cuda/csrc/mtp.cu:78-117 */
void gbo_row_argmax(const float* logits, int rows, int vocab, int32_t* out);
void gbo_mtp_pick(const uint16_t* logits, int n, int32_t* out_id, float* out_p);

#ifdef __cplusplus
}
#endif
#endif
