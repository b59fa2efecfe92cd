/*
 * CPU oracle of the token-sampling path -- TEST INFRASTRUCTURE ONLY (the checker for the tests, the smoke check and
 * the bench's cpu_baseline leg; the product library never links or calls it).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math). Every floating-point operation below is a single
 * IEEE-754 operation in the order written; fmaf is the fused multiply-add, rounded once.
 *
 * Mode K follows the reference file by file (citations at each function). Mode U is specified here; see the comment
 * block above gbo_sample_row.
 */
#include "gbs_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

/* =====================================================================================================================
 * Mode K -- crates/sampling/src/lib.rs
 * ===================================================================================================================== */

/* splitmix64 finaliser: crates/sampling/src/lib.rs:122-129 */
uint64_t gbo_mix(uint64_t x) {
    x ^= x >> 30;
    x *= 0xBF58476D1CE4E5B9ULL;
    x ^= x >> 27;
    x *= 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

/* (x >> 11) * 2^-53 + 2^-54, capped at the largest double below 1: crates/sampling/src/lib.rs:131-141 */
double gbo_unit_open(uint64_t x) {
    const double two_m53 = 1.0 / 9007199254740992.0;
    const double v = (double)(x >> 11) * two_m53 + two_m53 / 2.0;
    const double below_one = 1.0 - two_m53;
    return v < below_one ? v : below_one;
}

/* crates/sampling/src/lib.rs:143-150 */
double gbo_uniform(uint64_t seed, uint64_t position, uint64_t id) {
    uint64_t x = gbo_mix(seed + 0x9E3779B97F4A7C15ULL);
    x = gbo_mix(x ^ (position * 0xD1B54A32D192ED03ULL));
    x = gbo_mix(x ^ id);
    return gbo_unit_open(x);
}

/* numpy's float64 pairwise sum: crates/sampling/src/lib.rs:152-181 */
double gbo_pairwise_sum(const double* a, size_t n) {
    if (n < 8) {
        double r = 0.0;
        for (size_t i = 0; i < n; ++i) r += a[i];
        return r;
    }
    if (n <= 128) {
        double r[8];
        for (int j = 0; j < 8; ++j) r[j] = a[j];
        size_t i = 8;
        for (; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; ++j) r[j] += a[i + j];
        double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; ++i) res += a[i];
        return res;
    }
    size_t n2 = n / 2;
    n2 -= n2 % 8;
    return gbo_pairwise_sum(a, n2) + gbo_pairwise_sum(a + n2, n - n2);
}

/* ---- SHA-256 (FIPS 180-4), for seed_for ---- */
static uint32_t rotr32(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static const uint32_t SHA_K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5, 0xd807aa98, 0x12835b01,
    0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc,
    0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147,
    0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116, 0x1e376c08,
    0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3, 0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208,
    0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

typedef struct {
    uint32_t h[8];
    uint8_t buf[64];
    size_t fill;
    uint64_t bytes;
} Sha256;

static void sha_init(Sha256* s) {
    static const uint32_t h0[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(s->h, h0, sizeof h0);
    s->fill = 0;
    s->bytes = 0;
}

static void sha_block(Sha256* s, const uint8_t* p) {
    uint32_t w[64];
    for (int i = 0; i < 16; ++i) w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
        const uint32_t s0 = rotr32(w[i - 15], 7) ^ rotr32(w[i - 15], 18) ^ (w[i - 15] >> 3);
        const uint32_t s1 = rotr32(w[i - 2], 17) ^ rotr32(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = s->h[0], b = s->h[1], c = s->h[2], d = s->h[3], e = s->h[4], f = s->h[5], g = s->h[6], h = s->h[7];
    for (int i = 0; i < 64; ++i) {
        const uint32_t S1 = rotr32(e, 6) ^ rotr32(e, 11) ^ rotr32(e, 25);
        const uint32_t ch = (e & f) ^ (~e & g);
        const uint32_t t1 = h + S1 + ch + SHA_K[i] + w[i];
        const uint32_t S0 = rotr32(a, 2) ^ rotr32(a, 13) ^ rotr32(a, 22);
        const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
        const uint32_t t2 = S0 + mj;
        h = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    s->h[0] += a; s->h[1] += b; s->h[2] += c; s->h[3] += d; s->h[4] += e; s->h[5] += f; s->h[6] += g; s->h[7] += h;
}

static void sha_update(Sha256* s, const uint8_t* p, size_t n) {
    s->bytes += n;
    while (n) {
        size_t take = 64 - s->fill;
        if (take > n) take = n;
        memcpy(s->buf + s->fill, p, take);
        s->fill += take;
        p += take;
        n -= take;
        if (s->fill == 64) {
            sha_block(s, s->buf);
            s->fill = 0;
        }
    }
}

static void sha_final(Sha256* s, uint8_t out[32]) {
    const uint64_t bits = s->bytes * 8;
    uint8_t pad = 0x80;
    sha_update(s, &pad, 1);
    const uint8_t zero = 0;
    while (s->fill != 56) sha_update(s, &zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    sha_update(s, len, 8);
    for (int i = 0; i < 8; ++i) {
        out[4 * i] = (uint8_t)(s->h[i] >> 24);
        out[4 * i + 1] = (uint8_t)(s->h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(s->h[i] >> 8);
        out[4 * i + 3] = (uint8_t)s->h[i];
    }
}

void gbo_sha256(const uint8_t* data, size_t n, uint8_t out[32]) {
    Sha256 s;
    sha_init(&s);
    sha_update(&s, data, n);
    sha_final(&s, out);
}

static void sha_decimal(Sha256* s, uint64_t v) {
    uint8_t buf[20];
    int i = 20;
    do {
        buf[--i] = (uint8_t)('0' + v % 10);
        v /= 10;
    } while (v);
    sha_update(s, buf + i, (size_t)(20 - i));
}

/* sha256 of "t0,t1,...|salt", first 8 bytes little endian, top bit cleared: crates/sampling/src/lib.rs:95-120 */
uint64_t gbo_seed_for(const uint32_t* tokens, size_t n, uint64_t salt) {
    Sha256 s;
    sha_init(&s);
    for (size_t i = 0; i < n; ++i) {
        if (i) sha_update(&s, (const uint8_t*)",", 1);
        sha_decimal(&s, tokens[i]);
    }
    sha_update(&s, (const uint8_t*)"|", 1);
    sha_decimal(&s, salt);
    uint8_t d[32];
    sha_final(&s, d);
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = v << 8 | d[i];
    return v & ((1ULL << 63) - 1);
}

/* Sampling::validate: crates/sampling/src/lib.rs:56-67 */
int gbo_validate(const GboSampling* s) {
    if (!isfinite(s->temperature) || s->temperature < 0.0) return GBS_ROW_INVALID_PARAMS;
    if (!isfinite(s->top_p) || !(s->top_p >= 0.0 && s->top_p <= 1.0)) return GBS_ROW_INVALID_PARAMS;
    if (!isfinite(s->min_p) || !(s->min_p >= 0.0 && s->min_p <= 1.0)) return GBS_ROW_INVALID_PARAMS;
    return GBS_ROW_OK;
}

/* crates/sampling/src/lib.rs:45-52 (MARGIN = 8, :26) */
uint64_t gbo_candidate_count(const GboSampling* s, uint64_t vocab) {
    if (s->top_k == 0) return vocab;
    uint64_t c = s->top_k + 8 < s->top_k ? UINT64_MAX : s->top_k + 8;
    return c < vocab ? c : vocab;
}

/* (value desc, id asc), stable: numpy lexsort((ids, -values)), crates/sampling/src/lib.rs:183-191 */
static int before_vi(float va, uint32_t ia, size_t pa, float vb, uint32_t ib, size_t pb) {
    if (va > vb) return 1;
    if (va < vb) return 0;
    if (ia != ib) return ia < ib;
    return pa < pb;
}

static void order_idx(const float* v, const uint32_t* ids, size_t n, size_t* idx) {
    for (size_t i = 0; i < n; ++i) idx[i] = i;
    /* stable binary-insertion sort; n is a candidate list */
    for (size_t i = 1; i < n; ++i) {
        const size_t x = idx[i];
        size_t lo = 0, hi = i;
        while (lo < hi) {
            const size_t mid = (lo + hi) / 2;
            if (before_vi(v[x], ids[x], x, v[idx[mid]], ids[idx[mid]], idx[mid])) hi = mid;
            else lo = mid + 1;
        }
        memmove(idx + lo + 1, idx + lo, (i - lo) * sizeof(size_t));
        idx[lo] = x;
    }
}

/* try_choose: crates/sampling/src/lib.rs:206-267 */
int gbo_try_choose(const float* values, const uint32_t* ids, size_t n, uint64_t position, const GboSampling* s, uint32_t* out) {
    const int v = gbo_validate(s);
    if (v) return v;
    if (n == 0) return GBS_ROW_NO_CANDIDATES;
    for (size_t i = 0; i < n; ++i)
        if (isnan(values[i])) return GBS_ROW_NAN_LOGIT;
    if (s->temperature == 0.0) {
        size_t best = 0;
        for (size_t i = 1; i < n; ++i)
            if (values[i] > values[best] || (values[i] == values[best] && ids[i] < ids[best])) best = i;
        *out = ids[best];
        return GBS_ROW_OK;
    }
    size_t* ord = (size_t*)malloc(n * sizeof(size_t));
    double* scaled = (double*)malloc(n * sizeof(double));
    double* probs = (double*)malloc(n * sizeof(double));
    order_idx(values, ids, n, ord);
    size_t k = s->top_k > 0 ? (s->top_k < n ? (size_t)s->top_k : n) : n;
    if (k < 1) k = 1;
    const double t = s->temperature > 1e-6 ? s->temperature : 1e-6;
    for (size_t i = 0; i < k; ++i) scaled[i] = (double)values[ord[i]] / t;
    size_t keep = k;
    if (s->top_p > 0.0 && s->top_p < 1.0) {
        double mx = -INFINITY;
        for (size_t i = 0; i < k; ++i) mx = fmax(mx, scaled[i]);
        for (size_t i = 0; i < k; ++i) probs[i] = exp(scaled[i] - mx);
        const double total = gbo_pairwise_sum(probs, k);
        for (size_t i = 0; i < k; ++i) probs[i] /= total;
        double c = 0.0;
        size_t below = 0;
        for (size_t i = 0; i < k; ++i) {
            c += probs[i];
            if (c < s->top_p) ++below;
        }
        keep = below + 1 < k ? below + 1 : k;
    }
    if (s->min_p > 0.0) {
        const double floor_v = scaled[0] + log(s->min_p);
        size_t cnt = 0;
        for (size_t i = 0; i < keep; ++i)
            if (scaled[i] >= floor_v) ++cnt;
        keep = cnt > 1 ? cnt : 1;
    }
    size_t best = 0;
    double best_score = -INFINITY;
    for (size_t i = 0; i < keep; ++i) {
        const uint32_t id = ids[ord[i]];
        const double u = gbo_uniform(s->seed, position, id);
        const double g = -log(-log(u));
        const double score = scaled[i] + g;
        if (score > best_score) {
            best_score = score;
            best = i;
        }
    }
    *out = ids[ord[best]];
    free(ord);
    free(scaled);
    free(probs);
    return GBS_ROW_OK;
}

/*
 * Exact top-`count` of a logits row by (value desc, id asc): crates/sampling/src/lib.rs:282-305. A NaN anywhere is an
 * error. Scans once keeping a sorted list; an element enters only if strictly greater than the list's last value (a tie
 * never displaces a lower id, which came first).
 */
int gbo_try_top_candidates(const float* logits, size_t n, size_t count, uint32_t* ids, float* vals) {
    for (size_t i = 0; i < n; ++i)
        if (isnan(logits[i])) return GBS_ROW_NAN_LOGIT;
    const size_t take = count < n ? count : n;
    size_t len = 0;
    for (size_t i = 0; i < n; ++i) {
        const float v = logits[i];
        if (len == take && !(v > vals[len - 1])) continue;
        if (take == 0) break;
        size_t lo = 0, hi = len;
        while (lo < hi) { /* first position whose value is < v (ties stay ahead: lower id) */
            const size_t mid = (lo + hi) / 2;
            if (vals[mid] >= v) lo = mid + 1;
            else hi = mid;
        }
        const size_t last = len < take ? len : take - 1;
        memmove(vals + lo + 1, vals + lo, (last - lo) * sizeof(float));
        memmove(ids + lo + 1, ids + lo, (last - lo) * sizeof(uint32_t));
        vals[lo] = v;
        ids[lo] = (uint32_t)i;
        if (len < take) ++len;
    }
    return GBS_ROW_OK;
}

/* crates/spec/src/lib.rs:30-35 */
size_t gbo_accept(const uint32_t* drafts, size_t nd, const uint32_t* samples, size_t ns) {
    size_t a = 0;
    while (a < nd && a < ns && drafts[a] == samples[a]) ++a;
    return a;
}

/* crates/spec/src/tree.rs:417-438; path receives the accepted rows, returns their number */
size_t gbo_accept_tree(const uint32_t* tokens, const int32_t* parents, const uint32_t* samples, size_t n, size_t* path) {
    size_t len = 0, cur = 0;
    path[len++] = 0;
    for (;;) {
        const uint32_t s = samples[cur];
        size_t next = n;
        for (size_t r = cur + 1; r < n; ++r)
            if (parents[r] == (int32_t)cur && tokens[r] == s) {
                next = r;
                break;
            }
        if (next == n) return len;
        path[len++] = next;
        cur = next;
    }
}

/* =====================================================================================================================
 * Mode K -- the device contracts
 * ===================================================================================================================== */

/* f32 order key of crates/cuda/csrc/nemotron_glue.cu:191-203: NaN -> 0 (below -inf), -0 == +0 */
static uint32_t nemo_key32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0;
    if ((u << 1) == 0) return 0x80000000u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct {
    uint64_t key;
    int32_t id;
} KeyId;

/* the `count` largest u64 keys (distinct by construction: the low word is ~id) */
static void top_keys(const uint32_t* hi, int n, int count, KeyId* out) {
    int len = 0;
    for (int i = 0; i < n; ++i) {
        const uint64_t k = (uint64_t)hi[i] << 32 | (uint32_t)~(uint32_t)i;
        if (len == count && k <= out[len - 1].key) continue;
        int pos = len < count ? len : count - 1;
        while (pos > 0 && out[pos - 1].key < k) {
            out[pos] = out[pos - 1];
            --pos;
        }
        out[pos].key = k;
        out[pos].id = i;
        if (len < count) ++len;
    }
}

void gbo_topk_f32_row(const float* row, int vocab, int count, int32_t* ids, float* vals) {
    uint32_t* k = (uint32_t*)malloc((size_t)vocab * 4);
    for (int i = 0; i < vocab; ++i) k[i] = nemo_key32(row[i]);
    KeyId* t = (KeyId*)malloc((size_t)count * sizeof(KeyId));
    top_keys(k, vocab, count, t);
    for (int i = 0; i < count; ++i) {
        ids[i] = t[i].id;
        vals[i] = row[t[i].id];
    }
    free(k);
    free(t);
}

/* 16-bit float order key of crates/cuda/csrc/glue.cu:529-534 (bf16) and crates/cuda/csrc/glm_glue.cu:105-110 (fp16):
 * NaN -> -inf, -0 -> +0, then the sign-flip map */
static uint32_t key16(uint16_t u, uint16_t exp_mask, uint16_t neg_inf) {
    if ((u & 0x7FFF) > exp_mask) u = neg_inf;
    else if ((u & 0x7FFF) == 0) u = 0;
    return (u & 0x8000) ? (~(uint32_t)u & 0xFFFF) : ((uint32_t)u | 0x8000);
}

static float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    int e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    uint32_t u;
    if (e == 31) u = s | 0x7F800000u | (m << 13);
    else if (e == 0) {
        if (m == 0) u = s;
        else { /* subnormal: normalise */
            int sh = 0;
            while (!(m & 0x400)) {
                m <<= 1;
                ++sh;
            }
            m &= 0x3FF;
            u = s | (uint32_t)(113 - sh) << 23 | (m << 13);
        }
    } else u = s | (uint32_t)(e + 112) << 23 | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static void topk16_row(const uint16_t* row, int valid, int count, int32_t* ids, float* vals, int is_f16) {
    uint32_t* k = (uint32_t*)malloc((size_t)valid * 4);
    for (int i = 0; i < valid; ++i) k[i] = is_f16 ? key16(row[i], 0x7C00, 0xFC00) : key16(row[i], 0x7F80, 0xFF80);
    KeyId* t = (KeyId*)malloc((size_t)count * sizeof(KeyId));
    top_keys(k, valid, count, t);
    for (int i = 0; i < count; ++i) {
        ids[i] = t[i].id;
        const uint32_t tk = (uint32_t)(t[i].key >> 32);
        const uint16_t u = (uint16_t)((tk & 0x8000) ? (tk & 0x7FFF) : (~tk & 0xFFFF));
        vals[i] = is_f16 ? f16_to_f32(u) : bf16_to_f32(u);
    }
    free(k);
    free(t);
}

void gbo_topk_bf16_row(const uint16_t* row, int valid, int count, int32_t* ids, float* vals) { topk16_row(row, valid, count, ids, vals, 0); }
void gbo_topk_f16_row(const uint16_t* row, int valid, int count, int32_t* ids, float* vals) { topk16_row(row, valid, count, ids, vals, 1); }

/* keyed_pick_k: crates/cuda/csrc/glm_mtp.cu:266-280, its choose = try_choose over the first k candidates */
void gbo_keyed_pick_row(const int32_t* ids, const float* vals, int count, const GbsKeyedRow* p, int depth, int32_t* out_id,
                        float* out_val) {
    int pick = 0;
    if (p->keyed && p->temperature > 0.0) {
        const int k = (p->top_k > 0 && p->top_k < count) ? p->top_k : count;
        GboSampling s = {p->seed, p->temperature, (uint64_t)k, p->top_p, p->min_p};
        uint32_t uid[64] = {0};
        for (int i = 0; i < k; ++i) uid[i] = (uint32_t)ids[i];
        uint32_t chosen = 0;
        if (gbo_try_choose(vals, uid, (size_t)k, p->first_position + (uint64_t)depth, &s, &chosen) == GBS_ROW_OK) {
            for (int i = 0; i < k; ++i)
                if (uid[i] == chosen) {
                    pick = i;
                    break;
                }
        }
    }
    *out_id = ids[pick];
    *out_val = vals[pick];
}

int gbo_keyed_sample_row(const void* row, int dtype, int valid, const GbsKeyedRow* p, int depth, int32_t* out_id, float* out_val) {
    *out_id = -1;
    if (out_val) *out_val = NAN;
    GboSampling s = {p->seed, p->temperature, (uint64_t)(p->top_k > 0 ? p->top_k : 0), p->top_p, p->min_p};
    if (p->top_k < 1 || p->top_k > 56 || gbo_validate(&s)) return GBS_ROW_INVALID_PARAMS;
    const int count = p->top_k + 8 < valid ? p->top_k + 8 : valid;
    int32_t ids[64];
    float vals[64];
    if (dtype == GBS_DTYPE_F32) gbo_topk_f32_row((const float*)row, valid, count, ids, vals);
    else if (dtype == GBS_DTYPE_BF16) gbo_topk_bf16_row((const uint16_t*)row, valid, count, ids, vals);
    else gbo_topk_f16_row((const uint16_t*)row, valid, count, ids, vals);
    uint32_t uid[64];
    for (int i = 0; i < count; ++i) uid[i] = (uint32_t)ids[i];
    uint32_t chosen;
    const int st = gbo_try_choose(vals, uid, (size_t)count, p->first_position + (uint64_t)depth, &s, &chosen);
    if (st) return st;
    *out_id = (int32_t)chosen;
    if (out_val)
        for (int i = 0; i < count; ++i)
            if (uid[i] == chosen) {
                *out_val = vals[i];
                break;
            }
    return GBS_ROW_OK;
}

/* =====================================================================================================================
 * Mode U -- the extended pipeline (no reference code; this is its definition)
 *
 * Per row, with x the logit (bf16 widened exactly), c the count, all float operations f32 IEEE in the order written:
 *   1. penalties:   if c > 0: l = (x > 0 ? x * rinv : x * rep), rinv = 1.0f / rep;  l = l - ((float)c * freq + pres)
 *   2. mask:        bit (i & 31) of word i >> 5 clear -> l = -inf
 *   3. a NaN l is the row error NanLogit; the allowed set A = {i : l_i > -inf}; A empty -> NoCandidates.
 *   4. order:       (l desc, id asc) with -0 == +0. greedy = first of A in that order.
 *   5. T == 0:      the token is greedy.
 *   6. masses:      M = l_greedy, c2 = 1.44269504f / T (f32 division). E(l) = 2^44 if l == M; else y = (l - M) * c2,
 *                   0 unless y >= -64; n = rintf(y), f = y - n (exact), p = 2^f by a degree-7 Taylor polynomial in fmaf
 *                   Horner form, m = (u32)(p * 2^24) (exact), E = m * 2^(n + 20), truncated. E(M) = 2^44, E <= 2^44.
 *   7. top-k:       K = the first min(top_k, |A|) of A in order (all of A when top_k == 0).
 *   8. top-p:       if 0 < top_p < 1: P = ceil(top_p * Z_K) exactly; keep = min(1 + #{j : C_j < P}, |K|), where C_j is
 *                   the inclusive prefix mass in order (crates/sampling/src/lib.rs:241-251's rule, in integers).
 *   9. min-p:       if min_p > 0: Q = ceil(min_p * 2^44); the kept set is {j < keep : E_j >= Q} (a filter on the
 *                   top-p prefix; it holds the first token, whose mass is 2^44 >= Q). The reference's rule
 *                   (crates/sampling/src/lib.rs:253-259) counts and truncates, which is the same set whenever the
 *                   masses are monotone along the order.
 *  10. draw:        Z = sum of the kept masses; t = floor(u * Z) exactly; the kept tokens taken in ascending id order, the
 *                   token is the first whose running mass sum exceeds t.
 *  prob = (float)((double)E_token / (double)Z); logprob = log-softmax over A at temperature T (1 when T == 0), double
 *  (NaN when the maximum is +inf, or when 1/T overflows f32: a subnormal temperature, for which every token but the
 *  maximum has probability 0 to within any f32 arithmetic).
 * ===================================================================================================================== */

uint32_t gbo_order_key_f32(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u << 1) == 0) return 0x80000000u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

float gbo_penalized_logit(float x, int32_t count, const GbsRowParams* p, float rinv) {
    float l = x;
    if (count > 0) {
        l = (l > 0.0f) ? l * rinv : l * p->repetition;
        const float a = (float)count * p->frequency;
        const float b = a + p->presence;
        l = l - b;
    }
    return l;
}

float gbo_temp_scale(float temperature) { return 1.44269504088896340736f / temperature; }

/* 2^f for f in [-0.5, 0.5]: Taylor series of exp(f ln 2) to degree 7 (coefficients (ln 2)^j / j!), Horner in fmaf */
static float pow2_frac(float f) {
    float p = 1.52527338e-05f;
    p = fmaf(p, f, 1.54035304e-04f);
    p = fmaf(p, f, 1.33335581e-03f);
    p = fmaf(p, f, 9.61812911e-03f);
    p = fmaf(p, f, 5.55041087e-02f);
    p = fmaf(p, f, 2.40226507e-01f);
    p = fmaf(p, f, 6.93147181e-01f);
    p = fmaf(p, f, 1.0f);
    return p;
}

uint64_t gbo_mass(float l, float lmax, float c2) {
    if (l == lmax) return 1ULL << 44;
    const float d = l - lmax;
    const float y = d * c2;
    if (!(y >= -64.0f)) return 0;
    const float n = rintf(y);
    const float f = y - n;
    const float p = pow2_frac(f);
    const uint32_t m = (uint32_t)(p * 16777216.0f);
    const int sh = (int)n + 20;
    if (sh >= 0) return (uint64_t)m << sh;
    if (sh <= -32) return 0;
    return (uint64_t)(m >> -sh);
}

/* floor(x * z) for finite x >= 0, exactly; *exact says whether the product was an integer */
static u128 mul_floor128(float x, u128 z, int* exact) {
    uint32_t b;
    memcpy(&b, &x, 4);
    const uint32_t e = (b >> 23) & 0xFF;
    uint64_t m = b & 0x7FFFFF;
    int sh;
    if (e == 0) sh = 149;
    else {
        m |= 0x800000;
        sh = 150 - (int)e;
    }
    if (m == 0 || z == 0) {
        if (exact) *exact = 1;
        return 0;
    }
    /* 152-bit product in three words */
    const u128 lo = (u128)m * (uint64_t)z;
    const u128 hi = (u128)m * (uint64_t)(z >> 64);
    uint64_t w0 = (uint64_t)lo;
    const u128 mid = (lo >> 64) + (uint64_t)hi;
    uint64_t w1 = (uint64_t)mid;
    uint64_t w2 = (uint64_t)((hi >> 64) + (mid >> 64));
    if (sh <= 0) { /* x >= 2^23: not used by the pipeline; left shift */
        if (exact) *exact = 1;
        return ((u128)w1 << 64 | w0) << (-sh);
    }
    int ex = 1;
    /* check and drop the low sh bits */
    int s = sh;
    while (s >= 64) {
        if (w0) ex = 0;
        w0 = w1;
        w1 = w2;
        w2 = 0;
        s -= 64;
    }
    if (s > 0) {
        if (w0 & ((1ULL << s) - 1)) ex = 0;
        w0 = (w0 >> s) | (w1 << (64 - s));
        w1 = (w1 >> s) | (w2 << (64 - s));
        w2 >>= s;
    }
    if (exact) *exact = ex;
    return (u128)w1 << 64 | w0;
}

uint64_t gbo_mul_floor(float x, uint64_t z, int* exact) { return (uint64_t)mul_floor128(x, z, exact); }

static uint64_t mul_ceil64(float x, uint64_t z) {
    int ex;
    const uint64_t f = (uint64_t)mul_floor128(x, z, &ex);
    return f + (ex ? 0 : 1);
}

static float load_logit(const void* logits, int dtype, size_t i) {
    if (dtype == GBS_DTYPE_BF16) return bf16_to_f32(((const uint16_t*)logits)[i]);
    if (dtype == GBS_DTYPE_F16) return f16_to_f32(((const uint16_t*)logits)[i]);
    return ((const float*)logits)[i];
}

static int cand_before(uint32_t ka, int ia, uint32_t kb, int ib) { return ka > kb || (ka == kb && ia < ib); }

static int by_id_asc(const void* a, const void* b) {
    const int x = *(const int*)a, y = *(const int*)b;
    return (x > y) - (x < y);
}

typedef struct {
    uint32_t k;
    int id;
} OKey;

static int okey_desc(const void* a, const void* b) {
    const OKey* x = (const OKey*)a;
    const OKey* y = (const OKey*)b;
    if (x->k != y->k) return x->k > y->k ? -1 : 1;
    return (x->id > y->id) - (x->id < y->id);
}

int gbo_row_params_invalid(const GbsRowParams* p, float u) {
    if (!(isfinite(p->temperature) && p->temperature >= 0.0f)) return 1;
    if (!(p->top_p >= 0.0f && p->top_p <= 1.0f)) return 1;
    if (!(p->min_p >= 0.0f && p->min_p <= 1.0f)) return 1;
    if (!(isfinite(p->repetition) && p->repetition > 0.0f)) return 1;
    if (!isfinite(p->presence) || !isfinite(p->frequency)) return 1;
    if (p->top_k < 0) return 1;
    if (!(u >= 0.0f && u < 1.0f)) return 1;
    return 0;
}

void gbo_sample_row(const void* logits, int dtype, int vocab, const int32_t* counts, const uint32_t* mask, const GbsRowParams* p,
                    float u, GboSampleOut* out) {
    out->id = -1;
    out->greedy = -1;
    out->prob = 0.0f;
    out->logprob = NAN;
    out->kept = 0;
    out->z_kept = 0;
    if (gbo_row_params_invalid(p, u)) {
        out->status = GBS_ROW_INVALID_PARAMS;
        return;
    }
    const float rinv = 1.0f / p->repetition;
    float* l = (float*)malloc((size_t)vocab * sizeof(float));
    int nan = 0, g = -1;
    uint32_t gk = 0;
    size_t n_allowed = 0;
    for (int i = 0; i < vocab; ++i) {
        float v = gbo_penalized_logit(load_logit(logits, dtype, (size_t)i), counts ? counts[i] : 0, p, rinv);
        if (mask && !((mask[i >> 5] >> (i & 31)) & 1u)) v = -INFINITY;
        if (isnan(v)) nan = 1;
        l[i] = v;
        if (v > -INFINITY) {
            ++n_allowed;
            const uint32_t k = gbo_order_key_f32(v);
            if (g < 0 || k > gk) {
                g = i;
                gk = k;
            }
        }
    }
    if (nan) {
        out->status = GBS_ROW_NAN_LOGIT;
        free(l);
        return;
    }
    if (g < 0) {
        out->status = GBS_ROW_NO_CANDIDATES;
        free(l);
        return;
    }
    out->greedy = g;
    const float T = p->temperature;
    const float M = l[g];
    if (T == 0.0f) {
        out->id = g;
        out->prob = 1.0f;
        out->kept = 1;
    } else {
        const float c2 = gbo_temp_scale(T);
        size_t kk = n_allowed;
        if (p->top_k > 0 && (size_t)p->top_k < kk) kk = (size_t)p->top_k;
        OKey* cand = (OKey*)malloc(kk * sizeof(OKey));
        if (kk == n_allowed) {
            size_t j = 0;
            for (int i = 0; i < vocab; ++i)
                if (l[i] > -INFINITY) {
                    cand[j].k = gbo_order_key_f32(l[i]);
                    cand[j].id = i;
                    ++j;
                }
            qsort(cand, kk, sizeof(OKey), okey_desc);
        } else { /* bounded insertion: a later id never displaces an equal key */
            size_t len = 0;
            for (int i = 0; i < vocab; ++i) {
                if (!(l[i] > -INFINITY)) continue;
                const uint32_t k = gbo_order_key_f32(l[i]);
                if (len == kk && !cand_before(k, i, cand[len - 1].k, cand[len - 1].id)) continue;
                size_t pos = len < kk ? len : kk - 1;
                while (pos > 0 && cand_before(k, i, cand[pos - 1].k, cand[pos - 1].id)) {
                    cand[pos] = cand[pos - 1];
                    --pos;
                }
                cand[pos].k = k;
                cand[pos].id = i;
                if (len < kk) ++len;
            }
        }
        uint64_t* E = (uint64_t*)malloc(kk * sizeof(uint64_t));
        uint64_t zk = 0;
        for (size_t j = 0; j < kk; ++j) {
            E[j] = gbo_mass(l[cand[j].id], M, c2);
            zk += E[j];
        }
        size_t keep = kk;
        if (p->top_p > 0.0f && p->top_p < 1.0f) {
            const uint64_t P = mul_ceil64(p->top_p, zk);
            uint64_t c = 0;
            size_t below = 0;
            for (size_t j = 0; j < kk; ++j) {
                c += E[j];
                if (c < P) ++below;
            }
            keep = below + 1 < kk ? below + 1 : kk;
        }
        /* min-p filters the prefix: a token stays if its mass is at least Q (the first token, of mass 2^44, always does) */
        const uint64_t Q = p->min_p > 0.0f ? mul_ceil64(p->min_p, 1ULL << 44) : 0;
        uint64_t z = 0;
        size_t nk = 0;
        int* byid = (int*)malloc(keep * sizeof(int) * 2);
        for (size_t j = 0; j < keep; ++j) {
            if (E[j] < Q) continue;
            z += E[j];
            byid[2 * nk] = cand[j].id;
            byid[2 * nk + 1] = (int)j;
            ++nk;
        }
        const uint64_t t = (uint64_t)mul_floor128(u, z, NULL);
        /* ascending id order over the kept set: E is indexed by rank, so sort (id, rank) pairs */
        qsort(byid, nk, sizeof(int) * 2, by_id_asc);
        uint64_t acc = 0;
        int chosen = -1;
        uint64_t ec = 0;
        for (size_t j = 0; j < nk; ++j) {
            acc += E[byid[2 * j + 1]];
            if (acc > t) {
                chosen = byid[2 * j];
                ec = E[byid[2 * j + 1]];
                break;
            }
        }
        out->id = chosen;
        out->prob = (float)((double)ec / (double)z);
        out->kept = (int32_t)nk;
        out->z_kept = z;
        free(byid);
        free(E);
        free(cand);
    }
    /* logprob over A, double */
    {
        const double Tp = T > 0.0f ? (double)T : 1.0;
        const double m = (double)M;
        double s = 0.0;
        if (isinf(M) || (T > 0.0f && isinf(gbo_temp_scale(T)))) { /* undefined: a +inf maximum, or 1/T beyond f32 */
            out->logprob = NAN;
        } else {
            for (int i = 0; i < vocab; ++i)
                if (l[i] > -INFINITY) s += exp(((double)l[i] - m) / Tp);
            out->logprob = ((double)l[out->id] - m) / Tp - log(s);
        }
    }
    out->status = GBS_ROW_OK;
    free(l);
}

/* ---- speculative verification ---- */

/* argmax by (l desc, id asc), -1 if every entry is -inf; *nan set on a NaN */
static int row_argmax(const float* r, int vocab, int* nan) {
    int g = -1;
    uint32_t gk = 0;
    for (int i = 0; i < vocab; ++i) {
        const float v = r[i];
        if (isnan(v)) {
            *nan = 1;
            continue;
        }
        if (v > -INFINITY) {
            const uint32_t k = gbo_order_key_f32(v);
            if (g < 0 || k > gk) {
                g = i;
                gk = k;
            }
        }
    }
    return g;
}

/* Z = sum of masses of a row whose maximum is r[g] */
static uint64_t row_mass_sum(const float* r, int vocab, float M, float c2) {
    uint64_t z = 0;
    for (int i = 0; i < vocab; ++i)
        if (r[i] > -INFINITY) z += gbo_mass(r[i], M, c2);
    return z;
}

void gbo_spec_verify_seq(const float* target, const float* draft, int width, int vocab, const int32_t* draft_ids,
                         const float* temperatures, const float* u_accept, float u_resample, int32_t* tokens, GboSpecOut* out) {
    for (int j = 0; j <= width; ++j) tokens[j] = -1;
    out->accepted = 0;
    int bad = !(u_resample >= 0.0f && u_resample < 1.0f);
    for (int j = 0; j <= width; ++j) bad |= !(isfinite(temperatures[j]) && temperatures[j] >= 0.0f);
    for (int j = 0; j < width; ++j) bad |= !(u_accept[j] >= 0.0f && u_accept[j] < 1.0f) || draft_ids[j] < 0 || draft_ids[j] >= vocab;
    if (bad) {
        out->status = GBS_ROW_INVALID_PARAMS;
        return;
    }
    int nan = 0, empty = 0;
    for (int j = 0; j <= width; ++j) {
        empty |= row_argmax(target + (size_t)j * vocab, vocab, &nan) < 0;
        if (j < width) empty |= row_argmax(draft + (size_t)j * vocab, vocab, &nan) < 0;
    }
    if (nan || empty) {
        out->status = nan ? GBS_ROW_NAN_LOGIT : GBS_ROW_NO_CANDIDATES;
        return;
    }
    out->status = GBS_ROW_OK;
    for (int j = 0; j <= width; ++j) {
        const float* tr = target + (size_t)j * vocab;
        const float T = temperatures[j];
        int dummy = 0;
        const int gp = row_argmax(tr, vocab, &dummy);
        if (j == width) { /* bonus: a draw from p */
            int tok = gp;
            if (T > 0.0f) {
                const float c2 = gbo_temp_scale(T);
                const uint64_t zp = row_mass_sum(tr, vocab, tr[gp], c2);
                const uint64_t t = (uint64_t)mul_floor128(u_resample, zp, NULL);
                uint64_t acc = 0;
                for (int i = 0; i < vocab; ++i) {
                    if (!(tr[i] > -INFINITY)) continue;
                    acc += gbo_mass(tr[i], tr[gp], c2);
                    if (acc > t) {
                        tok = i;
                        break;
                    }
                }
            }
            tokens[j] = tok;
            out->accepted = width;
            return;
        }
        const int x = draft_ids[j];
        int accept;
        const float* dr = draft + (size_t)j * vocab;
        uint64_t zp = 0, zq = 0;
        float c2 = 0.0f;
        int gq = -1;
        if (T == 0.0f) accept = (x == gp);
        else {
            c2 = gbo_temp_scale(T);
            gq = row_argmax(dr, vocab, &dummy);
            zp = row_mass_sum(tr, vocab, tr[gp], c2);
            zq = row_mass_sum(dr, vocab, dr[gq], c2);
            const uint64_t ep = tr[x] > -INFINITY ? gbo_mass(tr[x], tr[gp], c2) : 0;
            const uint64_t eq = dr[x] > -INFINITY ? gbo_mass(dr[x], dr[gq], c2) : 0;
            const u128 a = (u128)eq * zp;
            const u128 b = (u128)ep * zq;
            accept = mul_floor128(u_accept[j], a, NULL) < b;
        }
        if (accept) {
            tokens[j] = x;
            continue;
        }
        int tok = gp;
        if (T > 0.0f) { /* residual max(p - q, 0) in integers: max(Ep * Zq - Eq * Zp, 0) */
            u128 R = 0;
            for (int i = 0; i < vocab; ++i) {
                const u128 a = (u128)(tr[i] > -INFINITY ? gbo_mass(tr[i], tr[gp], c2) : 0) * zq;
                const u128 b = (u128)(dr[i] > -INFINITY ? gbo_mass(dr[i], dr[gq], c2) : 0) * zp;
                if (a > b) R += a - b;
            }
            const u128 t = mul_floor128(u_resample, R, NULL);
            u128 acc = 0;
            for (int i = 0; i < vocab; ++i) {
                const u128 a = (u128)(tr[i] > -INFINITY ? gbo_mass(tr[i], tr[gp], c2) : 0) * zq;
                const u128 b = (u128)(dr[i] > -INFINITY ? gbo_mass(dr[i], dr[gq], c2) : 0) * zp;
                if (a > b) {
                    acc += a - b;
                    if (acc > t) {
                        tok = i;
                        break;
                    }
                }
            }
        }
        tokens[j] = tok;
        out->accepted = j;
        return;
    }
}

/* =====================================================================================================================
 * Batch drivers (threads over rows)
 * ===================================================================================================================== */

typedef struct {
    int kind;
    int r0, r1;
    /* keyed */
    const void* logits;
    int dtype, stride, valid, depth;
    const GbsKeyedRow* kparams;
    int32_t* out_ids;
    /* mode U */
    int vocab;
    const int32_t* counts;
    const uint32_t* mask;
    const GbsRowParams* params;
    const float* uniforms;
    int32_t* out_greedy;
    float* out_probs;
    double* out_logprobs;
    int32_t* out_status;
    /* spec */
    const float* target;
    const float* draft;
    int width;
    const int32_t* draft_ids;
    const float* temperatures;
    const float* u_accept;
    const float* u_resample;
    int32_t* out_accepted;
    int32_t* out_tokens;
} Job;

static size_t esize(int dtype) { return dtype == GBS_DTYPE_F32 ? 4 : 2; }

static void* run_job(void* arg) {
    Job* j = (Job*)arg;
    for (int r = j->r0; r < j->r1; ++r) {
        if (j->kind == 0) {
            const char* row = (const char*)j->logits + (size_t)r * j->stride * esize(j->dtype);
            gbo_keyed_sample_row(row, j->dtype, j->valid, &j->kparams[r], j->depth, &j->out_ids[r], NULL);
        } else if (j->kind == 1) {
            const char* row = (const char*)j->logits + (size_t)r * j->stride * esize(j->dtype);
            const size_t words = ((size_t)j->vocab + 31) / 32;
            GboSampleOut o;
            gbo_sample_row(row, j->dtype, j->vocab, j->counts ? j->counts + (size_t)r * j->vocab : NULL,
                           j->mask ? j->mask + (size_t)r * words : NULL, &j->params[r], j->uniforms[r], &o);
            j->out_ids[r] = o.id;
            if (j->out_greedy) j->out_greedy[r] = o.greedy;
            if (j->out_probs) j->out_probs[r] = o.prob;
            if (j->out_logprobs) j->out_logprobs[r] = o.logprob;
            if (j->out_status) j->out_status[r] = o.status;
        } else {
            const int w = j->width;
            const size_t rows0 = (size_t)r * (w + 1);
            GboSpecOut o;
            gbo_spec_verify_seq(j->target + rows0 * j->vocab, j->draft + rows0 * j->vocab, w, j->vocab, j->draft_ids + (size_t)r * w,
                                j->temperatures + rows0, j->u_accept + (size_t)r * w, j->u_resample[r],
                                j->out_tokens + rows0, &o);
            j->out_accepted[r] = o.accepted;
            if (j->out_status) j->out_status[r] = o.status;
        }
    }
    return NULL;
}

static int run_threads(Job* base, int rows, int threads) {
    if (threads < 1) threads = 1;
    if (threads > rows) threads = rows > 0 ? rows : 1;
    pthread_t th[256];
    Job jobs[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; ++t) {
        jobs[t] = *base;
        jobs[t].r0 = (int)((long long)rows * t / threads);
        jobs[t].r1 = (int)((long long)rows * (t + 1) / threads);
    }
    if (threads == 1) {
        run_job(&jobs[0]);
        return 0;
    }
    for (int t = 0; t < threads; ++t) pthread_create(&th[t], NULL, run_job, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
    return 0;
}

int gbo_batch_keyed_sample(const void* logits, int dtype, int rows, int stride, int valid, const GbsKeyedRow* params, int depth,
                           int32_t* out_ids, int threads) {
    Job j;
    memset(&j, 0, sizeof j);
    j.kind = 0;
    j.logits = logits;
    j.dtype = dtype;
    j.stride = stride;
    j.valid = valid;
    j.kparams = params;
    j.depth = depth;
    j.out_ids = out_ids;
    return run_threads(&j, rows, threads);
}

int gbo_batch_sample(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts,
                     const uint32_t* mask, const GbsRowParams* params, const float* uniforms, int32_t* out_ids,
                     int32_t* out_greedy, float* out_probs, double* out_logprobs, int32_t* out_status, int threads) {
    Job j;
    memset(&j, 0, sizeof j);
    j.kind = 1;
    j.logits = logits;
    j.dtype = dtype;
    j.stride = stride;
    j.vocab = vocab;
    j.counts = counts;
    j.mask = mask;
    j.params = params;
    j.uniforms = uniforms;
    j.out_ids = out_ids;
    j.out_greedy = out_greedy;
    j.out_probs = out_probs;
    j.out_logprobs = out_logprobs;
    j.out_status = out_status;
    return run_threads(&j, rows, threads);
}

int gbo_batch_spec_verify(const float* target, const float* draft, int n_seq, int width, int vocab, const int32_t* draft_ids,
                          const float* temperatures, const float* u_accept, const float* u_resample, int32_t* out_accepted,
                          int32_t* out_tokens, int32_t* out_status, int threads) {
    Job j;
    memset(&j, 0, sizeof j);
    j.kind = 2;
    j.target = target;
    j.draft = draft;
    j.width = width;
    j.vocab = vocab;
    j.draft_ids = draft_ids;
    j.temperatures = temperatures;
    j.u_accept = u_accept;
    j.u_resample = u_resample;
    j.out_accepted = out_accepted;
    j.out_tokens = out_tokens;
    j.out_status = out_status;
    return run_threads(&j, n_seq, threads);
}

/* =====================================================================================================================
 * The draft head's selector walk (crates/cuda/csrc/dflash2.cu:436-519, walk_kernel; its keyed choice is
 * crates/cuda/csrc/keyed.cuh:50-112, keyed_choose).
 * ===================================================================================================================== */

/* keyed_choose: order the k <= 64 scored candidates by (score desc, id asc, NaN last) by insertion, then at temperature 0
 * the first; otherwise try_choose's steps in double over all k (top_k = k) with the Gumbel argmax keyed on `position`.
 * `margin` (nullable): the winner's lead over the runner-up in the maximised quantity, 30 with one candidate in play. */
int gbo_keyed_choose(const float* scores, const int32_t* c_row, int k, uint64_t seed, double temperature, double top_p, double min_p,
                     uint64_t position, float* margin) {
    int ord[64];
    for (int i = 0; i < k; ++i) {
        int j = i;
        while (j > 0) {
            const float va = scores[ord[j - 1]], vb = scores[i];
            const int before = (vb > va) || (vb == va && c_row[i] < c_row[ord[j - 1]]) || (va != va && vb == vb);
            if (!before) break;
            ord[j] = ord[j - 1];
            --j;
        }
        ord[j] = i;
    }
    if (temperature == 0.0) {
        if (margin) *margin = k > 1 ? scores[ord[0]] - scores[ord[1]] : 30.f;
        return ord[0];
    }
    const double t = temperature > 1e-6 ? temperature : 1e-6;
    double sc[64], pr[64] = {0};
    int keep = k;
    for (int i = 0; i < k; ++i) sc[i] = (double)scores[ord[i]] / t;
    if (top_p > 0.0 && top_p < 1.0) {
        const double mx = sc[0];
        for (int i = 0; i < k; ++i) pr[i] = exp(sc[i] - mx);
        const double total = gbo_pairwise_sum(pr, (size_t)k);
        double c = 0.0;
        int below = 0;
        for (int i = 0; i < k; ++i) {
            c += pr[i] / total;
            if (c < top_p) ++below;
        }
        keep = below + 1 < k ? below + 1 : k;
    }
    if (min_p > 0.0) {
        const double floor_v = sc[0] + log(min_p);
        int n = 0;
        for (int i = 0; i < keep; ++i)
            if (sc[i] >= floor_v) ++n;
        keep = n > 1 ? n : 1;
    }
    int best = 0;
    double best_score = -INFINITY, second_score = -INFINITY;
    for (int i = 0; i < keep; ++i) {
        const double u = gbo_uniform(seed, position, (uint64_t)(uint32_t)c_row[ord[i]]);
        const double score = sc[i] + (-log(-log(u)));
        if (score > best_score) {
            second_score = best_score;
            best_score = score;
            best = i;
        } else if (score > second_score) {
            second_score = score;
        }
    }
    if (margin) *margin = keep > 1 ? (float)fmin(best_score - second_score, 30.0) : 30.f;
    return ord[best];
}

/* walk_kernel, one sequence at a time. Row i of sequence b (rows base .. base + nrows): a_g[r] = f16 pred[prev][r] *
 * gate[row][r] (f32); score[c] = unary[c] + dot, the dot summed as the kernel's 32 lanes do (lane l: fmaf over
 * r = l, l + 32, ... in order; then the xor butterfly over offsets 16, 8, 4, 2, 1; lane 0's value); keyed rows take
 * keyed_choose at first_position + i, the others the first maximum (strict >) with the gap to the runner-up. */
void gbo_selector_walk(const int32_t* anchor, const int32_t* ids, const float* vals, const void* gate, int gate_f32,
                       const uint16_t* pred_cb, const uint16_t* succ_cb, int n_seq, int rows, int k, int rank,
                       const GboWalkSampling* ws, const int32_t* row_off, int32_t* out, float* conf, float* margin) {
    float* a_g = (float*)malloc((size_t)rank * sizeof(float));
    float scores[64];
    for (int b = 0; b < n_seq; ++b) {
        const int base = row_off ? row_off[b] : b * rows;
        const int nrows = row_off ? row_off[b + 1] - base : rows;
        int pred = anchor[b];
        for (int i = 0; i < nrows; ++i) {
            const size_t row = (size_t)(base + i);
            for (int r = 0; r < rank; ++r) {
                const float g = gate_f32 ? ((const float*)gate)[row * rank + r] : bf16_to_f32(((const uint16_t*)gate)[row * rank + r]);
                a_g[r] = f16_to_f32(pred_cb[(size_t)pred * rank + r]) * g;
            }
            const int32_t* c_row = ids + row * k;
            const float* u_row = vals + row * k;
            for (int c = 0; c < k; ++c) {
                const uint16_t* b_row = succ_cb + (size_t)c_row[c] * rank;
                float lanes[32], nl[32];
                for (int l = 0; l < 32; ++l) {
                    float dot = 0.f;
                    for (int r = l; r < rank; r += 32) dot = fmaf(a_g[r], f16_to_f32(b_row[r]), dot);
                    lanes[l] = dot;
                }
                for (int o = 16; o > 0; o >>= 1) {
                    for (int l = 0; l < 32; ++l) nl[l] = lanes[l] + lanes[l ^ o];
                    memcpy(lanes, nl, sizeof(lanes));
                }
                scores[c] = u_row[c] + lanes[0];
            }
            int best = 0;
            float bs = scores[0], mg = 30.f;
            if (ws && ws[b].keyed) {
                best = gbo_keyed_choose(scores, c_row, k, ws[b].seed, ws[b].temperature, ws[b].top_p, ws[b].min_p,
                                        ws[b].first_position + (uint64_t)i, &mg);
                bs = scores[best];
            } else {
                for (int c = 1; c < k; ++c)
                    if (scores[c] > bs) {
                        bs = scores[c];
                        best = c;
                    }
                float second = -INFINITY;
                for (int c = 0; c < k; ++c)
                    if (c != best && scores[c] > second) second = scores[c];
                mg = k > 1 ? fminf(bs - second, 30.f) : 30.f;
            }
            pred = c_row[best];
            out[row] = pred;
            if (conf) conf[row] = bs;
            if (margin) margin[row] = mg;
        }
    }
    free(a_g);
}

/* ------------------------------------------------------------------------------------------------ DSV4 Markov walk
 * crates/cuda/csrc/dsv4_mtp_gpu.cu: candidates :1233-1262 (thread t of 256 keeps the 4 largest of v = t, t + 256, ...,
 * strict >), bias :1264-1311 (per candidate, lane j of 32 sums e[8j + q] * h[8j + q] for q = 0..7 by fmaf in order, the
 * 32 partial sums reduced by the butterfly xor 16, 8, 4, 2, 1 as lane 0 sees it; the logit gains the sum in place),
 * picks :1313-1462 (non-finite scores become -inf with id 0x7fffffff; order value desc, id asc). */
static float bf16f(uint16_t h) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)h << 16;
    return c.f;
}

static int mw_before(float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); }

void gbo_markov_walk(float* logits, int32_t* ids, float* conf, const uint16_t* embed, const uint16_t* head, int walk_rows, int vocab,
                     int keyed, int cand_k, uint64_t seed, double temperature, double top_p, double min_p, uint64_t base_pos) {
    enum { NC = 1024, RANK = 256, NONE = 0x7fffffff };
    int32_t* cand = (int32_t*)malloc(sizeof(int32_t) * (size_t)walk_rows * NC);
    for (int r = 0; r < walk_rows; ++r) {
        const float* lr = logits + (size_t)r * vocab;
        for (int t = 0; t < 256; ++t) {
            float b[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            int bi[4] = {0, 0, 0, 0};
            for (int v = t; v < vocab; v += 256) {
                const float x = lr[v];
                if (!(x > b[3])) continue;
                int pos = 3;
                while (pos > 0 && x > b[pos - 1]) {
                    b[pos] = b[pos - 1];
                    bi[pos] = bi[pos - 1];
                    --pos;
                }
                b[pos] = x;
                bi[pos] = v;
            }
            for (int q = 0; q < 4; ++q) cand[(size_t)r * NC + t * 4 + q] = bi[q];
        }
    }
    float sc[NC];
    int sid[NC];
    for (int k = 0; k < walk_rows; ++k) {
        float* lr = logits + (size_t)k * vocab;
        const int tok = ids[k];
        const int ok = (unsigned)tok < (unsigned)vocab;
        for (int idx = 0; idx < NC; ++idx) {
            const int v = cand[(size_t)k * NC + idx];
            if ((unsigned)v >= (unsigned)vocab) {
                sc[idx] = -INFINITY;
                continue;
            }
            float part[32];
            for (int j = 0; j < 32; ++j) {
                float a = 0.0f;
                for (int q = 0; q < 8; ++q) {
                    const float e = ok ? bf16f(embed[(size_t)tok * RANK + j * 8 + q]) : 0.0f;
                    a = fmaf(e, bf16f(head[(size_t)v * RANK + j * 8 + q]), a);
                }
                part[j] = a;
            }
            for (int m = 16; m >= 1; m >>= 1) {
                float nx[32];
                for (int j = 0; j < 32; ++j) nx[j] = part[j] + part[j ^ m];
                memcpy(part, nx, sizeof(part));
            }
            lr[v] = lr[v] + part[0];
            sc[idx] = lr[v];
        }
        /* (value desc, id asc) order of the 1024 candidates */
        int ord[NC];
        float vv[NC];
        for (int i = 0; i < NC; ++i) {
            const int fin = isfinite(sc[i]);
            vv[i] = fin ? sc[i] : -INFINITY;
            sid[i] = fin ? cand[(size_t)k * NC + i] : NONE;
            ord[i] = i;
        }
        for (int i = 1; i < NC; ++i) { /* insertion sort: 1024 keys, a test oracle */
            const int x = ord[i];
            int j = i;
            while (j > 0 && mw_before(vv[x], sid[x], vv[ord[j - 1]], sid[ord[j - 1]])) {
                ord[j] = ord[j - 1];
                --j;
            }
            ord[j] = x;
        }
        if (!keyed) {
            const int b = sid[ord[0]];
            ids[k + 1] = b != NONE ? b : 0;
            continue;
        }
        const int kk = cand_k < 1 ? 1 : (cand_k > 64 ? 64 : cand_k);
        float ts[64];
        int32_t ti[64];
        int valid = 0;
        for (int i = 0; i < kk; ++i) {
            ts[i] = vv[ord[i]];
            ti[i] = sid[ord[i]];
        }
        while (valid < kk && isfinite(ts[valid]) && ti[valid] != NONE) ++valid;
        if (valid == 0) {
            ids[k + 1] = 0;
            if (conf) conf[k] = 0.0f;
            continue;
        }
        float margin = 30.0f;
        const int ch = gbo_keyed_choose(ts, ti, valid, seed, temperature, top_p, min_p, base_pos + (uint64_t)k, &margin);
        if (!isfinite(margin)) margin = -30.0f;
        ids[k + 1] = ti[ch] != NONE ? ti[ch] : 0;
        if (conf) conf[k] = 1.0f / (1.0f + expf(-margin));
    }
    free(cand);
}

/* ---------------------------------------------------------------------------------------------- draft-head argmax picks */

/* crates/cuda/csrc/dsv4_mtp_gpu.cu:503-539 (argmax_k): per row the first index of the largest value that is above
 * -inf (a NaN never compares greater; +0 and -0 compare equal, so the earlier one stays); 0 when there is none. */
void gbo_row_argmax(const float* logits, int rows, int vocab, int32_t* out) {
    for (int r = 0; r < rows; ++r) {
        const float* x = logits + (size_t)r * vocab;
        float bv = -INFINITY;
        int bi = 0;
        for (int i = 0; i < vocab; ++i) {
            if (x[i] > bv) {
                bv = x[i];
                bi = i;
            }
        }
        out[r] = bi;
    }
}

/* crates/cuda/csrc/mtp.cu:78-117 (pick_kernel): the argmax of a bf16 row as above (0 when no value is above -inf),
 * and p = 1 / sum_i exp(x_i - max), summed here in double (the reference sums __expf terms in float). p is NaN when
 * the row holds a NaN or its maximum is not finite (max = -inf when no value is above -inf). */
void gbo_mtp_pick(const uint16_t* logits, int n, int32_t* out_id, float* out_p) {
    float bv = -INFINITY;
    int bi = 0;
    for (int i = 0; i < n; ++i) {
        const float v = bf16_to_f32(logits[i]);
        if (v > bv) {
            bv = v;
            bi = i;
        }
    }
    double t = 0.0;
    for (int i = 0; i < n; ++i) t += exp((double)bf16_to_f32(logits[i]) - (double)bv);
    *out_id = bi;
    *out_p = (float)(1.0 / t);
}
