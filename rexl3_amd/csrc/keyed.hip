// REXL3's keyed sampler on the device.
//
//  - keyed_choose_wave: `try_choose` (crates/sampling/src/lib.rs:210-267) over a row's sorted candidates, one wave per
//    row: the top_p / min_p cuts in double exactly as the reference orders them (numpy pairwise sum and the sequential
//    cumsum run on lane 0, at most 64 terms), the Gumbel noise of each kept candidate on its own lane, and an argmax that
//    keeps the first candidate on ties, as the reference's strict `>` does.
//  - gb_glm_keyed_pick (crates/cuda/csrc/glm_mtp.cu:266-297), gb_qfn_greedy_gather (crates/cuda/csrc/qfn_verify.cu:11-40).
//  - gb_dsv4_mtp_argmax (crates/cuda/csrc/dsv4_mtp_gpu.cu:981-985), gb_mtp_pick (crates/cuda/csrc/mtp.cu:162-166): the
//    draft heads' argmax picks.
//  - gbs_keyed_sample_rows: exact top-(top_k + 8) over the full row and the keyed draw in ONE launch (keyed_fast_k: one
//    block per row, or a few per row with a last-block hand-off when there are fewer rows than CUs). Only the chosen id
//    leaves the device.
//  - gbs_accept / gbs_accept_tree: crates/spec/src/lib.rs:30-35 and crates/spec/src/tree.rs:417-438.
//  - gbs_tree_verify: a tree round on the device, keyed draws at each node's position then the accept walk.
#include <hip/hip_fp16.h>

#include "gbs_select.hpp"

using namespace gbs;
using namespace gbs::sel;

namespace {

__device__ __forceinline__ u64 sm_mix(u64 x) {
    x ^= x >> 30;
    x *= 0xBF58476D1CE4E5B9ull;
    x ^= x >> 27;
    x *= 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// crates/sampling/src/lib.rs:131-150
__device__ __forceinline__ double keyed_uniform(u64 seed, u64 position, u64 id) {
    u64 x = sm_mix(seed + 0x9E3779B97F4A7C15ull);
    x = sm_mix(x ^ (position * 0xD1B54A32D192ED03ull));
    x = sm_mix(x ^ id);
    const double two_m53 = 1.0 / 9007199254740992.0;
    const double u = (double)(x >> 11) * two_m53 + two_m53 * 0.5;
    const double below_one = 1.0 - two_m53;
    return u < below_one ? u : below_one;
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    return __longlong_as_double((long long)readlane64((u64)__double_as_longlong(v), lane));
}

// numpy's float64 pairwise sum for n <= 64 of a[i] held on lane i (the same order as pairwise_small), read lane by
// lane into scalar registers: no LDS round trip per term
__device__ __forceinline__ double pairwise_lanes(double a, int n) {
    if (n < 8) {
        double r = 0.0;
        for (int i = 0; i < n; ++i) r += readlane_f64(a, i);
        return r;
    }
    double r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = readlane_f64(a, j);
    const int full = n - (n % 8);
    // (unrolled: each block's reads are issued ahead of its additions)
#pragma unroll
    for (int b = 1; b < 8; ++b) {
        if (b * 8 < full) {
            double v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = readlane_f64(a, b * 8 + j);
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] += v[j];
        }
    }
    int i = full;
    double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += readlane_f64(a, i);
    return res;
}

// `try_choose` over vals[0..k), ids[0..k) (LDS, already in (value desc, id asc) order, no NaN), temperature > 0.
// Returns the chosen index (wave-uniform). The sums run in the reference's order on values read lane by lane (every
// lane computes the same scalar sequence); cross-lane moves are readlanes and DPP/permlane swaps, not LDS.
__device__ int keyed_choose_wave(const float* vals, const u32* ids, int k, u64 seed, double temperature, double top_p, double min_p,
                                 u64 position, float* margin = nullptr) {
    const int l = lane_id();
    const double t = temperature > 1e-6 ? temperature : 1e-6;
    const double sc = l < k ? (double)vals[l] / t : 0.0;
    const double sc0 = readlane_f64(sc, 0);
    int keep = k;
    if (top_p > 0.0 && top_p < 1.0) {
        // the maximum of `scaled` is its first entry: the values are sorted and t > 0
        const double e = l < k ? exp(sc - sc0) : 0.0;
        const double total = pairwise_lanes(e, k);
        // the quotients probs[i] / total on their own lanes (the same IEEE divisions)
        const double q = l < k ? e / total : 0.0;
        // below = the count of running sums c_i = q_0 + ... + q_i (added in order, rounded at each step) under top_p.
        // A scan across the lanes gives each lane a sum of the same terms in another order (a tree of depth 6): with
        // nonnegative terms both are within 63u and 6u of the exact sum (u = 2^-53), so a lane whose scan value is
        // below top_p / (1 + 2^-45), or at least top_p / (1 - 2^-45), has its c_i on the same side. Only when some
        // lane falls between does the ordered chain run.
        double sp = q;
#pragma unroll
        for (int m = 1; m < WAVE; m <<= 1) {
            const double o = __shfl_up(sp, (unsigned)m, WAVE);
            if (l >= m) sp += o;
        }
        const bool sure_below = sp * (1.0 + 0x1p-45) < top_p, sure_above = sp * (1.0 - 0x1p-45) >= top_p;
        int below = __popcll(ballot(l < k && sure_below));
        if (ballot(l < k && !sure_below && !sure_above)) {
            // Eight quotients at a time are read into scalar registers ahead of their additions, and the running
            // sums are compared after the chain. Lanes from k on hold 0, and adding 0 leaves a sum unchanged.
            double c = 0.0;
            below = 0;
            for (int i0 = 0; i0 < k; i0 += 8) {
                double v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = readlane_f64(q, i0 + j);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    c += v[j];
                    v[j] = c;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) below += (i0 + j < k && v[j] < top_p) ? 1 : 0;
            }
        }
        keep = below + 1 < k ? below + 1 : k;
    }
    if (min_p > 0.0) {
        const double floor_v = sc0 + log(min_p);
        const int cnt = __popcll(ballot(l < keep && sc >= floor_v));
        keep = cnt > 1 ? cnt : 1;
    }
    // Gumbel argmax; a NaN or -inf score never wins (strict >), the first index wins ties, index 0 if nothing beats -inf
    double score = -INFINITY;
    if (l < keep) {
        const double u = keyed_uniform(seed, position, (u64)ids[l]);
        score = sc + (-log(-log(u)));
    }
    const bool live = score > -INFINITY;  // false for NaN
    double best = live ? score : -INFINITY;
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1)
        best = fmax(best, __longlong_as_double((long long)xor_lane64((u64)__double_as_longlong(best), m)));
    const u64 hit = ballot(live && score == best);
    const int chosen = hit ? (int)__builtin_ctzll(hit) : 0;
    if (margin) {
        // keyed.cuh's margin: the chosen score's lead over the best other kept score, at most 30 (30 with one kept)
        double second = (live && l != chosen) ? score : -INFINITY;
#pragma unroll
        for (int m = 1; m < WAVE; m <<= 1)
            second = fmax(second, __longlong_as_double((long long)xor_lane64((u64)__double_as_longlong(second), m)));
        *margin = keep > 1 ? (float)fmin(best - second, 30.0) : 30.f;
    }
    return chosen;
}

// ------------------------------------------------------------------------------------------------ gb_glm_keyed_pick

struct KeyedRowDev {
    u64 seed, first_position;
    double temperature, top_p, min_p;
    int top_k, keyed;
};
static_assert(sizeof(KeyedRowDev) == 48, "KeyedRow is 48 bytes");

__device__ __forceinline__ bool row_before(float va, u32 ia, int pa, float vb, u32 ib, int pb) {
    const bool na = va != va, nb = vb != vb;
    if (na != nb) return nb;  // a number before a NaN
    if (!na && va != vb) return va > vb;
    if (ia != ib) return ia < ib;
    return pa < pb;
}

// one wave per row (4 rows per block)
__global__ void __launch_bounds__(256) keyed_pick_k(const int* __restrict__ ids, const float* __restrict__ vals, int count, int rows,
                                                    const KeyedRowDev* __restrict__ params, int depth, int* __restrict__ out_ids,
                                                    float* __restrict__ out_vals) {
    __shared__ float s_v[4][64];
    __shared__ u32 s_i[4][64];
    __shared__ u32 s_tid[4][64];
    const int w = threadIdx.x / WAVE, l = lane_id();
    const int r = blockIdx.x * 4 + w;
    if (r >= rows) return;
    const int* c_row = ids + (size_t)r * count;
    const float* v_row = vals + (size_t)r * count;
    const KeyedRowDev p = params[r];
    int pick = 0;
    if (p.keyed && p.temperature > 0.0) {
        const int k = p.top_k > 0 && p.top_k < count ? p.top_k : count;
        // order the first k by (value desc, id asc), stable; rank by counting (k <= 64)
        const float v = l < k ? v_row[l] : 0.f;
        const u32 id = l < k ? (u32)c_row[l] : 0u;
        int rank = 0;
        bool nan_any = false;
        for (int j = 0; j < k; ++j) {
            const float vj = v_row[j];
            const u32 ij = (u32)c_row[j];
            nan_any |= vj != vj;
            if (l < k && row_before(vj, ij, j, v, id, l)) ++rank;
        }
        // try_choose refuses a NaN among the candidates; such a row keeps the first candidate
        if (!nan_any) {
            if (l < k) {
                s_v[w][rank] = v;
                s_i[w][rank] = (u32)l;  // original index
            }
            wave_lds_sync();
            // sorted token ids for the chooser
            if (l < k) s_tid[w][l] = (u32)c_row[s_i[w][l]];
            wave_lds_sync();
            const int b = keyed_choose_wave(s_v[w], s_tid[w], k, p.seed, p.temperature, p.top_p, p.min_p,
                                            p.first_position + (u64)depth);
            pick = (int)s_i[w][b];
        }
    }
    if (l == 0) {
        out_ids[r] = c_row[pick];
        out_vals[r] = v_row[pick];
    }
}

// ------------------------------------------------------------------------------------------------ greedy gather

__global__ void greedy_gather_k(const int* __restrict__ ids, const float* __restrict__ vals, int count, int rows,
                                int* __restrict__ out_ids, float* __restrict__ out_vals) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const size_t base = (size_t)r * count;
    bool nan = false;
    for (int c = 0; c < count; ++c) nan |= vals[base + c] != vals[base + c];
    out_ids[r] = ids[base];
    out_vals[r] = nan ? __uint_as_float(0x7fc00000u) : vals[base];
}

// ------------------------------------------------------------------------------------------------ draft-head argmax picks
// One 1024-thread block per row. The largest value above -inf, lowest id on ties, is the largest order key
// okey << 32 | ~id over those elements (NaN and -inf never count; +-0 compare equal); key 0 means none.

constexpr int PICK_NT = 1024;

__device__ __forceinline__ u64 pick_key(float v, u32 id) { return v > -INFINITY ? make_key(okey_f32(v), id) : 0ull; }

// the block's largest key (every thread gets it)
__device__ __forceinline__ u64 block_max_key(u64 k, u64* s_red) {
    const int w = (int)threadIdx.x / WAVE, l = lane_id();
    k = wave_max_u64(k);
    if (l == 0) s_red[w] = k;
    __syncthreads();
    u64 b = l < PICK_NT / WAVE ? s_red[l] : 0ull;
    b = wave_max_u64(b);
    __syncthreads();
    return b;
}

// f32 [rows, vocab] -> out[r]: the argmax of row r (0 when no element is above -inf)
__global__ void __launch_bounds__(PICK_NT) row_argmax_k(const float* __restrict__ logits, int vocab, bool vec, int* __restrict__ out) {
    __shared__ u64 s_red[PICK_NT / WAVE];
    const int r = blockIdx.x, tid = (int)threadIdx.x;
    const float* row = logits + (size_t)r * vocab;
    u64 best = 0;
    if (vec) {
        const float4* row4 = (const float4*)row;
        for (int i = tid; i < vocab / 4; i += PICK_NT) {
            const float4 v = row4[i];
            const u32 e = (u32)i * 4u;
            const u64 a = max(pick_key(v.x, e), pick_key(v.y, e + 1)), b = max(pick_key(v.z, e + 2), pick_key(v.w, e + 3));
            best = max(best, max(a, b));
        }
    } else {
        for (int i = tid; i < vocab; i += PICK_NT) best = max(best, pick_key(row[i], (u32)i));
    }
    best = block_max_key(best, s_red);
    if (tid == 0) out[r] = best ? (int)key_id(best) : 0;
}

// one bf16 row [n] -> out_id[j]: its argmax (0 when no element is above -inf); out_p[j]: 1 / sum_i exp(x_i - max),
// the softmax probability of the maximum (NaN when the row holds a NaN or no finite maximum)
__global__ void __launch_bounds__(PICK_NT) mtp_pick_k(const u16* __restrict__ logits, int n, bool vec, int* __restrict__ out_id,
                                                      float* __restrict__ out_p, int j) {
    __shared__ u64 s_red[PICK_NT / WAVE];
    __shared__ float s_sum[PICK_NT / WAVE];
    const int tid = (int)threadIdx.x, w = tid / WAVE, l = lane_id();
    auto bf = [](u32 h) { return __uint_as_float(h << 16); };
    u64 best = 0;
    if (vec) {
        const uint4* row8 = (const uint4*)logits;
        for (int i = tid; i < n / 8; i += PICK_NT) {
            const uint4 v = row8[i];
            const u32 e = (u32)i * 8u;
            const u32 wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                best = max(best, max(pick_key(bf(wd[q] & 0xFFFFu), e + 2 * q), pick_key(bf(wd[q] >> 16), e + 2 * q + 1)));
        }
    } else {
        for (int i = tid; i < n; i += PICK_NT) best = max(best, pick_key(bf(logits[i]), (u32)i));
    }
    best = block_max_key(best, s_red);
    const float mx = best ? okey_to_f32(key_ok(best)) : -INFINITY;
    // second read of the row (from L2): the sum of exp(x - max)
    float a = 0.f;
    if (vec) {
        const uint4* row8 = (const uint4*)logits;
        for (int i = tid; i < n / 8; i += PICK_NT) {
            const uint4 v = row8[i];
            const u32 wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) a += __expf(bf(wd[q] & 0xFFFFu) - mx) + __expf(bf(wd[q] >> 16) - mx);
        }
    } else {
        for (int i = tid; i < n; i += PICK_NT) a += __expf(bf(logits[i]) - mx);
    }
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) a += __shfl_xor(a, m, WAVE);
    if (l == 0) s_sum[w] = a;
    __syncthreads();
    if (tid == 0) {
        float t = 0.f;
        for (int o = 0; o < PICK_NT / WAVE; ++o) t += s_sum[o];
        out_id[j] = best ? (int)key_id(best) : 0;
        out_p[j] = 1.f / t;
    }
}

// ------------------------------------------------------------------------------------------------ fused keyed sampler

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// The per-row arrival counters (zero between launches) sit at fixed offsets in the first KEYED_CTL_BYTES, room for
// 65535 rows whatever this launch's row count; the partial lists after them are written before they are read. So a
// workspace cleared once serves launches of any shape.
constexpr size_t KEYED_CTL_BYTES = (size_t)65536 * 4;

int keyed_fast_splits(int rows, int valid);

size_t keyed_ws_bytes(int rows, int valid) {
    if (rows <= 0 || valid <= 0) return 0;
    return KEYED_CTL_BYTES + (size_t)rows * keyed_fast_splits(rows, valid) * WAVE * sizeof(u64);
}

__device__ __forceinline__ bool keyed_params_ok(const KeyedRowDev& p) {
    const bool t_ok = isfinite(p.temperature) && p.temperature >= 0.0;
    const bool p_ok = isfinite(p.top_p) && p.top_p >= 0.0 && p.top_p <= 1.0;
    const bool m_ok = isfinite(p.min_p) && p.min_p >= 0.0 && p.min_p <= 1.0;
    return t_ok && p_ok && m_ok && p.top_k >= 1 && p.top_k <= 56;
}

// ------------------------------------------------------------------------------------------------ fused keyed sampler,
// one block per row
//
// try_choose over each row's exact top-(top_k + 8), on the north-star kernel's streaming design: a block of KNT threads per row (rows
// split over blocks only when there are fewer rows than CUs). Wave-steps of KWSTEP contiguous elements (KGROUPS
// 4-element groups per lane) are handed out through an LDS counter, two in flight per wave; each wave keeps its gated
// top-64 list, the gate raised by the block bound of every wave's best keys. With one block per row the block merges
// its wave lists and draws; otherwise the blocks hand their lists to the row's last block.
#ifndef GBS_KEYED_LATE_B
#define GBS_KEYED_LATE_B 1  // each wave's second wave-step issued once its first has arrived (0: at the start)
#endif
#ifndef GBS_KEYED_NT
#define GBS_KEYED_NT 1024
#endif
#ifndef GBS_KEYED_GROUPS
#define GBS_KEYED_GROUPS 4
#endif
constexpr int KNT = GBS_KEYED_NT;
constexpr int KNW = KNT / WAVE;
constexpr int KGROUPS = GBS_KEYED_GROUPS;
constexpr int KGS = WAVE * 4;           // elements between a lane's groups
constexpr int KWSTEP = KGS * KGROUPS;   // elements of one wave-step
constexpr int KBUF = WAVE * (4 + 1);  // < 64 keys left after a flush + one 4-element group per lane (flushed per group)
#ifndef GBS_KEYED_BLOCKS
#define GBS_KEYED_BLOCKS 256
#endif
constexpr int KF_TARGET_BLOCKS = GBS_KEYED_BLOCKS;
constexpr u32 NEG_INF_OK = 0x007FFFFFu;  // okey_f32(-inf)
constexpr int KF_MIN_CHUNK = 4096;

int keyed_fast_splits(int rows, int valid) {
    int s = (KF_TARGET_BLOCKS + rows - 1) / rows;
    const int by_size = (valid + KF_MIN_CHUNK - 1) / KF_MIN_CHUNK;
    if (s > by_size) s = by_size;
    return s < 1 ? 1 : s;
}

template <int DT>
struct KRaw {
    typename std::conditional<DT == DT_F32, u32x4, u32x2>::type x[KGROUPS];
};

template <int DT>
__device__ __forceinline__ void kraw_keys(const KRaw<DT>& r, int j, u32 (&k)[4]) {
    if constexpr (DT == DT_F32) {
        const u32x4 v = r.x[j];
        k[0] = okey_f32_nanlow(__uint_as_float(v.x)); k[1] = okey_f32_nanlow(__uint_as_float(v.y));
        k[2] = okey_f32_nanlow(__uint_as_float(v.z)); k[3] = okey_f32_nanlow(__uint_as_float(v.w));
    } else {
        const u32x2 v = r.x[j];
        k[0] = okey_16<DT == DT_F16>(v.x); k[1] = okey_16<DT == DT_F16>(v.x >> 16);
        k[2] = okey_16<DT == DT_F16>(v.y); k[3] = okey_16<DT == DT_F16>(v.y >> 16);
    }
}

template <int DT>
__global__ void __launch_bounds__(KNT, 1) keyed_fast_k(const void* logits, long long stride, int valid, int chunk,
                                                       const KeyedRowDev* __restrict__ params, int depth, bool vec, unsigned* counters,
                                                       u64* parts, int* out_ids, float* out_vals, int* out_status) {
    __shared__ u64 s_buf[KNW][KBUF];
    __shared__ u64 s_list[KNW][WAVE];
    __shared__ float s_v[WAVE];
    __shared__ u32 s_id[WAVE];
    __shared__ unsigned s_flag;
    __shared__ u64 s_thr;
    __shared__ u32 s_top[KNW * WaveTop<KBUF>::TOPN];
    __shared__ int s_next;
    const int S = gridDim.x, sp = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x, w = tid / WAVE, l = lane_id();
    const size_t esz = DT == DT_F32 ? 4 : 2;
    const void* row = (const char*)logits + (size_t)r * (size_t)stride * esz;
    const int lo = sp * chunk;
    const int hi = min(valid, lo + chunk);
    // The buffer resource covers this block's chunk, [lo, hi) rounded up to a whole group (inside the row): loads past it
    // return zeros and touch no memory, so a refill is issued whether or not its wave-step exists (a fixed count of loads
    // per refill keeps the compiler's wait counts exact: a buffer waits for its own loads only). The last wave-step's
    // elements at or past `hi` are not offered.
    const u32 nbytes = (u32)max(0, (hi + 3) / 4 * 4 - lo) * (u32)esz;
    const __amdgpu_buffer_rsrc_t R =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>((const char*)row + (size_t)lo * esz), (short)0, (int)nbytes, 0x00020000);
    const int nws = vec ? (hi - lo + KWSTEP - 1) / KWSTEP : 0;
    auto load = [&](int idx, KRaw<DT>& b) {
        const u32 e = (u32)(idx * KWSTEP + l * 4);  // from the chunk's start
#pragma unroll
        for (int j = 0; j < KGROUPS; ++j) {
            if constexpr (DT == DT_F32) b.x[j] = __builtin_amdgcn_raw_buffer_load_b128(R, (e + j * KGS) * 4u, 0, 2);
            else b.x[j] = __builtin_amdgcn_raw_buffer_load_b64(R, (e + j * KGS) * 2u, 0, 2);
        }
    };
    // wave w's first two wave-steps (w and KNW + w) are fixed: the first's loads go out before the block's first barrier
    // and the row's parameters, the second's once the first has arrived (a lighter queue ahead of the seeding barrier);
    // later ones come from an LDS counter
    KRaw<DT> A, B;
    KRaw<DT>& B0 = B;  // the second buffer, under a name the step lambda's parameter does not hide
    if (w < nws) load(w, A);
    if (!GBS_KEYED_LATE_B && KNW + w < nws) load(KNW + w, B);
    if (tid == 0) {
        s_thr = 0;
        s_next = 2 * KNW;
    }
    if (tid < KNW * WaveTop<KBUF>::TOPN) s_top[tid] = 0;
    __syncthreads();
    const KeyedRowDev p = params[r];
    const bool ok = keyed_params_ok(p);
    const int count = ok ? min(p.top_k + 8, valid) : min(WAVE, valid);
    WaveTop<KBUF> wt;
    wt.init(s_buf[w], count, 0ull, &s_thr);
    wt.set_top(s_top, w, KNW);
    int e0 = lo;
    if (vec) {
        auto grab = [&]() {
            int t = 0;
            if (l == 0) t = __hip_atomic_fetch_add(&s_next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            return __builtin_amdgcn_readfirstlane(t);
        };
        // the keys of one loaded wave-step (out of the chunk: key 0, not offered); `first` seeds the gate. The step's
        // words are copied out of the buffer first and the buffer is refilled at once, at one place for every path, so
        // that the compiler's wait counts keep the other buffer's loads in flight.
        auto step = [&](KRaw<DT>& B, int idx, auto first_c, auto&& reload) __attribute__((always_inline)) {
            constexpr bool first = decltype(first_c)::value;
            const int e = lo + idx * KWSTEP + l * 4;
            wt.apply_shared();
            wt.prefetch_shared();
            const KRaw<DT> C = B;
            if (first && GBS_KEYED_LATE_B && KNW + w < nws) load(KNW + w, B0);  // once this wave-step has arrived
            reload();
            // f32 rows whose gate is a float at or above -inf test the gate with one float compare per element (NaN
            // never passes, as its key 0 is below any such gate); the order keys are built for the elements that pass
            if constexpr (DT == DT_F32 && !first) {
                if (wt.gate >= NEG_INF_OK) {
                    float v[KGROUPS * 4];
                    bool in[KGROUPS * 4];
#pragma unroll
                    for (int j = 0; j < KGROUPS; ++j) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            in[j * 4 + q] = e + j * KGS + q < hi;
                            v[j * 4 + q] = __uint_as_float(C.x[j][q]);
                        }
                    }
                    const float gf = okey_to_f32(wt.gate);
                    bool any = false;
#pragma unroll
                    for (int i = 0; i < KGROUPS * 4; ++i) any |= in[i] && v[i] >= gf;
                    if (ballot(any)) {
#pragma unroll
                        for (int j = 0; j < KGROUPS; ++j) {
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const int i = j * 4 + q;
                                const bool pass = in[i] && v[i] >= gf;
                                wt.offer_ok(pass ? okey_f32_nanlow(v[i]) : 0u, (u32)(e + j * KGS + q), pass);
                            }
                            wt.flush(false);
                        }
                    }
                    return;
                }
            }
            u32 k[KGROUPS * 4];
            bool in[KGROUPS * 4];
#pragma unroll
            for (int j = 0; j < KGROUPS; ++j) {
                u32 kj[4];
                kraw_keys<DT>(C, j, kj);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    in[j * 4 + q] = e + j * KGS + q < hi;
                    k[j * 4 + q] = in[j * 4 + q] ? kj[q] : 0u;
                }
            }
            if (first) {
                u32 m = 0;
#pragma unroll
                for (int i = 0; i < KGROUPS * 4; ++i) m = k[i] > m ? k[i] : m;
                wt.seed(m);
                __syncthreads();
                wt.block_bound();
            }
            const u32 g = wt.gate;
            bool any = false;
#pragma unroll
            for (int i = 0; i < KGROUPS * 4; ++i) any |= in[i] && k[i] >= g;
            if (ballot(any)) {
#pragma unroll
                for (int j = 0; j < KGROUPS; ++j) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) wt.offer_ok(k[j * 4 + q], (u32)(e + j * KGS + q), in[j * 4 + q]);
                    wt.flush(false);
                }
            }
        };
        int ia = w;        // loaded at the kernel's start
        int ib = KNW + w;  // likewise
        if (ia >= nws) {
            // no wave-step of its own: take part in the block's seeding barrier
            wt.seed(0u);
            __syncthreads();
            wt.block_bound();
        } else {
            int na = 0, nb = 0;
            auto refill_a = [&]() {
                na = grab();
                load(na, A);  // past the chunk when na >= nws: zeros, no memory read
            };
            auto refill_b = [&]() {
                nb = grab();
                load(nb, B);
            };
            // the first wave-step (it seeds the gate), then the buffers in turn
            step(A, ia, std::true_type{}, refill_a);
            ia = na;
            if (ib < nws) {
                for (;;) {
                    step(B, ib, std::false_type{}, refill_b);
                    ib = nb;
                    if (ia >= nws) break;
                    step(A, ia, std::false_type{}, refill_a);
                    ia = na;
                    if (ib >= nws) break;
                }
            }
        }
        e0 = hi;
    }
    // unaligned rows: one guarded group per lane per round
    const int rounds = (hi - e0 + KNT * 4 - 1) / (KNT * 4);
    for (int rr = 0; rr < rounds; ++rr) {
        const int eg = e0 + rr * KNT * 4 + tid * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) wt.offer_ok(eg + q < hi ? elem_key<DT>(row, eg + q) : 0u, (u32)(eg + q), eg + q < hi);
        wt.flush(false);
    }
    wt.prefetch_shared();
    wt.apply_shared();
    wt.flush(true);
    u64 list = block_tree_merge<KNW>(wt.list, s_list);
    if (S > 1) {
        if (tid < WAVE) st_agent(&parts[((size_t)r * S + sp) * WAVE + tid], list);
        if (!arrive_last(&counters[r], (unsigned)S, &s_flag)) return;
        list = block_merge_lists<KNW>(parts + (size_t)r * S * WAVE, S, s_list);
    }
    if (tid >= WAVE) return;
    int status = ok ? GBS_ROW_OK : GBS_ROW_INVALID_PARAMS;
    const u32 id = key_id(list);
    float v = 0.f;
    if (l < count && list != 0ull) {  // the first `count` keys are elements of the row (every valid element is offered)
        if (DT == DT_F32) v = ((const float*)row)[id];
        else v = okey16_to_f32<DT == DT_F16>(key_ok(list));
    }
    if (status == GBS_ROW_OK && ballot(l < count && v != v)) status = GBS_ROW_NAN_LOGIT;
    int pick = 0;
    if (status == GBS_ROW_OK && p.temperature > 0.0) {
        s_v[l] = v;
        s_id[l] = id;
        wave_lds_sync();
        const int k = min(p.top_k, count);
        pick = keyed_choose_wave(s_v, s_id, k, p.seed, p.temperature, p.top_p, p.min_p, p.first_position + (u64)depth);
    }
    const u32 pid = readlane32(id, pick);
    const float pv = __uint_as_float(readlane32(__float_as_uint(v), pick));
    if (l == 0) {
        out_ids[r] = status == GBS_ROW_OK ? (int)pid : -1;
        if (out_vals) out_vals[r] = status == GBS_ROW_OK ? pv : __uint_as_float(0x7fc00000u);
        if (out_status) out_status[r] = status;
    }
}

// ------------------------------------------------------------------------------------------------ selector walk
// The draft head's selector chain walk (crates/cuda/csrc/dflash2.cu:436-519 kernel, 595-660 entry points): per
// sequence, each draft row's k <= 64 candidates are scored as unary[c] + <pred[prev] * gate[row], succ[c]>, and the
// row's pick becomes the next row's predecessor.
//
// Layout: one block of WALK_NW waves per sequence, one candidate per lane. The score's float value is fixed by the
// reference: the dot product is 32 partial sums, partial j a chain of fused multiply-adds over r = j, j + 32, ...
// (ascending), combined by an xor butterfly over offsets 16, 8, 4, 2, 1. Here wave w computes partials
// 8w .. 8w + 7 of every candidate (lane c reads 8 consecutive f16 of succ[c] per 32-element slice: one 16-byte load),
// the partials meet in LDS, and wave 0 replays the butterfly inside each lane: at offset o, s[j] += s[j + o] for j < o
// (IEEE addition commutes, so this is the value every lane of the butterfly ends with).
//
// The pick, on wave 0:
//  - unkeyed: the first maximum in candidate order (strict >; a NaN first score stays the pick), with the gap to the
//    runner-up capped at 30;
//  - keyed (crates/cuda/csrc/keyed.cuh:50-112 semantics): each lane's place in the order (score desc, id asc, NaN
//    last, ties in candidate order) is counted against the other lanes' (score, id) pairs, the candidates are placed
//    in that order in LDS, then keyed_choose_wave runs try_choose over all k. Temperature 0 takes the first in order,
//    with the raw score gap to the second as its margin.

struct WalkSamplingDev {
    u64 seed, first_position;
    double temperature, top_p, min_p;
    int keyed, pad;
};
static_assert(sizeof(WalkSamplingDev) == 48, "WalkSampling is 48 bytes");

constexpr int WALK_NW = 4;                 // waves per sequence
constexpr int WALK_NT = WALK_NW * WAVE;    // threads per sequence
constexpr int WALK_PW = 32 / WALK_NW;      // partial sums per wave
constexpr int WALK_MAX_RANK = 8192;
static_assert(WALK_PW == 8, "one 16-byte f16 load feeds a wave's partials of one 32-element slice");

__device__ __forceinline__ float walk_gate(const void* gate, bool gate_f32, size_t at) {
    return gate_f32 ? ((const float*)gate)[at] : __uint_as_float((u32)((const u16*)gate)[at] << 16);
}

// true when candidate (vb, ib, pb) comes before (va, ia, pa): score desc, id asc, NaN after every number, otherwise
// candidate order
__device__ __forceinline__ bool walk_before(float vb, int ib, int pb, float va, int ia, int pa) {
    const bool nb = vb != vb, na = va != va;
    if (nb || na) return na && !nb ? true : (nb && na ? pb < pa : false);
    if (vb != va) return vb > va;
    if (ib != ia) return ib < ia;
    return pb < pa;
}

__global__ void __launch_bounds__(WALK_NT) walk_k(const int* __restrict__ anchor, const int* __restrict__ cand_ids,
                                                  const float* __restrict__ unary, const void* __restrict__ gate, int gate_f32,
                                                  const __half* __restrict__ pred_cb, const __half* __restrict__ succ_cb,
                                                  int* __restrict__ out, float* __restrict__ conf, int rows, int k, int rank,
                                                  const WalkSamplingDev* __restrict__ samp, const int* __restrict__ row_off,
                                                  float* __restrict__ margin) {
    extern __shared__ float s_ag[];                // [rank]: pred[prev] * gate[row]
    __shared__ float s_part[32][WAVE];             // partial sums, [partial][candidate]
    __shared__ float s_sorted_v[WAVE];
    __shared__ u32 s_sorted_id[WAVE];
    __shared__ int s_sorted_c[WAVE];
    __shared__ int s_prev;
    const int seq = blockIdx.x, w = threadIdx.x / WAVE, c = lane_id();
    const int first = row_off ? row_off[seq] : seq * rows;
    const int n_rows = row_off ? row_off[seq + 1] - first : rows;
    const bool keyed = samp != nullptr && samp[seq].keyed != 0;
    // 16-byte loads of 8 f16 need 16-byte aligned codebook rows
    const bool vec = (rank % 8) == 0 && aligned(succ_cb, 16);
    if (threadIdx.x == 0) s_prev = anchor[seq];
    __syncthreads();
    for (int i = 0; i < n_rows; ++i) {
        const size_t row = (size_t)(first + i);
        const __half* prow = pred_cb + (size_t)s_prev * rank;
        for (int r = threadIdx.x; r < rank; r += WALK_NT) s_ag[r] = __half2float(prow[r]) * walk_gate(gate, gate_f32 != 0, row * rank + r);
        __syncthreads();
        // partials 8w .. 8w + 7 of candidate c
        float p[WALK_PW];
#pragma unroll
        for (int j = 0; j < WALK_PW; ++j) p[j] = 0.f;
        if (c < k) {
            const __half* srow = succ_cb + (size_t)cand_ids[row * k + c] * rank;
            const int j0 = w * WALK_PW;
            if (vec) {
                const uint4* s16 = reinterpret_cast<const uint4*>(srow + j0);
                const int slices = rank / 32;
                int m = 0;
                for (; m + 4 <= slices; m += 4) {
                    uint4 q[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) q[u] = s16[(size_t)(m + u) * 4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const __half* h = reinterpret_cast<const __half*>(&q[u]);
                        const float* a = s_ag + (m + u) * 32 + j0;
#pragma unroll
                        for (int j = 0; j < WALK_PW; ++j) p[j] = fmaf(a[j], __half2float(h[j]), p[j]);
                    }
                }
                for (; m < slices; ++m) {
                    const uint4 q = s16[(size_t)m * 4];
                    const __half* h = reinterpret_cast<const __half*>(&q);
                    const float* a = s_ag + m * 32 + j0;
#pragma unroll
                    for (int j = 0; j < WALK_PW; ++j) p[j] = fmaf(a[j], __half2float(h[j]), p[j]);
                }
                // rank % 8 == 0: the last partial slice has whole groups of 8, each owned by one wave
                const int r0 = slices * 32 + j0;
                if (r0 < rank) {
                    const uint4 q = *reinterpret_cast<const uint4*>(srow + r0);
                    const __half* h = reinterpret_cast<const __half*>(&q);
#pragma unroll
                    for (int j = 0; j < WALK_PW; ++j) p[j] = fmaf(s_ag[r0 + j], __half2float(h[j]), p[j]);
                }
            } else {
                for (int base = j0; base < rank; base += 32) {
#pragma unroll
                    for (int j = 0; j < WALK_PW; ++j)
                        if (base + j < rank) p[j] = fmaf(s_ag[base + j], __half2float(srow[base + j]), p[j]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < WALK_PW; ++j) s_part[w * WALK_PW + j][c] = p[j];
        __syncthreads();
        if (w == 0) {
            // the butterfly, in lane
            float s[32];
#pragma unroll
            for (int j = 0; j < 32; ++j) s[j] = s_part[j][c];
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) {
#pragma unroll
                for (int j = 0; j < o; ++j) s[j] = s[j] + s[j + o];
            }
            const int cid = c < k ? cand_ids[row * k + c] : 0x7fffffff;
            const float score = c < k ? unary[row * k + c] + s[0] : -INFINITY;
            int pick;       // candidate index
            float mg;
            if (!keyed) {
                const float s0 = __shfl(score, 0);
                if (s0 != s0) {
                    pick = 0;
                } else {
                    float mx = (c < k && score == score) ? score : -INFINITY;
#pragma unroll
                    for (int m = 1; m < WAVE; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
                    pick = (int)__builtin_ctzll(ballot(c < k && score == mx));
                }
                float second = (c < k && c != pick && score == score) ? score : -INFINITY;
#pragma unroll
                for (int m = 1; m < WAVE; m <<= 1) second = fmaxf(second, __shfl_xor(second, m));
                const float best = __shfl(score, pick);
                mg = k > 1 ? fminf(best - second, 30.f) : 30.f;
            } else {
                // place in the order: the lanes before this one, counted over (score, id) broadcasts
                int place = 0;
                for (int o = 0; o < k; ++o) {
                    const float vo = __shfl(score, o);
                    const int io = __shfl(cid, o);
                    place += (o != c && walk_before(vo, io, o, score, cid, c)) ? 1 : 0;
                }
                if (c < k) {
                    s_sorted_v[place] = score;
                    s_sorted_id[place] = (u32)cid;
                    s_sorted_c[place] = c;
                }
                wave_lds_sync();
                const WalkSamplingDev sp = samp[seq];
                if (sp.temperature == 0.0) {
                    pick = s_sorted_c[0];
                    mg = k > 1 ? s_sorted_v[0] - s_sorted_v[1] : 30.f;
                } else {
                    float m_out = 30.f;
                    const int at = keyed_choose_wave(s_sorted_v, s_sorted_id, k, sp.seed, sp.temperature, sp.top_p, sp.min_p,
                                                     sp.first_position + (u64)i, &m_out);
                    pick = s_sorted_c[at];
                    mg = m_out;
                }
            }
            if (c == pick) {
                s_prev = cid;
                out[row] = cid;
                if (conf) conf[row] = score;
                if (margin) margin[row] = mg;
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------ accept steps

__global__ void accept_k(const int* __restrict__ drafts, const int* __restrict__ samples, int n_seq, int width, int* accepted) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n_seq) return;
    const int* d = drafts + (size_t)s * width;
    const int* x = samples + (size_t)s * (width + 1);
    int a = 0;
    while (a < width && d[a] == x[a]) ++a;
    accepted[s] = a;
}

__global__ void accept_tree_k(const int* __restrict__ tokens, const int* __restrict__ parents, const int* __restrict__ samples,
                              int n_tree, int nodes, int* path, int* path_len) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_tree) return;
    const int* tok = tokens + (size_t)t * nodes;
    const int* par = parents + (size_t)t * nodes;
    const int* smp = samples + (size_t)t * nodes;
    int* out = path + (size_t)t * nodes;
    int len = 0, cur = 0;
    out[len++] = 0;
    for (;;) {
        const int s = smp[cur];
        int next = -1;
        for (int r = cur + 1; r < nodes; ++r)
            if (par[r] == cur && tok[r] == s) {
                next = r;
                break;
            }
        if (next < 0) break;
        out[len++] = next;
        cur = next;
    }
    for (int i = len; i < nodes; ++i) out[i] = -1;
    path_len[t] = len;
}

// accept_tree_k over trees whose rows were sampled on the device: a tree with a failed row (status != 0) gets that
// status (its first failed row's), path_len 0 and an all -1 path, as the engine fails a sequence when any of its rows'
// try_choose fails (crates/engine/src/lib.rs:2376-2404).
__global__ void tree_commit_k(const int* __restrict__ tokens, const int* __restrict__ parents, const int* __restrict__ samples,
                              const int* __restrict__ row_status, int n_tree, int nodes, int* path, int* path_len, int* status) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_tree) return;
    int st = GBS_ROW_OK;
    for (int r = 0; r < nodes && st == GBS_ROW_OK; ++r) st = row_status[(size_t)t * nodes + r];
    if (status) status[t] = st;
    if (st == GBS_ROW_OK) return;  // accept_tree_k, launched after this kernel, leaves the path of an OK tree
    int* out = path + (size_t)t * nodes;
    for (int i = 0; i < nodes; ++i) out[i] = -1;
    path_len[t] = 0;
}

__global__ void accept_tree_ok_k(const int* __restrict__ tokens, const int* __restrict__ parents, const int* __restrict__ samples,
                                 const int* __restrict__ status, int n_tree, int nodes, int* path, int* path_len) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_tree || status[t] != GBS_ROW_OK) return;
    const int* tok = tokens + (size_t)t * nodes;
    const int* par = parents + (size_t)t * nodes;
    const int* smp = samples + (size_t)t * nodes;
    int* out = path + (size_t)t * nodes;
    int len = 0, cur = 0;
    out[len++] = 0;
    for (;;) {
        const int sv = smp[cur];
        int next = -1;
        for (int r = cur + 1; r < nodes; ++r)
            if (par[r] == cur && tok[r] == sv) {
                next = r;
                break;
            }
        if (next < 0) break;
        out[len++] = next;
        cur = next;
    }
    for (int i = len; i < nodes; ++i) out[i] = -1;
    path_len[t] = len;
}

__global__ void clear_k(uint4* p, size_t n16, unsigned char* tail, size_t ntail) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n16; j += stride) p[j] = make_uint4(0, 0, 0, 0);
    if (i < ntail) tail[i] = 0;
}

// ------------------------------------------------------------------------------------------------ DSV4 Markov walk
// The DSV4 draft head's keyed Markov walk (crates/cuda/csrc/dsv4_mtp_gpu.cu:1233-1480 kernels, 1662-1718 entry
// points). Per walk row k, 1024 candidates: thread t of 256 keeps the 4 largest logits of v = t, t + 256, ... Then,
// from the previous token p = ids[k], each candidate's logit gains <embed[p], head[v]> (bf16 tables [vocab, 256]) and the
// logits row keeps the sum. The next token is the argmax of the candidates, or the keyed choose (the device
// try_choose with its margin) over their top cand_k. Row k + 1's bias needs token k + 1, so each row is a launch of
// the bias kernel and a launch of the pick (the caller's workspace leaves no room for a hand-off counter).

constexpr int MW_CAND = 1024;
constexpr int MW_RANK = 256;
constexpr int MW_NT = 256;
constexpr u32 MW_NONE = 0x7fffffffu;

// The 72-byte Dsv4MtpRoundParams record (crates/cuda/src/dsv4_mtp_gpu.rs:2683-2701); the walk reads cand_k and the
// sampling fields on the device, so a captured graph replays with new values.
struct Dsv4RoundDev {
    int anchor, start_pos, reach, n_kv, window, block_size, cand_k, pad;
    u64 seed, base_pos;
    double temperature, top_p, min_p;
};
static_assert(sizeof(Dsv4RoundDev) == 72, "Dsv4MtpRoundParams is 72 bytes");

// Thread t's 4 largest of logits[v], v = t + 256 i, in descending order. The reference inserts with a strict > in
// increasing v, which is the order (value desc, v asc); a NaN or -inf never enters and an unfilled slot keeps
// (-inf, id 0) (reference :1233-1262). Here 512 threads per row: thread (g, j) of 8 x 64 loads the 4 values
// v = 256 i + 4j .. + 3 (slices t = 4j .. 4j + 3) for i = g, g + 8, ..., keeping a top-4 per slice; the 8 groups'
// lists of each slice are then merged in LDS.
constexpr int MW_CT = 512;
constexpr int MW_CG = MW_CT / 64;

struct Top4 {
    float v[4];
    int id[4];
    __device__ __forceinline__ void init() {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[q] = -INFINITY;
            id[q] = 0;
        }
    }
    // (x, i) after every entry that ranks before it (a larger value, or an equal one with a smaller id), by a
    // compare-and-select network: no run-time index, so the lists stay in registers
    __device__ __forceinline__ void insert(float x, int i) {
        bool b[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) b[q] = x > v[q] || (x == v[q] && i < id[q]);
#pragma unroll
        for (int q = 3; q >= 1; --q) {
            v[q] = b[q - 1] ? v[q - 1] : (b[q] ? x : v[q]);
            id[q] = b[q - 1] ? id[q - 1] : (b[q] ? i : id[q]);
        }
        v[0] = b[0] ? x : v[0];
        id[0] = b[0] ? i : id[0];
    }
};

__global__ void __launch_bounds__(MW_CT) mw_cands_k(const float* __restrict__ logits, int* __restrict__ cand_ids, int vocab) {
    __shared__ float s_v[MW_CG][256][4];
    __shared__ int s_i[MW_CG][256][4];
    const int row = blockIdx.x, g = threadIdx.x / 64, j = threadIdx.x % 64;
    const float* lr = logits + (size_t)row * vocab;
    Top4 t4[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) t4[q].init();
    const bool vec = (vocab & 3) == 0 && (((uintptr_t)lr) & 15) == 0;
    // MW_CU strides' loads in flight before any is ranked (the insert order does not matter: ties rank by id)
    constexpr int MW_CU = 8;
    for (int i0 = g; 256 * i0 < vocab; i0 += MW_CG * MW_CU) {
        float x[MW_CU][4];
#pragma unroll
        for (int u = 0; u < MW_CU; ++u) {
            const int v0 = 256 * (i0 + u * MW_CG) + 4 * j;
            if (vec && v0 + 4 <= vocab) {
                const float4 f = *reinterpret_cast<const float4*>(lr + v0);
                x[u][0] = f.x; x[u][1] = f.y; x[u][2] = f.z; x[u][3] = f.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) x[u][q] = v0 + q < vocab ? lr[v0 + q] : -INFINITY;
            }
        }
#pragma unroll
        for (int u = 0; u < MW_CU; ++u) {
            const int v0 = 256 * (i0 + u * MW_CG) + 4 * j;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (x[u][q] > -INFINITY) t4[q].insert(x[u][q], v0 + q);  // false for NaN and -inf, as the reference's x > -inf
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s_v[g][4 * j + q][r] = t4[q].v[r];
            s_i[g][4 * j + q][r] = t4[q].id[r];
        }
    __syncthreads();
    if (threadIdx.x >= 256) return;
    const int t = threadIdx.x;
    Top4 m;
    m.init();
    for (int gg = 0; gg < MW_CG; ++gg)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (s_v[gg][t][r] > -INFINITY) m.insert(s_v[gg][t][r], s_i[gg][t][r]);
    int4* o = reinterpret_cast<int4*>(cand_ids + (size_t)row * MW_CAND + t * 4);
    *o = make_int4(m.id[0], m.id[1], m.id[2], m.id[3]);
}

// One walk row's bias: 32 blocks of 256 threads; each half-wave (32 lanes, lane j owning dimensions 8j .. 8j + 7)
// scores 4 candidates: 8 fused multiply-adds in order, then a butterfly over the 32 lanes (xor 16, 8, 4, 2, 1) whose
// lane-0 total is added to the logit (reference :1264-1311).
__global__ void __launch_bounds__(MW_NT) mw_bias_k(float* __restrict__ logits, const int* __restrict__ token,
                                                   const u16* __restrict__ embed, const u16* __restrict__ head,
                                                   const int* __restrict__ cand_ids, float* __restrict__ cand_scores, int vocab) {
    const int t = *token;
    const bool ok = (unsigned)t < (unsigned)vocab;
    const int hw = threadIdx.x >> 5, j = threadIdx.x & 31;
    const int c_base = ((int)blockIdx.x * (MW_NT / 32) + hw) * 4;
    float e[8];
    if (ok) {
        const uint4 eu = *reinterpret_cast<const uint4*>(embed + (size_t)t * MW_RANK + j * 8);
        const u32 w[4] = {eu.x, eu.y, eu.z, eu.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            e[2 * q] = __uint_as_float(w[q] << 16);
            e[2 * q + 1] = __uint_as_float(w[q] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) e[q] = 0.0f;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int idx = c_base + c;
        const int v = cand_ids[idx];
        if ((unsigned)v < (unsigned)vocab) {  // uniform over the half-wave
            const uint4 hu = *reinterpret_cast<const uint4*>(head + (size_t)v * MW_RANK + j * 8);
            const u32 w[4] = {hu.x, hu.y, hu.z, hu.w};
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc = __builtin_fmaf(e[2 * q], __uint_as_float(w[q] << 16), acc);
                acc = __builtin_fmaf(e[2 * q + 1], __uint_as_float(w[q] & 0xFFFF0000u), acc);
            }
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 32);
            if (j == 0) {
                const float sc = logits[v] + acc;
                logits[v] = sc;
                cand_scores[idx] = sc;
            }
        } else if (j == 0) {
            cand_scores[idx] = -INFINITY;
        }
    }
}

// One walk row's pick over the 1024 candidate scores (a non-finite score counts as -inf with id 0x7fffffff). Keys
// order (value desc, id asc), -0 tying +0 as the reference's float compares do. KEYED: the exact top min(cand_k, 64)
// by a register sort and merge of the 1024 keys, then the keyed choose over the leading finite ones (reference
// :1363-1462); otherwise their maximum (:1313-1361).
template <bool KEYED>
__global__ void __launch_bounds__(MW_NT) mw_pick_k(const float* __restrict__ cand_scores, const int* __restrict__ cand_ids,
                                                   int* __restrict__ out_id, float* __restrict__ out_conf, int cand_k, u64 seed,
                                                   double temperature, double top_p, double min_p, u64 position,
                                                   const Dsv4RoundDev* __restrict__ rp) {
    __shared__ u64 s_list[MW_NT / WAVE][WAVE];
    if (KEYED && rp) {  // the device-params form: position = base_pos + step, the step passed in `position`
        cand_k = rp->cand_k;
        seed = rp->seed;
        temperature = rp->temperature;
        top_p = rp->top_p;
        min_p = rp->min_p;
        position += rp->base_pos;
    }
    __shared__ float s_sc[64];
    __shared__ int s_id[64];
    const int tid = threadIdx.x, l = lane_id();
    auto key_of = [&](float v, int id) -> u64 {
        const bool fin = __builtin_isfinite(v);
        const u32 ok = okey_f32(fin ? v : -INFINITY);
        const u32 i = fin ? (u32)id : MW_NONE;
        return ((u64)ok << 32) | (u64)(0xFFFFFFFFu - i);
    };
    // this wave's best 64 of its 256 keys: four lanes-wide lists sorted and merged
    u64 acc = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int c = tid * 4 + q;
        const u64 k = wave_sort_desc(key_of(cand_scores[c], cand_ids[c]));
        acc = q == 0 ? k : wave_merge_desc(acc, k);
    }
    const u64 top = block_tree_merge<MW_NT / WAVE>(acc, s_list);  // wave 0: the block's best 64, descending
    if (tid >= WAVE) return;
    const float v = okey_to_f32((u32)(top >> 32));
    const u32 id = 0xFFFFFFFFu - (u32)top;
    if (!KEYED) {
        if (l == 0) out_id[0] = id != MW_NONE ? (int)id : 0;
        return;
    }
    const int k = cand_k < 1 ? 1 : (cand_k > 64 ? 64 : cand_k);
    // the leading candidates with a finite score and a real id
    const u64 bad = ballot(l < k && (!__builtin_isfinite(v) || id == MW_NONE)) | (k < 64 ? ~0ull << k : 0ull);
    const int valid_k = bad ? (int)__builtin_ctzll(bad) : 64;
    if (l < k) {
        s_sc[l] = v;
        s_id[l] = (int)id;
    }
    wave_lds_sync();
    if (valid_k == 0) {
        if (l == 0) {
            out_id[0] = 0;
            if (out_conf) out_conf[0] = 0.0f;
        }
        return;
    }
    // the device keyed choose over the sorted candidates (keyed.cuh:50-112): greedy with the first two's gap at T = 0,
    // otherwise try_choose on the wave with the margin of the chosen Gumbel score
    float margin = 30.0f;
    int chosen = 0;
    if (temperature == 0.0) margin = valid_k > 1 ? s_sc[0] - s_sc[1] : 30.f;
    else chosen = keyed_choose_wave(s_sc, (const u32*)s_id, valid_k, seed, temperature, top_p, min_p, position, &margin);
    if (!__builtin_isfinite(margin)) margin = -30.0f;
    if (l == 0) {
        out_id[0] = (u32)s_id[chosen] != MW_NONE ? s_id[chosen] : 0;
        if (out_conf) out_conf[0] = 1.0f / (1.0f + expf(-margin));
    }
}

int launch_markov_walk(void* logits, int* ids, float* conf, const void* embed, const void* head, void* cand_ids_ws,
                       void* cand_scores_ws, int walk_rows, int vocab, int rank, bool keyed, int cand_k, u64 seed, double temperature,
                       double top_p, double min_p, u64 base_pos, const void* params, void* stream) {
    if (!logits || !ids || !embed || !head || !cand_ids_ws || !cand_scores_ws) return GBS_ERR_INVALID;
    if (walk_rows <= 0 || vocab < MW_CAND || rank != MW_RANK || (keyed && !params && cand_k < 1)) return GBS_ERR_INVALID;
    if (params && !aligned(params, 8)) return GBS_ERR_INVALID;
    const Dsv4RoundDev* rp = (const Dsv4RoundDev*)params;  // a device pointer: read only by the kernels
    if (!aligned(embed, 16) || !aligned(head, 16) || !aligned(cand_ids_ws, 16) || !aligned(cand_scores_ws, 16)) return GBS_ERR_INVALID;
    const hipStream_t st = to_stream(stream);
    float* lg = (float*)logits;
    int* cids = (int*)cand_ids_ws;
    float* cs = (float*)cand_scores_ws;
    hipLaunchKernelGGL(mw_cands_k, dim3(walk_rows), dim3(MW_CT), 0, st, (const float*)lg, cids, vocab);
    for (int k = 0; k < walk_rows; ++k) {
        hipLaunchKernelGGL(mw_bias_k, dim3(MW_CAND / ((MW_NT / 32) * 4)), dim3(MW_NT), 0, st, lg + (size_t)k * vocab, (const int*)(ids + k),
                           (const u16*)embed, (const u16*)head, (const int*)(cids + (size_t)k * MW_CAND), cs, vocab);
        if (keyed)
            hipLaunchKernelGGL(mw_pick_k<true>, dim3(1), dim3(MW_NT), 0, st, (const float*)cs, (const int*)(cids + (size_t)k * MW_CAND),
                               ids + k + 1, conf ? conf + k : nullptr, cand_k, seed, temperature, top_p, min_p,
                               (rp ? 0ull : base_pos) + (u64)k, rp);
        else
            hipLaunchKernelGGL(mw_pick_k<false>, dim3(1), dim3(MW_NT), 0, st, (const float*)cs, (const int*)(cids + (size_t)k * MW_CAND),
                               ids + k + 1, (float*)nullptr, 1, (u64)0, 0.0, 0.0, 0.0, (u64)0, (const Dsv4RoundDev*)nullptr);
    }
    return launch_status();
}

}  // namespace

GBS_EXPORT int gb_glm_keyed_pick(const int* ids, const float* vals, int count, int rows, const void* params, int depth, int* out_ids,
                                 float* out_vals, void* stream) {
    if (rows < 0 || count < 1 || count > GBS_MAX_COUNT || depth < 0) return GBS_ERR_INVALID;
    if (rows == 0) return 0;
    if (!ids || !vals || !params || !out_ids || !out_vals) return GBS_ERR_INVALID;
    hipLaunchKernelGGL(keyed_pick_k, dim3((rows + 3) / 4), dim3(256), 0, to_stream(stream), ids, vals, count, rows,
                       (const KeyedRowDev*)params, depth, out_ids, out_vals);
    return launch_status();
}

GBS_EXPORT int gb_qfn_greedy_gather(const void* ids, const void* vals, int count, int rows, void* out_ids, void* out_vals, void* stream) {
    if (!ids || !vals || !out_ids || !out_vals || rows < 0 || count <= 0 || count > GBS_MAX_COUNT) return GBS_ERR_INVALID;
    if (rows == 0) return 0;
    hipLaunchKernelGGL(greedy_gather_k, dim3((rows + 127) / 128), dim3(128), 0, to_stream(stream), (const int*)ids, (const float*)vals,
                       count, rows, (int*)out_ids, (float*)out_vals);
    return launch_status();
}

GBS_EXPORT int gb_dsv4_mtp_argmax(const float* logits, int* out, int rows, int vocab, void* stream) {
    if (!logits || !out || rows <= 0 || vocab <= 0) return GBS_ERR_INVALID;
    const bool vec = vocab % 4 == 0 && aligned(logits, 16);
    hipLaunchKernelGGL(row_argmax_k, dim3(rows), dim3(PICK_NT), 0, to_stream(stream), logits, vocab, vec, out);
    return launch_status();
}

GBS_EXPORT int gb_mtp_pick(const void* logits, int n, void* out_id, void* out_p, int j, void* stream) {
    if (n < 1 || j < 0 || !logits || !out_id || !out_p) return GBS_ERR_INVALID;
    const bool vec = n % 8 == 0 && aligned(logits, 16);
    hipLaunchKernelGGL(mtp_pick_k, dim3(1), dim3(PICK_NT), 0, to_stream(stream), (const u16*)logits, n, vec, (int*)out_id, (float*)out_p, j);
    return launch_status();
}

GBS_EXPORT int gbs_workspace_clear(void* ws, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    if (!ws || !aligned(ws, 16)) return GBS_ERR_INVALID;
    const size_t n16 = bytes / 16, ntail = bytes % 16;
    size_t blocks = (n16 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(clear_k, dim3((unsigned)blocks), dim3(256), 0, to_stream(stream), (uint4*)ws, n16,
                       (unsigned char*)ws + n16 * 16, ntail);
    return launch_status();
}

GBS_EXPORT size_t gbs_keyed_sample_workspace_bytes(int rows, int valid) { return keyed_ws_bytes(rows, valid); }

GBS_EXPORT int gbs_keyed_sample_rows(const void* logits, int dtype, int rows, int stride, int valid, const GbsKeyedRow* params, int depth,
                                     int* out_ids, float* out_vals, int* out_status, void* ws, size_t ws_bytes, void* stream) {
    if (rows < 0 || stride <= 0 || valid <= 0 || valid > stride || depth < 0) return GBS_ERR_INVALID;
    if (dtype != GBS_DTYPE_F32 && dtype != GBS_DTYPE_BF16 && dtype != GBS_DTYPE_F16) return GBS_ERR_INVALID;
    if (rows == 0) return 0;
    if (rows > 65535 || !logits || !params || !out_ids || !ws || !aligned(ws, 256)) return GBS_ERR_INVALID;
    if (ws_bytes < keyed_ws_bytes(rows, valid)) return GBS_ERR_INVALID;
    unsigned* counters = (unsigned*)ws;
    u64* parts = (u64*)((char*)ws + KEYED_CTL_BYTES);
    const KeyedRowDev* p = (const KeyedRowDev*)params;
    const int S = keyed_fast_splits(rows, valid);
    int chunk = (valid + S - 1) / S;
    chunk = (chunk + 3) / 4 * 4;
    const size_t esz = dtype == GBS_DTYPE_F32 ? 4 : 2;
    const bool vec = stride % 4 == 0 && aligned(logits, 4 * esz);
    const dim3 grid(S, rows);
    if (dtype == GBS_DTYPE_F32)
        hipLaunchKernelGGL(keyed_fast_k<DT_F32>, grid, dim3(KNT), 0, to_stream(stream), logits, (long long)stride, valid, chunk, p,
                           depth, vec, counters, parts, out_ids, out_vals, out_status);
    else if (dtype == GBS_DTYPE_BF16)
        hipLaunchKernelGGL(keyed_fast_k<DT_BF16>, grid, dim3(KNT), 0, to_stream(stream), logits, (long long)stride, valid, chunk, p,
                           depth, vec, counters, parts, out_ids, out_vals, out_status);
    else
        hipLaunchKernelGGL(keyed_fast_k<DT_F16>, grid, dim3(KNT), 0, to_stream(stream), logits, (long long)stride, valid, chunk, p,
                           depth, vec, counters, parts, out_ids, out_vals, out_status);
    return launch_status();
}

GBS_EXPORT int gbs_accept(const int* drafts, const int* samples, int n_seq, int width, int* accepted, void* stream) {
    if (n_seq < 0 || width < 0) return GBS_ERR_INVALID;
    if (n_seq == 0) return 0;
    if (!samples || !accepted || (width > 0 && !drafts)) return GBS_ERR_INVALID;
    hipLaunchKernelGGL(accept_k, dim3((n_seq + 127) / 128), dim3(128), 0, to_stream(stream), drafts, samples, n_seq, width, accepted);
    return launch_status();
}

GBS_EXPORT int gbs_accept_tree(const int* tokens, const int* parents, const int* samples, int n_tree, int nodes, int* path, int* path_len,
                               void* stream) {
    if (n_tree < 0 || nodes < 1) return GBS_ERR_INVALID;
    if (n_tree == 0) return 0;
    if (!tokens || !parents || !samples || !path || !path_len) return GBS_ERR_INVALID;
    hipLaunchKernelGGL(accept_tree_k, dim3((n_tree + 63) / 64), dim3(64), 0, to_stream(stream), tokens, parents, samples, n_tree, nodes,
                       path, path_len);
    return launch_status();
}

GBS_EXPORT size_t gbs_tree_verify_workspace_bytes(int n_tree, int nodes, int valid) {
    if (n_tree <= 0 || nodes <= 0 || valid <= 0 || (long long)n_tree * nodes > 65535) return 0;
    const int rows = n_tree * nodes;
    return align256(keyed_ws_bytes(rows, valid)) + align256((size_t)rows * 4);
}

GBS_EXPORT int gbs_tree_verify(const void* logits, int dtype, int n_tree, int nodes, int stride, int valid, const GbsKeyedRow* params,
                               const int* tokens, const int* parents, int* out_samples, int* out_path, int* out_path_len,
                               int* out_status, void* ws, size_t ws_bytes, void* stream) {
    if (n_tree < 0 || nodes < 1 || stride <= 0 || valid <= 0 || valid > stride) return GBS_ERR_INVALID;
    if (n_tree == 0) return 0;
    if ((long long)n_tree * nodes > 65535 || !tokens || !parents || !out_samples || !out_path || !out_path_len || !out_status ||
        !ws || !aligned(ws, 256))
        return GBS_ERR_INVALID;
    const int rows = n_tree * nodes;
    if (ws_bytes < gbs_tree_verify_workspace_bytes(n_tree, nodes, valid)) return GBS_ERR_INVALID;
    const size_t kb = align256(keyed_ws_bytes(rows, valid));
    int* row_status = (int*)((char*)ws + kb);
    int rc = gbs_keyed_sample_rows(logits, dtype, rows, stride, valid, params, 0, out_samples, nullptr, row_status, ws, kb, stream);
    if (rc) return rc;
    // the trees' statuses (a tree is OK when all its rows are), then the accept walk of the OK trees
    int* tst = out_status;
    hipLaunchKernelGGL(tree_commit_k, dim3((n_tree + 63) / 64), dim3(64), 0, to_stream(stream), tokens, parents, out_samples, row_status,
                       n_tree, nodes, out_path, out_path_len, tst);
    rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(accept_tree_ok_k, dim3((n_tree + 63) / 64), dim3(64), 0, to_stream(stream), tokens, parents, out_samples, tst,
                       n_tree, nodes, out_path, out_path_len);
    return launch_status();
}

namespace {
int launch_walk(const void* anchor, const void* topk_ids, const void* topk_vals, const void* gate, int gate_is_f32,
                const void* pred_codebook, const void* succ_codebook, int n_seq, int rows, int k, int rank, const void* sampling,
                const void* row_off, void* out_tokens, void* conf, void* margin, void* stream) {
    const size_t smem = (size_t)rank * sizeof(float);
    hipLaunchKernelGGL(walk_k, dim3(n_seq), dim3(WALK_NT), smem, to_stream(stream), (const int*)anchor, (const int*)topk_ids,
                       (const float*)topk_vals, gate, gate_is_f32, (const __half*)pred_codebook, (const __half*)succ_codebook,
                       (int*)out_tokens, (float*)conf, rows, k, rank, (const WalkSamplingDev*)sampling, (const int*)row_off,
                       (float*)margin);
    return launch_status();
}
}  // namespace

GBS_EXPORT int gb_dflash_selector_walk_keyed(const void* anchor, const void* topk_ids, const void* topk_vals, const void* gate,
                                             int gate_is_f32, const void* pred_codebook, const void* succ_codebook, int n_seq, int rows,
                                             int k, int rank, const void* sampling, void* out_tokens, void* conf, void* stream) {
    if (n_seq <= 0 || rows <= 0) return 0;
    if (k < 1 || k > 64 || rank < 1 || rank > WALK_MAX_RANK) return GBS_ERR_INVALID;
    return launch_walk(anchor, topk_ids, topk_vals, gate, gate_is_f32, pred_codebook, succ_codebook, n_seq, rows, k, rank, sampling,
                       nullptr, out_tokens, conf, nullptr, stream);
}

GBS_EXPORT int gb_dflash_selector_walk_ragged(const void* anchor, const void* topk_ids, const void* topk_vals, const void* gate,
                                              int gate_is_f32, const void* pred_codebook, const void* succ_codebook, int n_seq, int k,
                                              int rank, const void* sampling, const void* row_off, void* out_tokens, void* conf,
                                              void* margin, void* stream) {
    if (n_seq <= 0) return 0;
    if (k < 1 || k > 64 || rank < 1 || rank > WALK_MAX_RANK || !row_off) return GBS_ERR_INVALID;
    return launch_walk(anchor, topk_ids, topk_vals, gate, gate_is_f32, pred_codebook, succ_codebook, n_seq, 0, k, rank, sampling,
                       row_off, out_tokens, conf, margin, stream);
}

GBS_EXPORT int gb_dflash_selector_walk(const void* anchor, const void* topk_ids, const void* topk_vals, const void* gate, int gate_is_f32,
                                       const void* pred_codebook, const void* succ_codebook, int n_seq, int rows, int k, int rank,
                                       void* out_tokens, void* conf, void* stream) {
    return gb_dflash_selector_walk_keyed(anchor, topk_ids, topk_vals, gate, gate_is_f32, pred_codebook, succ_codebook, n_seq, rows, k,
                                         rank, nullptr, out_tokens, conf, stream);
}

GBS_EXPORT int gb_dsv4_mtp_markov_walk_fast_bf16(void* logits, int* ids, const void* embed, const void* head, void* cand_ids_ws,
                                                 void* cand_scores_ws, int walk_rows, int vocab, int rank, void* stream) {
    return launch_markov_walk(logits, ids, nullptr, embed, head, cand_ids_ws, cand_scores_ws, walk_rows, vocab, rank, false, 1, 0, 0.0,
                              0.0, 0.0, 0, nullptr, stream);
}

GBS_EXPORT int gb_dsv4_mtp_markov_walk_keyed_bf16(void* logits, int* ids, float* conf, const void* embed, const void* head,
                                                  void* cand_ids_ws, void* cand_scores_ws, int walk_rows, int vocab, int rank,
                                                  int cand_k, unsigned long long seed, double temperature, double top_p, double min_p,
                                                  unsigned long long base_pos, void* stream) {
    return launch_markov_walk(logits, ids, conf, embed, head, cand_ids_ws, cand_scores_ws, walk_rows, vocab, rank, true, cand_k, seed,
                              temperature, top_p, min_p, base_pos, nullptr, stream);
}

GBS_EXPORT int gb_dsv4_mtp_markov_walk_keyed_bf16_params(void* logits, int* ids, float* conf, const void* embed, const void* head,
                                                         void* cand_ids_ws, void* cand_scores_ws, int walk_rows, int vocab, int rank,
                                                         const void* params, void* stream) {
    if (!params) return GBS_ERR_INVALID;
    return launch_markov_walk(logits, ids, conf, embed, head, cand_ids_ws, cand_scores_ws, walk_rows, vocab, rank, true, 1, 0, 0.0, 0.0,
                              0.0, 0, params, stream);
}

GBS_EXPORT const char* gbs_version(void) { return "gbsample-hip 0.1 (gfx950)"; }
