// The extended sampling pipeline (penalties, grammar bitmask, temperature, top-k/top-p/min-p, the inverse-CDF draw from
// one caller uniform per row), exact in integer masses. The definition of every step is in gbs_modeu.hpp and in the
// comment of sample_fast_k.
//
// Single-pass kernel (kmax in [1, 64]): grid (splits, rows) x 512 threads (8 waves); at 256 rows and more one block per row.
// One read of the row's logits, counts and mask words, in wave-steps of 1024 contiguous elements handed out through an
// LDS counter. Per element a lane computes the penalised, masked logit, the NaN flag and the online log-sum-exp, and
// offers the order key to its wave's gated top-64 list. The waves' lists are merged by a tree in LDS; with one block per
// row wave 0 then finishes the row (masses of the <= 64 candidates, the exact top-p cut and min-p filter, the draw in
// ascending id order, the log-probability). With several blocks per row the blocks hand their lists, LSE and NaN flag
// to the row's last block through the workspace.
#include <mutex>
#include <type_traits>

#include "gbs_modeu.hpp"
#include "pipeline_full.hpp"

using namespace gbs;
using namespace gbs::modeu;

namespace {

#ifndef GBS_FAST_MINBLOCKS
#define GBS_FAST_MINBLOCKS 1
#endif
#ifndef GBS_FAST_THREADS
#define GBS_FAST_THREADS 512
#endif
constexpr int NT = GBS_FAST_THREADS;
#ifndef GBS_FAST_LOAD_AUX
#define GBS_FAST_LOAD_AUX 2
#endif
constexpr int LOAD_AUX = GBS_FAST_LOAD_AUX;  // cache-policy bits of the logits and counts loads (2: non-temporal)
#ifndef GBS_FAST_MASK_AUX
#define GBS_FAST_MASK_AUX 0
#endif
constexpr int MASK_AUX = GBS_FAST_MASK_AUX;  // cache-policy bits of the mask-word loads
constexpr int NW = NT / WAVE;
#ifndef GBS_FAST_LATE_B
#define GBS_FAST_LATE_B 1  // the second buffer's first load: 0 at the start, 1 once the first's data has arrived, 2 after the seeding barrier
#endif
#ifndef GBS_FAST_GROUPS
#define GBS_FAST_GROUPS 4
#endif
#ifndef GBS_FAST_BLOCKS
#define GBS_FAST_BLOCKS 256
#endif
constexpr int GROUPS = GBS_FAST_GROUPS;  // 4-element groups per lane per step of the main loop
constexpr int HALF = 4;                  // groups ranked together
constexpr int GS = WAVE * 4;             // elements between a lane's groups: a wave-step is WAVE * 4 * GROUPS contiguous
constexpr int WSTEP = GS * GROUPS;       // elements of one wave-step
#ifndef GBS_FAST_FLUSH_GROUPS
#define GBS_FAST_FLUSH_GROUPS 1
#endif
constexpr int FLUSH_GROUPS = GBS_FAST_FLUSH_GROUPS;  // groups offered between two flushes of the wave buffer
constexpr int BUF = WAVE * (FLUSH_GROUPS * 4 + 1);
constexpr u64 FLOOR_KEY = ((u64)NEG_INF_KEY << 32) | 0xFFFFFFFFull;  // every -inf key is at or below it

constexpr int FAST_TARGET_BLOCKS = GBS_FAST_BLOCKS;
#ifndef GBS_FAST_MIN_CHUNK
#define GBS_FAST_MIN_CHUNK 8192
#endif
constexpr int FAST_MIN_CHUNK = GBS_FAST_MIN_CHUNK;  // elements: a row is split into chunks of at least this many

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int fast_splits(int rows, int vocab) {
    int s = (FAST_TARGET_BLOCKS + rows - 1) / rows;
    const int by_size = (vocab + FAST_MIN_CHUNK - 1) / FAST_MIN_CHUNK;
    if (s > by_size) s = by_size;
    if (s < 1) s = 1;
    return s;
}

// Workspace. Its first CTL_BYTES are the control region (pipeline_full.hpp): per-row arrival counters, which must be
// zero between launches, at offsets that depend only on the row (room for 65535 rows whatever this launch's row count);
// every launch leaves them zero. The full-distribution path keeps its counters in the same region, and per-row dispatch
// its flags, so one workspace serves launches of any shape on either path. The partial results after the region are
// written before they are read.
constexpr size_t CTL_BYTES = SAMPLE_CTL_BYTES;

struct FastWs {
    unsigned* arrive;  // [rows] the row's blocks that have handed over their partials
    u64* lists;     // [rows][S][64]
    Lse* lse;       // [rows][S]
    unsigned* nan;  // [rows][S]
    unsigned* defer;  // [rows] per-row dispatch: 1 for a row left to the full path (null without per-row dispatch)
    FsRow* fsrows;    // [rows] per-row dispatch: the full path's record of each row left to it
};

size_t fast_part_bytes(int rows, int S) {
    return align256((size_t)rows * S * WAVE * 8) + align256((size_t)rows * S * sizeof(Lse)) + align256((size_t)rows * S * 4);
}

FastWs fast_ws(void* ws, int rows, int S) {
    char* p = (char*)ws + CTL_BYTES;
    FastWs w;
    w.arrive = (unsigned*)ws;
    w.lists = (u64*)p;
    p += align256((size_t)rows * S * WAVE * 8);
    w.lse = (Lse*)p;
    p += align256((size_t)rows * S * sizeof(Lse));
    w.nan = (unsigned*)p;
    w.defer = nullptr;
    w.fsrows = nullptr;
    return w;
}

// One step of the main loop: GROUPS 4-element groups per lane, raw (unconverted) so that nothing waits on a load
// until the group is processed, one step later.
template <int DT>
struct RawStep {
    typename std::conditional<DT == GBS_DTYPE_F32, u32x4, u32x2>::type x[GROUPS];
    u32x4 c[GROUPS];
    u32 m[GROUPS];
};

// Buffer resources of one row (base, no stride, `bytes` records): a load at or past the row's end returns zeros and
// touches no memory. Every offset, the per-group ones included, goes into the per-lane offset, which the range check
// covers.
struct RowRsrc {
    __amdgpu_buffer_rsrc_t x, c, m;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, u32 bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Issue one wave-step's loads (e: the lane's first element).
template <int DT, bool COUNTS, bool MASK>
__device__ __forceinline__ void load_step(const RowRsrc& R, u32 e, RawStep<DT>& r) {
    constexpr u32 ESZ = DT == GBS_DTYPE_F32 ? 4 : 2;
#pragma unroll
    for (int j = 0; j < GROUPS; ++j) {
        // logits and counts are read once: non-temporal loads (cache policy bit 1)
        if constexpr (DT == GBS_DTYPE_F32) r.x[j] = __builtin_amdgcn_raw_buffer_load_b128(R.x, (e + j * GS) * ESZ, 0, LOAD_AUX);
        else r.x[j] = __builtin_amdgcn_raw_buffer_load_b64(R.x, (e + j * GS) * ESZ, 0, LOAD_AUX);
        if constexpr (COUNTS) r.c[j] = __builtin_amdgcn_raw_buffer_load_b128(R.c, (e + j * GS) * 4u, 0, LOAD_AUX);
        if constexpr (MASK) r.m[j] = __builtin_amdgcn_raw_buffer_load_b32(R.m, ((e >> 5) + j * (GS / 32)) * 4u, 0, MASK_AUX);
    }
}

template <int DT>
__device__ __forceinline__ void unpack_x(const RawStep<DT>& r, int j, float (&x)[4]) {
    if constexpr (DT == GBS_DTYPE_F32) {
        const u32x4 v = r.x[j];
        x[0] = __uint_as_float(v.x); x[1] = __uint_as_float(v.y); x[2] = __uint_as_float(v.z); x[3] = __uint_as_float(v.w);
    } else {
        const u32x2 v = r.x[j];
        widen2<DT>(v.x, x[0], x[1]);
        widen2<DT>(v.y, x[2], x[3]);
    }
}

template <int DT>
__device__ __forceinline__ float load_x1(const void* row, int e) {
    if constexpr (DT == GBS_DTYPE_F32) return ((const float*)row)[e];
    else return widen1<DT>((u32)((const u16*)row)[e]);
}

// The row's finish, on one wave. `list` holds the row's best 64 keys (lane = rank).
struct RowOut {
    int id, greedy, status;
    float prob, logprob;
};

constexpr int ROW_DEFERRED = -1;  // internal status: the row's cut is not provably inside the list (full path)

// Relative bound on |Z - Zf| / Z, where Z is a row's exact integer mass total and Zf = lse.s * 2^44 its value from the
// f32 online log-sum-exp over the same values at the same maximum: the exponents agree to |y| * 2^-23 (|y| < 64), the
// masses are 2^(44 + y) to within 2^-21, and the per-lane sums of at most 2^11 terms and their merges add at most
// 2^-12; 2^-10 leaves a margin of four.
constexpr double LSE_MASS_BOUND = 1.0 / 1024.0;

constexpr int SMALL_KEPT = 16;  // kept sets up to this size skip the sort by id

// An upper bound of the top-k set's exact mass for a row whose list (zk: its mass, e_last: its last mass) is full: from
// the log-sum-exp (top_k 0, and any top_k), and from the list for top_k above 64. 0 when no bound is known (the
// log-sum-exp is not at the maximum, or the maximum or 1/T is not finite).
__device__ __forceinline__ double kn_total_bound(const RowParamsDev& p, Lse lse, float M, float clp, u64 zk, u64 e_last) {
    double hi = 0.0;
    const bool lse_ok = lse.m == M && __builtin_isfinite(M) && __builtin_isfinite(clp) && lse.s > 0.0f && __builtin_isfinite(lse.s);
    if (lse_ok) hi = ceil(ldexp((double)lse.s, 44) * (1.0 + LSE_MASS_BOUND));
    if (p.top_k > WAVE) {
        const double k_hi = (double)zk + (double)(p.top_k - WAVE) * (double)e_last;
        hi = (hi == 0.0 || k_hi < hi) ? k_hi : hi;
    }
    // every mass is at most 2^44 and rows hold at most 2^19 tokens: the bound stays below 2^63
    const double cap = ldexp(1.0, 63) - 1.0;
    return hi > cap ? cap : hi;
}

// `open`: per-row dispatch's row without a top-k the list can hold (top_k 0 or above 64): its list holds the row's best
// 64 keys, and the row is finished here only when its cut provably lies inside them, else the status is ROW_DEFERRED.
__device__ RowOut finish_row(u64 list, const RowParamsDev& p, float u, bool invalid, bool nan, int count, Lse lse, float clp,
                             bool open = false) {
    RowOut o{-1, -1, GBS_ROW_OK, 0.f, __uint_as_float(0x7fc00000u)};
    const int l = lane_id();
    if (invalid) {
        o.status = GBS_ROW_INVALID_PARAMS;
        return o;
    }
    if (nan) {
        o.status = GBS_ROW_NAN_LOGIT;
        return o;
    }
    const u64 top = readlane64(list, 0);
    if (top <= FLOOR_KEY) {
        o.status = GBS_ROW_NO_CANDIDATES;
        return o;
    }
    const bool valid = l < count && list > FLOOR_KEY;
    const int kn = __popcll(ballot(valid));
    o.greedy = (int)key_id(top);
    const float M = okey_to_f32(key_ok(top));
    const float lval = okey_to_f32(key_ok(list));
    int chosen_rank = 0;
    if (p.temperature == 0.0f) {
        o.id = o.greedy;
        o.prob = 1.0f;
    } else {
        const float c2 = temp_scale(p.temperature);
        const u64 E = valid ? (mass_fast_ok(M, c2) ? mass_fast(lval, M, c2) : mass(lval, M, c2)) : 0ull;
        const u64 C = wave_scan_u64(E);
        const u64 zk = readlane64(C, WAVE - 1);
        const bool topp = p.top_p > 0.0f && p.top_p < 1.0f;
        // min-p filters the top-p prefix (the first token, of mass 2^44 >= Q, always stays)
        const u64 Q = p.min_p > 0.0f ? mul_ceil64(p.min_p, MASS_ONE) : 0ull;
        int keep = kn;
        if (open && kn == WAVE) {
            // The list is full, so the row has tokens beyond it. The top-k set's mass Z_K is bounded: at least the
            // list's; at most, for top_k above 64, the list's plus (top_k - 64) times its last mass; for top_k 0 it is
            // the row's total, which the log-sum-exp gives to within LSE_MASS_BOUND. The top-p cut is exact when both
            // ends of the bound put it at the same place inside the list; without top-p, min-p must drop the last entry.
            const u64 e_last = readlane64(E, WAVE - 1);
            const u64 zmax = (u64)kn_total_bound(p, lse, M, clp, zk, e_last);
            u64 zlo = zk, zhi = zmax;
            if (p.top_k == 0 && zhi != 0ull) {
                const double zf = ldexp((double)lse.s, 44);
                const u64 lo = (u64)(zf * (1.0 - LSE_MASS_BOUND));
                zlo = lo > zlo ? lo : zlo;
            }
            bool ok = false;
            if (topp) {
                if (zhi != 0ull && zlo <= zhi) {
                    const int blo = __popcll(ballot(valid && C < mul_ceil64(p.top_p, zlo)));
                    const int bhi = __popcll(ballot(valid && C < mul_ceil64(p.top_p, zhi)));
                    ok = blo == bhi && bhi < WAVE;
                    keep = blo + 1;
                }
            } else {
                ok = Q > 0ull && e_last < Q;
            }
            if (!ok) {
                o.status = ROW_DEFERRED;
                return o;
            }
        } else if (topp) {
            const u64 P = mul_ceil64(p.top_p, zk);
            const int below = __popcll(ballot(valid && C < P));
            keep = below + 1 < kn ? below + 1 : kn;
        }
        const bool kept = l < keep && E >= Q;
        const u64 km = ballot(kept);
        const u64 z = wave_sum_u64(kept ? E : 0ull);
        const u64 t = (u64)mul_floor(u, (u128)z, nullptr);
        if (__popcll(km) <= SMALL_KEPT) {
            // few kept tokens: each one's running mass in ascending id order by a scalar loop over the others, then
            // the smallest id whose running mass exceeds t
            const u32 idj = key_id(list);
            u64 cum = 0;
            for (u64 mm = km; mm; mm &= mm - 1ull) {
                const int i = (int)__builtin_ctzll(mm);
                const u64 Ei = readlane64(E, i);
                const u32 idi = (u32)__builtin_amdgcn_readlane((int)idj, i);
                cum += idi <= idj ? Ei : 0ull;
            }
            u64 hit = ballot(kept && cum > t);
            int f = (int)__builtin_ctzll(hit | (1ull << 63));
            u32 best = 0xFFFFFFFFu;
            for (; hit; hit &= hit - 1ull) {
                const int i = (int)__builtin_ctzll(hit);
                const u32 idi = (u32)__builtin_amdgcn_readlane((int)idj, i);
                if (idi < best) {
                    best = idi;
                    f = i;
                }
            }
            chosen_rank = f;
            o.id = (int)best;
            o.prob = (float)((double)readlane64(E, f) / (double)z);
        } else {
            // kept tokens in ascending id order: sort (id << 6 | rank) in 32 bits (ids below 2^25, ranks below 64)
            static_assert(GBS_MAX_VOCAB <= (1 << 25), "ids fit in 26 bits beside a 6-bit rank");
            const u32 sk = wave_sort_asc32(kept ? ((key_id(list) << 6) | (u32)l) : 0xFFFFFFFFu);
            const bool skept = sk != 0xFFFFFFFFu;
            const int rank = (int)(sk & 63u);
            const u64 Es = shfl64(E, skept ? rank : 0);
            const u64 cum = wave_scan_u64(skept ? Es : 0ull);
            const u64 hit = ballot(skept && cum > t);
            const int f = hit ? (int)__builtin_ctzll(hit) : 0;
            const u32 skf = (u32)__builtin_amdgcn_readlane((int)sk, f);
            chosen_rank = (int)(skf & 63u);
            o.id = (int)(skf >> 6);
            const u64 ec = readlane64(Es, f);
            o.prob = (float)((double)ec / (double)z);
        }
    }
    // log-softmax of the chosen token over the allowed tokens, base-2 online sums
    const float lx = __uint_as_float(readlane32(__float_as_uint(lval), chosen_rank));
    if (isinf(M) || !isfinite(clp)) o.logprob = __uint_as_float(0x7fc00000u);  // undefined: +inf maximum, 1/T beyond f32
    else o.logprob = ((lx - lse.m) * clp - log2f(lse.s)) * 0.6931471805599453f;
    return o;
}

__device__ __forceinline__ void write_row(int r, const RowOut& o, int* out_ids, int* out_greedy, float* out_probs,
                                          float* out_logprobs, int* out_status) {
    out_ids[r] = o.id;
    if (out_greedy) out_greedy[r] = o.greedy;
    if (out_probs) out_probs[r] = o.prob;
    if (out_logprobs) out_logprobs[r] = o.status == GBS_ROW_OK ? o.logprob : __uint_as_float(0x7fc00000u);
    if (out_status) out_status[r] = o.status;
}

template <int DT, bool COUNTS, bool MASK, bool LOGPROB>
__global__ void __launch_bounds__(NT, GBS_FAST_MINBLOCKS) sample_fast_k(const void* __restrict__ logits, long long stride, int vocab, int chunk,
                                                    const int* __restrict__ counts, const u32* __restrict__ mask,
                                                    const RowParamsDev* __restrict__ params, const float* __restrict__ uniforms,
                                                    int kmax, bool vec, FastWs ws, int* __restrict__ out_ids,
                                                    int* __restrict__ out_greedy, float* __restrict__ out_probs,
                                                    float* __restrict__ out_logprobs, int* __restrict__ out_status) {
    __shared__ u64 s_buf[NW][BUF];
    __shared__ u64 s_list[NW][WAVE];
    __shared__ Lse s_lse[NW];
    __shared__ unsigned s_nan[NW];
    __shared__ unsigned s_flag;
    __shared__ u64 s_thr;
    __shared__ u32 s_top[NW * WaveTop<BUF>::TOPN];
    const int S = gridDim.x, sp = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x, w = tid / WAVE, l = lane_id();
    const size_t esz = DT == GBS_DTYPE_F32 ? 4 : 2;
    const void* row = (const char*)logits + (size_t)r * (size_t)stride * esz;
    const int* crow = COUNTS ? counts + (size_t)r * vocab : nullptr;
    const u32* mrow = MASK ? mask + (size_t)r * ((vocab + 31) / 32) : nullptr;
    const int lo = sp * chunk;
    const int hi = min(vocab, lo + chunk);
    // Wave-steps of WSTEP contiguous elements: wave w's first two (w and NW + w) are fixed, so their loads go out at
    // once, before the block's first barrier and the row's parameters; later ones come from an LDS counter.
    const int nws = vec ? (hi - lo + WSTEP - 1) / WSTEP : 0;
    const RowRsrc R{rsrc(row, (u32)vocab * (u32)esz), rsrc(crow, COUNTS ? (u32)vocab * 4u : 0u),
                    rsrc(mrow, MASK ? (u32)((vocab + 31) / 32) * 4u : 0u)};
    auto wstep_e = [&](int idx) { return lo + idx * WSTEP + l * 4; };
    RawStep<DT> A, B;
    if (w < nws) load_step<DT, COUNTS, MASK>(R, (u32)wstep_e(w), A);
    if (!GBS_FAST_LATE_B && NW + w < nws) load_step<DT, COUNTS, MASK>(R, (u32)wstep_e(NW + w), B);
    auto late_b = [&](int when) {
        if (GBS_FAST_LATE_B == when && NW + w < nws) load_step<DT, COUNTS, MASK>(R, (u32)wstep_e(NW + w), B);
    };
    __shared__ int s_next;
    if (tid == 0) {
        s_thr = 0;
        s_next = 2 * NW;
    }
    if (tid < NW * WaveTop<BUF>::TOPN) s_top[tid] = 0;
    __syncthreads();
    const RowParamsDev p = params[r];
    const float u = uniforms[r];
    // kmax < 0: per-row dispatch; a row with top_k 0 or above 64 is `open` (its list keeps 64 keys)
    const bool mixed = kmax < 0;
    const bool open = mixed && (p.top_k == 0 || p.top_k > WAVE);
    const bool invalid = params_invalid(p, u) || (!mixed && (p.top_k < 1 || p.top_k > kmax));
    const int count = invalid ? 1 : (open ? WAVE : p.top_k);
    const float rinv = 1.0f / p.repetition;
    const float rep = p.repetition, freq = p.frequency, pres = p.presence;  // plain scalars for the element loop
    const float clp = p.temperature > 0.0f ? temp_scale(p.temperature) : 1.44269504088896340736f;

    WaveTop<BUF> wt;
    wt.init(s_buf[w], count, FLOOR_KEY, &s_thr);
    wt.set_top(s_top, w, NW);
    Lse lse{-INFINITY, 0.f};

    // the penalised logit of one element, in the operation order of the definition:
    // c > 0: (x > 0 ? x * rinv : x * rep) - ((float)c * freq + pres); otherwise x.
    auto penalized = [&](float x, int c) {
        float v = x;
        if (COUNTS) {
            const float a = x * (x > 0.0f ? rinv : rep);
            const float b = (float)c * freq + pres;
            v = c > 0 ? a - b : x;
        }
        return v;
    };
    u32 nanv = 0;  // per lane: a NaN was seen
    const float lse_c = clp;
    // one 4-element group: penalties, mask, NaN flag, keys offered to the wave list, online log-sum-exp.
    // The mask is applied with a bitfield insert: bfe_i32 of the element's bit is all ones or all zeros.
    auto group = [&](const float (&x)[4], const int (&c)[4], u32 mbits, int eg) {
        float lv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float v = penalized(x[q], c[q]);
            const u32 keep = (u32)__builtin_amdgcn_sbfe((int)mbits, q, 1);
            lv[q] = __uint_as_float((__float_as_uint(v) & keep) | (0xFF800000u & ~keep));
        }
        nanv |= (__builtin_isunordered(lv[0], lv[1]) | __builtin_isunordered(lv[2], lv[3])) ? 1u : 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) wt.offer_f(lv[q], (u32)(eg + q));
        if (LOGPROB) {
            const float gm = fmaxf(fmaxf(lv[0], lv[1]), fmaxf(lv[2], lv[3]));
            if (gm > lse.m) {
                lse.s = lse.m == -INFINITY ? 0.f : lse.s * __builtin_amdgcn_exp2f((lse.m - gm) * lse_c);
                lse.m = gm;
            }
            if (lse.m != -INFINITY) {
#pragma unroll
                for (int q = 0; q < 4; ++q) lse.s += __builtin_amdgcn_exp2f((lv[q] - lse.m) * lse_c);
            }
        }
    };

    int e0 = lo;
    if (vec) {
        // Wave-steps of WSTEP contiguous elements (GROUPS 4-element groups per lane, GS apart): all of a wave-step's
        // loads are issued together, then it is ranked in halves of HALF groups. Wave w takes wave-step w first (the
        // gate is seeded from it); later wave-steps go to whichever wave asks first (an LDS counter), so that waves
        // the memory system serves late do not hold the block. The last wave-step may run past the chunk: its loads
        // stay inside the row (the buffer resource returns zeros past the row's end) and its out-of-chunk groups are
        // masked to -inf.
        constexpr int NE = HALF * 4;
        auto penal_fn = [&](RawStep<DT>& B, int h, int e, bool guard, float (&lv)[NE]) __attribute__((always_inline)) {
#pragma unroll
            for (int jj = 0; jj < HALF; ++jj) {
                const int j = h * HALF + jj;
                const int eg = e + j * GS;
                float x[4];
                unpack_x<DT>(B, j, x);
                u32 mb = MASK ? (B.m[j] >> (eg & 31)) : 0xFu;
                if (guard && eg >= hi) mb = 0u;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32 keep = (MASK || guard) ? (u32)__builtin_amdgcn_sbfe((int)mb, q, 1) : 0xFFFFFFFFu;
                    float v = x[q];
                    if (COUNTS) {
                        const int c = (int)B.c[j][q];
                        if (ballot(c > 0 && keep != 0u)) v = penalized(x[q], c);
                    }
                    lv[jj * 4 + q] = __uint_as_float((__float_as_uint(v) & keep) | (0xFF800000u & ~keep));
                }
            }
        };
        // NaN flag, gate test and offers, online log-sum-exp of one half (element i of lane group jj: id e + jj*GS + q)
        auto rank_fn = [&](const float (&lv)[NE], int e) __attribute__((always_inline)) {
            bool nan_step = false;
#pragma unroll
            for (int i = 0; i < NE; i += 2) nan_step |= __builtin_isunordered(lv[i], lv[i + 1]);
            nanv |= nan_step ? 1u : 0u;
            // group maxima, then the half's maximum (a NaN element never raises either, and never passes the gate)
            float gmax[HALF];
#pragma unroll
            for (int jj = 0; jj < HALF; ++jj)
                gmax[jj] = fmaxf(fmaxf(lv[jj * 4], lv[jj * 4 + 1]), fmaxf(lv[jj * 4 + 2], lv[jj * 4 + 3]));
            float gm = gmax[0];
#pragma unroll
            for (int jj = 1; jj < HALF; ++jj) gm = fmaxf(gm, gmax[jj]);
            // the gate in two levels: the half's maximum, then each group's; only a group with a candidate tests its
            // elements (a lane whose values are all NaN also tests its elements, which never pass)
            if (ballot(!(gm < wt.gate_f))) {
#pragma unroll
                for (int jj = 0; jj < HALF; ++jj) {
                    if (ballot(!(gmax[jj] < wt.gate_f))) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) wt.offer_f(lv[jj * 4 + q], (u32)(e + jj * GS + q));
                        wt.flush(false);
                    }
                }
            }
            if (LOGPROB) {
                if (gm > lse.m) {
                    lse.s = lse.m == -INFINITY ? 0.f : lse.s * __builtin_amdgcn_exp2f((lse.m - gm) * lse_c);
                    lse.m = gm;
                }
                // a half that is -inf on every lane adds exactly 0
                if (lse.m != -INFINITY && ballot(gm != -INFINITY)) {
                    // the difference first: exact for values near the maximum at any magnitude (a product l * c
                    // rounded at |l| ~ 1e6 would shift every exponent by up to ulp(l * c))
#pragma unroll
                    for (int i = 0; i < NE; ++i) lse.s += __builtin_amdgcn_exp2f((lv[i] - lse.m) * lse_c);
                }
            }
        };
        // rank one loaded wave-step (idx: its index; the last one is guarded; the first of each wave seeds the gate).
        // `reload` runs as soon as the step's logits are computed: the buffer's registers are free from there on, so
        // the next load is in flight while this step is ranked.
        static_assert(GROUPS == HALF, "one half per wave-step");
        auto step_fn = [&](RawStep<DT>& B, int e, int idx, bool first, auto&& reload) __attribute__((always_inline)) {
            const bool guard = idx == nws - 1;
            wt.apply_shared();
            wt.prefetch_shared();
            float lv[NE];
            if (guard) penal_fn(B, 0, e, true, lv);
            else penal_fn(B, 0, e, false, lv);
            if (first) {
                late_b(1);  // after this wave-step's data has arrived
                // the gate starts from the lanes' maxima of the first wave-step: the wave's count-th largest of
                // them, then the block bound of every wave's best ones
                u32 m = 0;
#pragma unroll
                for (int i = 0; i < NE; ++i) {
                    const u32 k = lv[i] != lv[i] ? 0u : okey_f32_fast(lv[i]);
                    m = k > m ? k : m;
                }
                wt.seed(m);
                __syncthreads();
                late_b(2);
                wt.block_bound();
            }
            reload();
            rank_fn(lv, e);
        };
        // Two wave-steps in flight per wave: A and B alternate; a buffer is reloaded with the next wave-step as soon
        // as it is ranked. A wave-step index at or past nws loads nothing and ends the loop.
        auto grab = [&]() {
            int t = 0;
            if (l == 0) t = __hip_atomic_fetch_add(&s_next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            return __builtin_amdgcn_readfirstlane(t);
        };
        int ia = w;       // loaded at the kernel's start
        int ib = NW + w;  // likewise
        if (ia >= nws) {
            // no wave-step of its own: take part in the block's seeding barrier
            wt.seed(0u);
            __syncthreads();
            wt.block_bound();
        } else {
            // the buffers in turn; each is refilled with the next wave-step as soon as its logits are computed
            auto refill = [&](RawStep<DT>& X, int& nx) {
                nx = grab();
                if (nx < nws) load_step<DT, COUNTS, MASK>(R, (u32)wstep_e(nx), X);
            };
            for (bool first = true;; first = false) {
                int na = 0, nb = 0;
                step_fn(A, wstep_e(ia), ia, first, [&]() { refill(A, na); });
                ia = na;
                if (ib >= nws) break;
                step_fn(B, wstep_e(ib), ib, false, [&]() { refill(B, nb); });
                ib = nb;
                if (ia >= nws) break;
            }
        }
        e0 = hi;
    }
    // the rest of the chunk (or all of it when 16-byte loads are not legal), one group per lane per round, guarded
    {
        const int rounds = (hi - e0 + NT * 4 - 1) / (NT * 4);
        for (int k = 0; k < rounds; ++k) {
            const int eg = e0 + k * NT * 4 + tid * 4;
            float x[4];
            int c[4];
            u32 mb = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool in = eg + q < hi;
                x[q] = in ? load_x1<DT>(row, eg + q) : 0.f;
                c[q] = (COUNTS && in) ? crow[eg + q] : 0;
                const u32 bit = MASK ? (in ? (mrow[(eg + q) >> 5] >> ((eg + q) & 31)) & 1u : 0u) : (in ? 1u : 0u);
                mb |= bit << q;
            }
            group(x, c, mb, eg);
            wt.flush(false);
        }
    }
    // the latest block bound first: the last partial buffer is filtered against it
    wt.prefetch_shared();
    wt.apply_shared();
    wt.flush(true);

    // block reduction: lists, LSE, NaN
    if (LOGPROB) lse = wave_lse(lse, clp);
    const bool wnan = ballot(nanv != 0u) != 0ull;
    Lse rl{-INFINITY, 0.f};
    unsigned rn = 0;
    u64 list;
    if (l == 0) {
        s_lse[w] = lse;
        s_nan[w] = wnan ? 1u : 0u;
    }
    wt.list = block_tree_merge<NW>(wt.list, s_list);  // also orders s_lse / s_nan before the reads below
    if (S == 1) {
        if (w != 0) return;
        if (l < NW) {
            rl = s_lse[l];
            rn = s_nan[l];
        }
        list = wt.list;
    } else {
        if (w == 0) {
            const size_t slot = (size_t)r * S + sp;
            st_agent(&ws.lists[slot * WAVE + l], wt.list);
            if (l == 0) {
                Lse b = s_lse[0];
                unsigned bn = s_nan[0];
                for (int o = 1; o < NW; ++o) {
                    if (LOGPROB) b = lse_merge(b, s_lse[o], clp);
                    bn |= s_nan[o];
                }
                st_agent_f2((float2*)&ws.lse[slot], make_float2(b.m, b.s));
                st_agent(&ws.nan[slot], bn);
            }
        }
        if (!arrive_last(&ws.arrive[r], (unsigned)S, &s_flag)) return;
        list = block_merge_lists<NW>(ws.lists + (size_t)r * S * WAVE, S, s_list);
        if (w != 0) return;
        for (int o = l; o < S; o += WAVE) {
            if (LOGPROB) {
                const float2 f = ld_agent_f2((const float2*)&ws.lse[(size_t)r * S + o]);
                rl = lse_merge(rl, Lse{f.x, f.y}, clp);
            }
            rn |= ld_agent(&ws.nan[(size_t)r * S + o]);
        }
    }
    if (LOGPROB) rl = wave_lse(rl, clp);  // lanes without a partial hold (-inf, 0)
    rn = wave_or(rn);
    const RowOut o = finish_row(list, p, u, invalid, rn != 0u, count, rl, clp, open);
    const u64 top = readlane64(list, 0);
    if (l == 0) {
        if (ws.defer) ws.defer[r] = o.status == ROW_DEFERRED ? 1u : 0u;
        if (o.status != ROW_DEFERRED) {
            write_row(r, o, out_ids, out_greedy, out_probs, out_logprobs, out_status);
        } else {
            // the full path's record of the row, as its pass 0 would write it (which it then skips): a flagged row is
            // valid, NaN-free, has 64 allowed tokens or more and T > 0; a top_k above 64 takes the radix path
            FsRow* fr = ws.fsrows + r;
            const float M = okey_to_f32(key_ok(top));
            const bool radix = p.top_k > WAVE || !mass_fast_ok(M, temp_scale(p.temperature));
            st_agent(&fr->top, top);
            st_agent((u32*)&fr->lse_m, __float_as_uint(rl.m));
            st_agent((u32*)&fr->lse_s, __float_as_uint(rl.s));
            st_agent(&fr->nallowed, (u32)WAVE);
            st_agent(&fr->bstar, FS_NBINS);
            st_agent(&fr->above, (u64)0);
            st_agent(&fr->P, (u64)0);
            st_agent(&fr->state, radix ? (u32)FS_RADIX : (u32)FS_CUT);
        }
    }
}

// calls f.template operator()<COUNTS, MASK, LOGPROB>() for the run-time flags
template <class F>
void dispatch_flags(bool c, bool m, bool lp, F&& f) {
    if (c && m && lp) f.template operator()<true, true, true>();
    else if (c && m) f.template operator()<true, true, false>();
    else if (c && lp) f.template operator()<true, false, true>();
    else if (c) f.template operator()<true, false, false>();
    else if (m && lp) f.template operator()<false, true, true>();
    else if (m) f.template operator()<false, true, false>();
    else if (lp) f.template operator()<false, false, true>();
    else f.template operator()<false, false, false>();
}

}  // namespace

GBS_EXPORT size_t gbs_sample_workspace_bytes(int rows, int vocab, int kmax) {
    if (rows <= 0 || vocab <= 0 || vocab > GBS_MAX_VOCAB || kmax < GBS_KMAX_MIXED || kmax > GBS_MAX_COUNT) return 0;
    if (kmax == 0) return sample_full_workspace_bytes(rows, vocab);
    const size_t fast = CTL_BYTES + fast_part_bytes(rows, fast_splits(rows, vocab));
    if (kmax > 0) return fast;
    // per-row dispatch: the single-pass kernel's workspace, then the full path's for the rows it leaves over
    const size_t full = sample_full_deferred_workspace_bytes(rows, vocab);
    return fast > full ? fast : full;
}

GBS_EXPORT int gbs_sample_rows(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts, const uint32_t* mask,
                               const GbsRowParams* params, const float* uniforms, int kmax, int* out_ids, int* out_greedy,
                               float* out_probs, float* out_logprobs, int* out_status, void* ws, size_t ws_bytes, void* stream) {
    if (rows < 0 || vocab <= 0 || vocab > GBS_MAX_VOCAB || stride < vocab || kmax < GBS_KMAX_MIXED || kmax > GBS_MAX_COUNT)
        return GBS_ERR_INVALID;
    if (dtype != GBS_DTYPE_F32 && dtype != GBS_DTYPE_BF16 && dtype != GBS_DTYPE_F16) return GBS_ERR_INVALID;
    if (rows == 0) return 0;
    if (rows > 65535 || !logits || !params || !uniforms || !out_ids) return GBS_ERR_INVALID;
    if (kmax == 0) {
        if (ws_bytes < sample_full_workspace_bytes(rows, vocab)) return GBS_ERR_INVALID;
        return launch_sample_full(logits, dtype, rows, stride, vocab, counts, mask, params, uniforms, out_ids, out_greedy, out_probs,
                                  out_logprobs, out_status, ws, ws_bytes, stream);
    }
    if (!ws || !aligned(ws, 256)) return GBS_ERR_INVALID;
    const int S = fast_splits(rows, vocab);
    if (ws_bytes < gbs_sample_workspace_bytes(rows, vocab, kmax)) return GBS_ERR_INVALID;
    int chunk = (vocab + S - 1) / S;
    chunk = (chunk + 31) / 32 * 32;  // whole mask words per chunk
    const size_t esz = dtype == GBS_DTYPE_F32 ? 4 : 2;
    const bool vec = stride % 4 == 0 && vocab % 4 == 0 && aligned(logits, 4 * esz) && (!counts || aligned(counts, 16));
    const hipStream_t st = to_stream(stream);
    const RowParamsDev* p = (const RowParamsDev*)params;
    const bool mixed = kmax == GBS_KMAX_MIXED;
    FastWs w = fast_ws(ws, rows, S);
    if (mixed) {
        w.defer = (unsigned*)((char*)ws + SAMPLE_DEFER_OFFSET);
        w.fsrows = (FsRow*)((char*)ws + SAMPLE_FSROW_OFFSET);
    }
    auto run = [&]<int DT>() {
        // per-row dispatch bounds open rows by the log-sum-exp: it is computed whether or not log-probabilities are asked
        dispatch_flags(counts != nullptr, mask != nullptr, mixed || out_logprobs != nullptr, [&]<bool C, bool M, bool L>() {
            hipLaunchKernelGGL((sample_fast_k<DT, C, M, L>), dim3(S, rows), dim3(NT), 0, st, logits, (long long)stride, vocab, chunk,
                               counts, mask, p, uniforms, kmax, vec, w, out_ids, out_greedy, out_probs, out_logprobs, out_status);
        });
    };
    if (dtype == GBS_DTYPE_F32) run.template operator()<GBS_DTYPE_F32>();
    else if (dtype == GBS_DTYPE_BF16) run.template operator()<GBS_DTYPE_BF16>();
    else run.template operator()<GBS_DTYPE_F16>();
    if (!mixed) return launch_status();
    const int rc = launch_status();
    if (rc != 0) return rc;
    // the rows the single pass left over (their flags set): the full-distribution path
    return launch_sample_full(logits, dtype, rows, stride, vocab, counts, mask, params, uniforms, out_ids, out_greedy, out_probs,
                              out_logprobs, out_status, ws, ws_bytes, stream, w.defer);
}

// ------------------------------------------------------------------------------------------------ allocation-free form
// gbs_sample_rows for callers that cannot allocate: the workspace is this file-scope device array, one copy per GPU,
// held until the process ends. Host code never passes the array's name to a kernel (on the host it is only a
// stand-in): at a device's first call its device address is looked up once, with that device current, and kept per
// device. The first call also clears the array (a fill kernel on the caller's stream, ahead of that call's launches);
// every later call starts from the zeroed arrival counters the previous one left. Calls on one GPU share the array:
// calls that overlap (other streams, other host threads) race.

namespace {

static __device__ __align__(256) unsigned char scratch[GBS_NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
void* g_scratch[NOALLOC_MAX_DEVICES] = {};
std::mutex g_scratch_mu;

// the calling device's copy of `scratch`, cleared on first use; nullptr (and *rc set) on a HIP error
void* device_scratch(void* stream, int* rc) {
    int d = -1;
    if ((*rc = (int)hipGetDevice(&d)) != 0) return nullptr;
    if (d < 0 || d >= NOALLOC_MAX_DEVICES) {
        *rc = GBS_ERR_INVALID;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[d] == nullptr) {
        void* ptr = nullptr;
        if ((*rc = (int)hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) != 0 || ptr == nullptr) {
            if (*rc == 0) *rc = GBS_ERR_INVALID;
            return nullptr;
        }
        if ((*rc = gbs_workspace_clear(ptr, GBS_NOALLOC_SCRATCH_BYTES, stream)) != 0) return nullptr;
        g_scratch[d] = ptr;
    }
    *rc = 0;
    return g_scratch[d];
}

}  // namespace

GBS_EXPORT int gbs_sample_rows_noalloc(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts,
                                       const uint32_t* mask, const GbsRowParams* params, const float* uniforms, int kmax, int* out_ids,
                                       int* out_greedy, float* out_probs, float* out_logprobs, int* out_status, void* stream) {
    if (rows < 0 || vocab <= 0 || vocab > GBS_MAX_VOCAB || stride < vocab || kmax < GBS_KMAX_MIXED || kmax > GBS_MAX_COUNT)
        return GBS_ERR_INVALID;
    if (dtype != GBS_DTYPE_F32 && dtype != GBS_DTYPE_BF16 && dtype != GBS_DTYPE_F16) return GBS_ERR_INVALID;
    if (rows == 0) return 0;
    if (rows > 65535) return GBS_ERR_INVALID;
    if (gbs_sample_workspace_bytes(rows, vocab, kmax) > GBS_NOALLOC_SCRATCH_BYTES) return GBS_ERR_NOALLOC_TOO_LARGE;
    int rc = 0;
    void* ws = device_scratch(stream, &rc);
    if (ws == nullptr) return rc;
    return gbs_sample_rows(logits, dtype, rows, stride, vocab, counts, mask, params, uniforms, kmax, out_ids, out_greedy, out_probs,
                           out_logprobs, out_status, ws, GBS_NOALLOC_SCRATCH_BYTES, stream);
}
