// The extended pipeline's full-distribution path (gbs_sample_rows with kmax == 0): any top_k (0 = off), top-p over the
// whole vocabulary, min-p and the inverse-CDF draw, exact in integer masses, with the same definition as the single-pass
// kernel (gbs_modeu.hpp).
//
// One block of 1024 threads per row; every pass streams the row's logits, counts and mask words again (coalesced
// 4-element groups). The exact cuts are radix selections over the 64-bit order keys (value, ~id), 11 bits per pass, on
// LDS histograms of (count, mass, largest key) per digit; a pass ends early when the crossing digit holds one key.
//   pass 0            row maximum (greedy id), NaN flag, number of allowed tokens, online log-sum-exp
//   top-k passes      the top_k-th key by count (and the mass above it)            if 0 < top_k < allowed
//   top-p passes      the key where the descending cumulative mass reaches P         if 0 < top_p < 1
//   draw passes       kept-mass sums per 4096-element tile, then a scan of the one tile holding the draw
// No radix pass sorts anything: each only counts the keys that share the prefix found so far.
#include "gbs_modeu.hpp"
#include "pipeline_full.hpp"

using namespace gbs;
using namespace gbs::modeu;

namespace {

constexpr int NTF = 1024;
constexpr int NWF = NTF / WAVE;
constexpr int DB = 11;
constexpr int NB = 1 << DB;
constexpr int TILE = NTF * 4;
constexpr int MAX_TILES = (GBS_MAX_VOCAB + TILE - 1) / TILE;
constexpr u32 VALID_MIN_OK = NEG_INF_KEY + 1u;  // order values above -inf

template <int DT, bool COUNTS, bool MASK>
struct Row {
    const void* x;
    const int* c;
    const u32* m;
    int vocab;
    bool vec;
    float rinv, rep, freq, pres;

    __device__ __forceinline__ float pen(float v, int cnt) const {
        if (COUNTS && cnt > 0) {
            const float a = v > 0.0f ? v * rinv : v * rep;
            return a - ((float)cnt * freq + pres);
        }
        return v;
    }

    // Raw loads of one 4-element group, for the pipelined streaming of whole rows (vec rows only): buffer loads whose
    // range check returns zeros past the row's end, so nothing waits on a bounds test before the loads are issued.
    // AUX: the logits' and counts' cache policy (2: non-temporal); mask words, shared by 32 elements, use the default.
    struct Raw {
        u32x4 x;  // f32: 4 values; bf16: the first two words
        u32x4 c;
        u32 m;
    };
    template <int AUX = 0>
    __device__ __forceinline__ void load_raw(int e, const __amdgpu_buffer_rsrc_t& rx, const __amdgpu_buffer_rsrc_t& rc,
                                             const __amdgpu_buffer_rsrc_t& rm, Raw& w) const {
        if (DT == GBS_DTYPE_F32) w.x = __builtin_amdgcn_raw_buffer_load_b128(rx, (u32)e * 4u, 0, AUX);
        else {
            const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rx, (u32)e * 2u, 0, AUX);
            w.x = u32x4{v.x, v.y, 0u, 0u};
        }
        if (COUNTS) w.c = __builtin_amdgcn_raw_buffer_load_b128(rc, (u32)e * 4u, 0, AUX);
        if (MASK) w.m = __builtin_amdgcn_raw_buffer_load_b32(rm, (u32)(e >> 5) * 4u, 0, 0);
    }
    // the penalised, masked logits of a raw group at e (out of range: -inf). The raw loads serve rows of whole groups
    // (vocab % 4 == 0), so a group is in range or out of it as a whole; the penalty is computed for every element and
    // selected, without branches.
    __device__ __forceinline__ void from_raw(const Raw& w, int e, float (&l)[4]) const {
        float xv[4];
        if (DT == GBS_DTYPE_F32) {
            xv[0] = __uint_as_float(w.x.x); xv[1] = __uint_as_float(w.x.y); xv[2] = __uint_as_float(w.x.z); xv[3] = __uint_as_float(w.x.w);
        } else {
            widen2<DT>(w.x.x, xv[0], xv[1]);
            widen2<DT>(w.x.y, xv[2], xv[3]);
        }
        const bool gin = e < vocab;
        const u32 mw = MASK ? w.m >> (e & 31) : 0xFu;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float v = xv[q];
            if (COUNTS) {
                const int cnt = (int)w.c[q];
                const float a = v > 0.0f ? v * rinv : v * rep;
                const float pv = a - ((float)cnt * freq + pres);
                v = cnt > 0 ? pv : v;
            }
            l[q] = gin && ((mw >> q) & 1u) ? v : -INFINITY;
        }
    }

    // the penalised, masked logits of elements e..e+3 (out of range: -inf)
    __device__ __forceinline__ void group(int e, float (&l)[4]) const {
        float xv[4];
        int cv[4] = {0, 0, 0, 0};
        if (vec && e + 4 <= vocab) {
            if (DT == GBS_DTYPE_F32) {
                const float4 v = *(const float4*)((const float*)x + e);
                xv[0] = v.x; xv[1] = v.y; xv[2] = v.z; xv[3] = v.w;
            } else {
                const uint2 v = *(const uint2*)((const u16*)x + e);
                widen2<DT>(v.x, xv[0], xv[1]);
                widen2<DT>(v.y, xv[2], xv[3]);
            }
            if (COUNTS) {
                const int4 cc = *(const int4*)(c + e);
                cv[0] = cc.x; cv[1] = cc.y; cv[2] = cc.z; cv[3] = cc.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool in = e + q < vocab;
                if constexpr (DT == GBS_DTYPE_F32) xv[q] = in ? ((const float*)x)[e + q] : 0.f;
                else xv[q] = in ? widen1<DT>((u32)((const u16*)x)[e + q]) : 0.f;
                if (COUNTS) cv[q] = in ? c[e + q] : 0;
            }
        }
        const u32 mw = MASK ? (e < vocab ? m[e >> 5] >> (e & 31) : 0u) : 0xFu;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool in = e + q < vocab && ((mw >> q) & 1u);
            l[q] = in ? pen(xv[q], cv[q]) : -INFINITY;
        }
    }
};

__device__ __forceinline__ bool valid_l(float v) { return v > -INFINITY; }  // false for NaN and -inf

// Pass 0 of a lane, one 4-element group at a time: the largest allowed value and its lowest id (the row's greedy key;
// -0 and +0 share a key, so float comparisons order values as the keys do), the NaN flag, the number of allowed tokens
// and the online log-sum-exp in base 2 (rescaled once per group, at the group's maximum).
struct Pass0Acc {
    float bv = -INFINITY;
    u32 bid = 0, nan = 0, nallowed = 0;
    Lse lse{-INFINITY, 0.f};

    __device__ __forceinline__ void add(const float (&l)[4], int e, float c) {
        nan |= (__builtin_isunordered(l[0], l[1]) | __builtin_isunordered(l[2], l[3])) ? 1u : 0u;
        nallowed += (u32)valid_l(l[0]) + (u32)valid_l(l[1]) + (u32)valid_l(l[2]) + (u32)valid_l(l[3]);
        const float gm = fmaxf(fmaxf(l[0], l[1]), fmaxf(l[2], l[3]));  // NaN only when all four are NaN
        if (gm > bv) {  // strictly: on a tie the earlier (lower) id stays
            bv = gm;
            bid = (u32)e + (l[0] == gm ? 0u : l[1] == gm ? 1u : l[2] == gm ? 2u : 3u);
        }
        if (gm > lse.m) {
            lse.s = lse.m == -INFINITY ? 0.f : lse.s * __builtin_amdgcn_exp2f((lse.m - gm) * c);
            lse.m = gm;
        }
        if (lse.m != -INFINITY) {
            // the difference first: exact near the maximum at any magnitude
#pragma unroll
            for (int q = 0; q < 4; ++q) lse.s += __builtin_amdgcn_exp2f((l[q] - lse.m) * c);
        }
    }
    __device__ __forceinline__ u64 key() const { return bv > -INFINITY ? make_key(okey_f32(bv), bid) : 0ull; }
};

// A load of what an earlier launch on the stream wrote (launch boundaries make it visible; a plain load may be served
// by the caches).
template <typename T>
__device__ __forceinline__ T ld_prev(const T* p) {
    return *p;
}

// The sum over the row's S blocks of at(o), a load of block o's value, in block order (the same in every block of the
// row), with eight loads in flight at a time.
template <class T, class F>
__device__ __forceinline__ T sum_blocks(int S, F&& at) {
    T acc = 0;
    for (int o0 = 0; o0 < S; o0 += 8) {
        T v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = o0 + j < S ? at(o0 + j) : T(0);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += v[j];
    }
    return acc;
}

// A buffer resource over [base, base + bytes). Both are the same on every lane (a row's), made visibly uniform so that
// the loads take the resource from scalar registers without a loop over lanes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t full_rsrc(const void* base, u32 bytes) {
    const u64 a = (u64)(uintptr_t)base;
    const u64 ua = ((u64)(u32)__builtin_amdgcn_readfirstlane((int)(u32)(a >> 32)) << 32) |
                   (u64)(u32)__builtin_amdgcn_readfirstlane((int)(u32)a);
    const int ub = __builtin_amdgcn_readfirstlane((int)bytes);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)ua, (short)0, ub, 0x00020000);
}

// Streams the row tile by tile (tile t: elements [t * TILE, (t + 1) * TILE), thread tid the group at t * TILE + 4 tid),
// calling f(t, e, l) with the group's penalised, masked logits; every thread calls f for every tile, so f may hold
// block barriers. Rows that allow 16-byte loads keep the loads of DEPTH tiles in flight.
#ifndef GBS_FULL_DEPTH
#define GBS_FULL_DEPTH 2  // tiles in flight per thread (config 3: 1 -> 115.7 us, 2 -> 116.8, 3 -> 119, 4 -> 120.9)
#endif
constexpr int DEPTH = GBS_FULL_DEPTH;
template <int DT, bool COUNTS, bool MASK, class F>
__device__ __forceinline__ void stream_tiles(const Row<DT, COUNTS, MASK>& R, int t0, int t1, F&& f) {
    const int tid = threadIdx.x;
    if (!R.vec || R.vocab % 4 != 0) {  // the buffer loads below read whole 4-element groups
        for (int t = t0; t < t1; ++t) {
            const int e = t * TILE + tid * 4;
            float l[4];
            R.group(e, l);
            f(t, e, l);
        }
        return;
    }
    const u32 esz = DT == GBS_DTYPE_F32 ? 4u : 2u;
    const __amdgpu_buffer_rsrc_t rx = full_rsrc(R.x, (u32)R.vocab * esz);
    const __amdgpu_buffer_rsrc_t rc = full_rsrc(R.c, COUNTS ? (u32)R.vocab * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rm = full_rsrc(R.m, MASK ? (u32)((R.vocab + 31) / 32) * 4u : 0u);
    typename Row<DT, COUNTS, MASK>::Raw buf[DEPTH];
#pragma unroll
    for (int k = 0; k < DEPTH; ++k)
        if (t0 + k < t1) R.load_raw((t0 + k) * TILE + tid * 4, rx, rc, rm, buf[k]);
    for (int tb = t0; tb < t1; tb += DEPTH) {
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) {
            const int t = tb + k;
            if (t < t1) {
                const int e = t * TILE + tid * 4;
                float l[4];
                R.from_raw(buf[k], e, l);
                if (t + DEPTH < t1) R.load_raw(e + DEPTH * TILE, rx, rc, rm, buf[k]);
                f(t, e, l);
            }
        }
    }
}

// Streams tiles [t0, t1) in wave-steps: step k covers elements [t0 * TILE + k * WS, + WS), WS = G * 256; wave w takes
// step w, then the next unclaimed one (lane l's group j at + j * 256 + 4 l); the next step's G groups per lane are in
// flight while a step is processed. The loads are issued whether or not their step exists (a step past the block's
// last reads at an offset past the row's end, which the buffer range check turns into zeros without a memory access),
// so every wait counts exactly the loads issued after the buffer it needs. f(t, e, l) is called per group and
// fe(t, q) once per step (q: the step's place in its tile, below TILE / WS); f and fe must not hold block barriers.
// pre() is called by every thread once the first step's loads are in flight, before any group is processed (it may
// hold block barriers); when it returns false (the same in every thread) nothing is processed.
#ifndef GBS_FS_STEPS
#define GBS_FS_STEPS 1
#endif
#ifndef GBS_FS_AUX0
#define GBS_FS_AUX0 2
#endif
#ifndef GBS_FS_AUXH
#define GBS_FS_AUXH 2
#endif
#ifndef GBS_FS_AUXC
#define GBS_FS_AUXC 2
#endif
#ifndef GBS_FS_STEP_GROUPS
#define GBS_FS_STEP_GROUPS 2
#endif
constexpr int SG = GBS_FS_STEP_GROUPS;
constexpr int STEPS_PER_TILE_MAX = NWF;  // TILE / 256: the steps of one group per lane
template <int G, int AUX, int DT, bool COUNTS, bool MASK, class F, class FE, class FP>
__device__ __forceinline__ void stream_steps(const Row<DT, COUNTS, MASK>& R, int t0, int t1, F&& f, FE&& fe, FP&& pre) {
    static_assert(TILE % (G * 256) == 0, "whole steps per tile");
    constexpr int WS = G * 256, SPT = TILE / WS;
    const int w = (int)threadIdx.x / WAVE, l = lane_id();
    if (!R.vec || R.vocab % 4 != 0) {  // one group per lane and step: wave w takes elements [w * 256, + 256) of each tile
        if (!pre()) return;
        for (int t = t0; t < t1; ++t) {
            const int e = t * TILE + (int)threadIdx.x * 4;
            float lv[4];
            R.group(e, lv);
            f(t, e, lv);
            fe(t, w);
        }
        return;
    }
    const u32 esz = DT == GBS_DTYPE_F32 ? 4u : 2u;
    const __amdgpu_buffer_rsrc_t rx = full_rsrc(R.x, (u32)R.vocab * esz);
    const __amdgpu_buffer_rsrc_t rc = full_rsrc(R.c, COUNTS ? (u32)R.vocab * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rm = full_rsrc(R.m, MASK ? (u32)((R.vocab + 31) / 32) * 4u : 0u);
    using Raw = typename Row<DT, COUNTS, MASK>::Raw;
    const int nsteps = (t1 - t0) * SPT;
    const int base = t0 * TILE + l * 4;
    constexpr int PAST = 1 << 29;  // an element index whose offsets lie past any row (rows hold at most 2^25 elements)
    auto load = [&](int k, Raw (&b)[G]) {
        const int e0 = k < nsteps ? base + k * WS : PAST;
#pragma unroll
        for (int j = 0; j < G; ++j) R.template load_raw<AUX>(e0 + j * 256, rx, rc, rm, b[j]);
    };
    auto use = [&](int k, const Raw (&b)[G]) {
        const int e0 = base + k * WS;
        const int t = t0 + k / SPT;
#pragma unroll
        for (int j = 0; j < G; ++j) {
            float lv[4];
            R.from_raw(b[j], e0 + j * 256, lv);
            f(t, e0 + j * 256, lv);
        }
        fe(t, k % SPT);
    };
    // one load site: the step's buffer is copied out once it has arrived, and the next step's loads go into it before
    // the copy is used. Wave w's first step is w. With four steps per wave or more, later steps go to whichever wave
    // asks first (an LDS counter), so that waves the memory system serves late do not hold the block (config 3: 82.3 ->
    // 79.4 us); with fewer, wave w takes w + NWF, w + 2 NWF, ... (the counter's barrier and round trips cost more than
    // they balance).
    const bool dyn = nsteps >= 4 * NWF;
    __shared__ int s_next;
    if (threadIdx.x == 0) s_next = NWF;
    Raw B[G];
    int k = w;
    load(k, B);
    if (!pre()) return;
    if (dyn) __syncthreads();  // the counter is set
    while (k < nsteps) {
        Raw C[G];
#pragma unroll
        for (int j = 0; j < G; ++j) C[j] = B[j];
        int kn = k + NWF;
        if (dyn) {
            if (l == 0) kn = atomicAdd(&s_next, 1);
            kn = __builtin_amdgcn_readfirstlane(kn);
        }
        load(kn, B);
        use(k, C);
        k = kn;
    }
}

template <int G, int AUX, int DT, bool COUNTS, bool MASK, class F, class FE>
__device__ __forceinline__ void stream_steps(const Row<DT, COUNTS, MASK>& R, int t0, int t1, F&& f, FE&& fe) {
    stream_steps<G, AUX>(R, t0, t1, f, fe, [] { return true; });
}

// the whole row
template <int DT, bool COUNTS, bool MASK, class F>
__device__ __forceinline__ void stream_tiles(const Row<DT, COUNTS, MASK>& R, F&& f) {
    stream_tiles(R, 0, (R.vocab + TILE - 1) / TILE, f);
}

__device__ __forceinline__ u32 wave_sum_u32(u32 v) {
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) v += xor_lane(v, m);
    return v;
}

// block totals over all threads (cross-lane moves by DPP and permlane swaps, one LDS slot per wave); every thread
// of the block calls them and receives the total
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* s_red) {
    const int w = threadIdx.x / WAVE;
    if constexpr (sizeof(T) == 8) v = (T)wave_sum_u64((u64)v);
    else v = (T)wave_sum_u32((u32)v);
    __syncthreads();
    if (lane_id() == 0) s_red[w] = v;
    __syncthreads();
    T r = 0;
    for (int o = 0; o < NWF; ++o) r += s_red[o];
    __syncthreads();
    return r;
}

__device__ __forceinline__ u64 block_max_u64(u64 v, u64* s_red) {
    const int w = threadIdx.x / WAVE;
    v = wave_max_u64(v);
    __syncthreads();
    if (lane_id() == 0) s_red[w] = v;
    __syncthreads();
    u64 r = 0;
    for (int o = 0; o < NWF; ++o) r = s_red[o] > r ? s_red[o] : r;
    __syncthreads();
    return r;
}

// The binned cut: 128 bins per unit of y = log2 of the mass relative to the maximum, down to y = -52 (below -51.5 every
// mass is 0; the last bin takes them).
constexpr int BINS_PER_UNIT = 128;
constexpr int NUNITS = 52;
constexpr int NBINS = NUNITS * BINS_PER_UNIT;
constexpr int CAP = NB;  // collected tokens of the crossing bin (keys in sh.maxk, masses in sh.mass)

// the bin of a token: min(floor(-128 y), NBINS - 1), y = (l - M) * c2 computed as the mass is
__device__ __forceinline__ u32 bin_of(float l, float M, float c2) {
    const float y = (l - M) * c2;
    return (u32)fminf(-y * (float)BINS_PER_UNIT, (float)(NBINS - 1));
}

struct Shared {
    u32 cnt[NB];
    u64 mass[NBINS];  // the radix digits' masses (NB), or the binned cut's mass per bin (NBINS)
    u64 maxk[NB];
    u64 red[NWF];
    u64 tile[MAX_TILES];
    u64 tilew[MAX_TILES][NWF];  // per-wave partial sums of a tile (no barrier per tile)
    float lse_m[NWF], lse_s[NWF];
    u64 bc[8];  // broadcast slots
    u32 ncol;   // tokens collected by the binned cut
};

static_assert(NBINS == (int)FS_NBINS, "the per-row record's bin count");

// The exact top-p key among the n tokens collected from the bins [r_lo, r_hi] of bin_of() (keys and masses in LDS):
// the one key K with above + G(K) < P <= above + G(K) + E(K), G(K) the mass of the collected keys larger than K (the
// bins hold the target: above < P <= above + their mass). They are split into NSUB sub-bins by the same y as the bins
// (sub = floor(NSUB (-128 y - r_lo) / (r_hi - r_lo + 1)), clamped; it never decreases as the value decreases, and
// equal values share it); a mass histogram of the sub-bins gives the one holding the target, and only its tokens are
// compared with each other. Every thread calls it; it returns the key on every thread. LDS: s_cnt holds the sub-bins' masses, then
// the list of the crossing sub-bin's tokens.
constexpr int NSUB = 256;
constexpr u32 SUB_LIST_CAP = NB - 2 * NSUB;  // u32 slots of s_cnt after the sub-bins' masses
__device__ u64 cut_collected(const u64* keys, const u64* masses, u32 n, u64 above, u64 P, float M, float c2, int r_lo, int r_hi,
                             u32* s_cnt, u64* s_bc) {
    const int tid = threadIdx.x, l = lane_id();
    u64* const s_sub = (u64*)s_cnt;
    u32* const s_list = s_cnt + 2 * NSUB;
    const float scale = (float)NSUB / (float)(r_hi - r_lo + 1);
    auto sub_of = [&](u64 key) {
        const float y = (okey_to_f32(key_ok(key)) - M) * c2;
        return (u32)fminf(fmaxf((-y * (float)BINS_PER_UNIT - (float)r_lo) * scale, 0.0f), (float)(NSUB - 1));
    };
    for (int i = tid; i < NSUB; i += NTF) s_sub[i] = 0;
    if (tid == 0) {
        s_bc[2] = 0;                        // tokens of the crossing sub-bin
        s_bc[3] = (u64)VALID_MIN_OK << 32;  // the cut, if none were found (cannot happen)
    }
    __syncthreads();
    for (u32 i = tid; i < n; i += NTF) atomicAdd((unsigned long long*)&s_sub[sub_of(keys[i])], (unsigned long long)masses[i]);
    __syncthreads();
    if (tid < WAVE) {
        // lane i holds sub-bins 4i .. 4i + 3
        u64 m4[4], tot = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            m4[q] = s_sub[4 * l + q];
            tot += m4[q];
        }
        const u64 incl = above + wave_scan_u64(tot);
        const int f = (int)__builtin_ctzll(ballot(incl >= P) | (1ull << 63));
        if (l == f) {
            u64 acc = incl - tot;
            int q = 0;
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                if (q == k && acc + m4[k] < P) {
                    acc += m4[k];
                    q = k + 1;
                }
            }
            s_bc[0] = (u64)(4 * f + q);
            s_bc[1] = acc;  // the mass above the crossing sub-bin
        }
    }
    __syncthreads();
    const u32 sstar = (u32)s_bc[0];
    for (u32 i = tid; i < n; i += NTF) {
        if (sub_of(keys[i]) == sstar) {
            const u32 k = atomicAdd((unsigned*)&s_bc[2], 1u);
            if (k < SUB_LIST_CAP) s_list[k] = i;
        }
    }
    __syncthreads();
    const u32 m = (u32)s_bc[2];
    const u64 base = s_bc[1];
    if (m <= SUB_LIST_CAP) {
        for (u32 t = tid; t < m; t += NTF) {
            const u32 i = s_list[t];
            const u64 ki = keys[i];
            u64 g = 0;
            for (u32 u = 0; u < m; ++u) {
                const u32 j = s_list[u];
                g += keys[j] > ki ? masses[j] : 0ull;
            }
            if (base + g < P && P <= base + g + masses[i]) s_bc[3] = ki;
        }
    } else {  // more tokens in one sub-bin than the list holds (equal values): compare them over the whole collection
        for (u32 i = tid; i < n; i += NTF) {
            const u64 ki = keys[i];
            if (sub_of(ki) != sstar) continue;
            u64 g = 0;
            for (u32 j = 0; j < n; ++j) g += (keys[j] > ki && sub_of(keys[j]) == sstar) ? masses[j] : 0ull;
            if (base + g < P && P <= base + g + masses[i]) s_bc[3] = ki;
        }
    }
    __syncthreads();
    const u64 kp = s_bc[3];
    __syncthreads();
    return kp;
}

// The same cut on one wave (the other waves of the block take no part): the sub-bins' histogram by LDS atomics, the
// crossing sub-bin by a wave scan, its tokens compacted by ballots, and the comparison among them. Returns the key in
// every lane. LDS as cut_collected.
__device__ u64 cut_collected_wave(const u64* keys, const u64* masses, u32 n, u64 above, u64 P, float M, float c2, int r_lo,
                                  int r_hi, u32* s_cnt) {
    const int l = lane_id();
    u64* const s_sub = (u64*)s_cnt;
    u32* const s_list = s_cnt + 2 * NSUB;
    const float scale = (float)NSUB / (float)(r_hi - r_lo + 1);
    auto sub_of = [&](u64 key) {
        const float y = (okey_to_f32(key_ok(key)) - M) * c2;
        return (u32)fminf(fmaxf((-y * (float)BINS_PER_UNIT - (float)r_lo) * scale, 0.0f), (float)(NSUB - 1));
    };
#pragma unroll
    for (int q = 0; q < NSUB / WAVE; ++q) s_sub[q * WAVE + l] = 0;
    for (u32 i = l; i < n; i += WAVE) atomicAdd((unsigned long long*)&s_sub[sub_of(keys[i])], (unsigned long long)masses[i]);
    // lane i holds sub-bins 4i .. 4i + 3
    u64 m4[4], tot = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        m4[q] = s_sub[4 * l + q];
        tot += m4[q];
    }
    const u64 incl = above + wave_scan_u64(tot);
    const int f = (int)__builtin_ctzll(ballot(incl >= P) | (1ull << 63));
    u64 acc = incl - tot;
    int q0 = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (q0 == k && acc + m4[k] < P) {
            acc += m4[k];
            q0 = k + 1;
        }
    }
    const u32 sstar = (u32)__builtin_amdgcn_readlane(4 * l + q0, f);
    const u64 base = readlane64(acc, f);  // the mass above the crossing sub-bin
    // its tokens, in order of the collection
    u32 m = 0;
    for (u32 i0 = 0; i0 < n; i0 += WAVE) {
        const u32 i = i0 + (u32)l;
        const bool in = i < n && sub_of(keys[i]) == sstar;
        const u64 mk = ballot(in);
        const u32 idx = m + mbcnt(mk);
        if (in && idx < SUB_LIST_CAP) s_list[idx] = i;
        m += (u32)__popcll(mk);
    }
    u64 kp = (u64)VALID_MIN_OK << 32;  // if none were found (cannot happen)
    if (m <= SUB_LIST_CAP) {
        for (u32 t0 = 0; t0 < m; t0 += WAVE) {
            const u32 t = t0 + (u32)l;
            bool hit = false;
            u64 ki = 0;
            if (t < m) {
                const u32 i = s_list[t];
                ki = keys[i];
                u64 g = 0;
                for (u32 v = 0; v < m; ++v) {
                    const u32 j = s_list[v];
                    g += keys[j] > ki ? masses[j] : 0ull;
                }
                hit = base + g < P && P <= base + g + masses[i];
            }
            const u64 hb = ballot(hit);
            if (hb) kp = readlane64(ki, (int)__builtin_ctzll(hb));
        }
    } else {  // more tokens in one sub-bin than the list holds (equal values): compare them over the whole collection
        for (u32 i0 = 0; i0 < n; i0 += WAVE) {
            const u32 i = i0 + (u32)l;
            bool hit = false;
            u64 ki = 0;
            if (i < n && sub_of(keys[i]) == sstar) {
                ki = keys[i];
                u64 g = 0;
                for (u32 j = 0; j < n; ++j) g += (keys[j] > ki && sub_of(keys[j]) == sstar) ? masses[j] : 0ull;
                hit = base + g < P && P <= base + g + masses[i];
            }
            const u64 hb = ballot(hit);
            if (hb) kp = readlane64(ki, (int)__builtin_ctzll(hb));
        }
    }
    return kp;
}

// Adds the kept collected tokens (key >= kp, mass >= Q) to their tiles' masses, on one wave. Collected tokens come in
// runs of one tile (each wave of the collection appends in ascending element order), so the wave sums its 64 tokens
// per run of equal tiles (a prefix sum over the lanes) and only a run's last lane adds to LDS: lanes do not contend for
// one tile's address.
// nw waves take part, this one as wave wi (chunks of 64 tokens wi, wi + nw, ...).
__device__ __forceinline__ void add_kept_to_tiles_wave(const u64* keys, const u64* masses, u32 n, u64 kp, u64 Q, u64* s_tile, int wi = 0,
                                                       int nw = 1) {
    const int l = lane_id();
    for (u32 j0 = (u32)wi * WAVE; j0 < n; j0 += (u32)nw * WAVE) {
        const u32 j = j0 + (u32)l;
        const bool in = j < n;
        const u64 k = in ? keys[j] : 0ull, E = in ? masses[j] : 0ull;
        const u64 v = in && k >= kp && E >= Q ? E : 0ull;
        const int t = in ? (int)(key_id(k) / TILE) : -1;
        const int tn = __shfl_down(t, 1, WAVE), tp = __shfl_up(t, 1, WAVE);
        const bool last = in && (l == WAVE - 1 || tn != t);
        const u64 starts = ballot(in && (l == 0 || tp != t));
        const u64 incl = wave_scan_u64(v);
        // the run's first lane s: the highest start at or below this lane; the run's sum is incl(l) - incl(s - 1)
        const u64 below = starts & (l == WAVE - 1 ? ~0ull : ((2ull << l) - 1ull));
        const int st = below ? 63 - __builtin_clzll(below) : 0;
        const u64 before = shfl64(incl, st > 0 ? st - 1 : 0);
        const u64 run = incl - (st > 0 ? before : 0ull);
        if (last && run) atomicAdd((unsigned long long*)&s_tile[t], (unsigned long long)run);
    }
}


// One radix selection over the keys >= lb of the row: the key K at which the descending cumulative weight (count when
// by_mass is false, mass otherwise) first reaches `target` -- weight(keys > K) < target <= weight(keys >= K).
// With frac_p > 0 the target is ceil(frac_p * total weight), the total being the first pass's sum.
// *mass_above receives the mass of the keys > K.
template <int DT, bool COUNTS, bool MASK>
__device__ u64 radix_select(const Row<DT, COUNTS, MASK>& R, float M, float c2, u64 lb, bool by_mass, u64 target, float frac_p,
                            u64* mass_above, u64* total_out, Shared& sh) {
    u64 prefix = 0;
    int plen = 0;
    u64 above = 0;
    for (;;) {
        const int db = 64 - plen < DB ? 64 - plen : DB;
        for (int i = threadIdx.x; i < NB; i += NTF) {
            sh.cnt[i] = 0;
            sh.mass[i] = 0;
            sh.maxk[i] = 0;
        }
        __syncthreads();
        const u64 pmask = plen == 0 ? 0ull : (~0ull << (64 - plen));
        for (int base = 0; base < R.vocab; base += TILE) {
            const int e = base + (int)threadIdx.x * 4;
            float l[4];
            R.group(e, l);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (!valid_l(l[q])) continue;
                const u64 key = make_key(okey_f32(l[q]), (u32)(e + q));
                if (key < lb || (key & pmask) != prefix) continue;
                const int d = (int)((key >> (64 - plen - db)) & ((1ull << db) - 1ull));
                atomicAdd(&sh.cnt[d], 1u);
                atomicAdd((unsigned long long*)&sh.mass[d], (unsigned long long)mass(l[q], M, c2));
                atomicMax((unsigned long long*)&sh.maxk[d], (unsigned long long)key);
            }
        }
        __syncthreads();
        // wave 0 finds the crossing digit, scanning digits from the largest down: lane i owns 32 digits
        if (threadIdx.x < WAVE) {
            const int l = lane_id();
            constexpr int PER = NB / WAVE;
            const int nd = 1 << db;
            u64 wsum = 0, msum = 0;
            for (int k = 0; k < PER; ++k) {
                const int d = nd - 1 - (l * PER + k);
                if (d >= 0) {
                    wsum += by_mass ? sh.mass[d] : (u64)sh.cnt[d];
                    msum += sh.mass[d];
                }
            }
            if (plen == 0 && frac_p > 0.0f) {
                const u64 tot = wave_sum_u64(wsum);
                if (total_out) *total_out = tot;
                target = mul_ceil64(frac_p, tot);
            }
            const u64 incl = wave_scan_u64(wsum);
            const u64 excl = incl - wsum;
            const u64 mincl = wave_scan_u64(msum);
            const u64 mexcl = mincl - msum;
            const u64 hit = ballot(incl >= target);
            const int f = hit ? (int)__builtin_ctzll(hit) : WAVE - 1;
            if (l == f) {
                u64 acc = excl, macc = mexcl;
                int dstar = 0;
                for (int k = 0; k < PER; ++k) {
                    const int d = nd - 1 - (l * PER + k);
                    if (d < 0) break;
                    const u64 w = by_mass ? sh.mass[d] : (u64)sh.cnt[d];
                    dstar = d;
                    if (acc + w >= target) break;
                    acc += w;
                    macc += sh.mass[d];
                }
                sh.bc[0] = (u64)dstar;
                sh.bc[1] = target - acc;
                sh.bc[2] = macc;
                sh.bc[3] = sh.cnt[dstar];
                sh.bc[4] = sh.maxk[dstar];
            }
        }
        __syncthreads();
        const int dstar = (int)sh.bc[0];
        target = sh.bc[1];
        above += sh.bc[2];
        const u64 cstar = sh.bc[3], kmax = sh.bc[4];
        __syncthreads();
        prefix |= (u64)dstar << (64 - plen - db);
        plen += db;
        if (cstar <= 1 || plen >= 64) {
            if (mass_above) *mass_above = above;
            return cstar == 1 ? kmax : prefix;
        }
    }
}

// ---- the binned cut (no top-k, finite maximum and 1/T): top-p and min-p in two reads of the row.
// Tokens are binned by y = (l - M) * c2 (log2 of the mass relative to the maximum, computed exactly as the mass is):
// bin = min(floor(-32 y), NBINS - 1), which never increases along the (value desc, id asc) order. Read 1 sums the
// masses per bin; the crossing bin b* is the first bin (from the top) where the cumulative mass reaches
// P = ceil(top_p * Z). Read 2 adds the kept masses of the bins above b* (mass >= Q, the min-p floor) per 4096-element
// tile and collects the keys and masses of bin b*; sorting the collected keys gives the exact top-p key (the first
// whose cumulative mass reaches P), and the kept ones of them are added to their tiles. Returns false (nothing kept
// of its state) when bin b* holds more than CAP tokens: the caller takes the radix path.

template <int DT, bool COUNTS, bool MASK>
__device__ bool binned_cut(const Row<DT, COUNTS, MASK>& R, float M, float c2, float top_p, u64 Q, u64* kp_out, Shared& sh) {
    const int tid = threadIdx.x, w = tid / WAVE, l = lane_id();
    const int ntiles = (R.vocab + TILE - 1) / TILE;
    const bool topp = top_p > 0.0f && top_p < 1.0f;
    u32 bstar = NBINS;  // no top-p: every bin is above the cut
    u64 above = 0, P = 0;
    if (topp) {
        for (int i = tid; i < NBINS; i += NTF) sh.mass[i] = 0;
        __syncthreads();
        stream_tiles(R, [&](int, int, const float (&lv)[4]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u64 E = mass_fast(lv[q], M, c2);
                if (E) atomicAdd((unsigned long long*)&sh.mass[bin_of(lv[q], M, c2)], (unsigned long long)E);
            }
        });
        __syncthreads();
        if (tid < WAVE) {
            // lane i owns bins [32 i, 32 i + 32): the total, P, then the bin where the cumulative mass reaches P
            constexpr int PB = NBINS / WAVE;
            u64 s = 0;
            for (int k = 0; k < PB; ++k) s += sh.mass[l * PB + k];
            const u64 Z = wave_sum_u64(s);
            const u64 Pv = mul_ceil64(top_p, Z);
            const u64 incl = wave_scan_u64(s);
            const u64 hit = ballot(incl >= Pv);
            const int f = (int)__builtin_ctzll(hit);  // P <= Z: some lane reaches it
            if (l == f) {
                u64 acc = incl - s;
                int b = l * PB;
                for (int k = 0; k < PB; ++k) {
                    b = l * PB + k;
                    if (acc + sh.mass[b] >= Pv) break;
                    acc += sh.mass[b];
                }
                sh.bc[0] = (u64)b;
                sh.bc[1] = acc;
                sh.bc[2] = Pv;
            }
        }
        __syncthreads();
        bstar = (u32)sh.bc[0];
        above = sh.bc[1];
        P = sh.bc[2];
    }
    // read 2: kept masses of the bins above b* per tile; the tokens of bin b* into (sh.maxk, sh.mass)
    if (tid == 0) sh.ncol = 0;
    __syncthreads();
    stream_tiles(R, [&](int t, int e, const float (&lv)[4]) {
        u64 s = 0;
        u64 Eq[4];
        bool col[4];
        int ncol = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            Eq[q] = mass_fast(lv[q], M, c2);
            const u32 b = topp ? bin_of(lv[q], M, c2) : 0u;
            const bool ok = valid_l(lv[q]);
            if (ok && b < bstar && Eq[q] >= Q) s += Eq[q];
            col[q] = ok && b == bstar;
            ncol += col[q] ? 1 : 0;
        }
        // the group's tokens of bin b*: one LDS append per wave (an exclusive scan of the lanes' counts)
        if (ballot(ncol > 0)) {
            const u64 inc = wave_scan_u64((u64)ncol);
            u32 base = 0;
            if (l == WAVE - 1) base = atomicAdd(&sh.ncol, (u32)inc);
            base = (u32)__builtin_amdgcn_readlane((int)base, WAVE - 1);
            u32 idx = base + (u32)(inc - (u64)ncol);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (col[q]) {
                    if (idx < (u32)CAP) {
                        sh.maxk[idx] = make_key(okey_f32(lv[q]), (u32)(e + q));
                        sh.mass[idx] = Eq[q];
                    }
                    ++idx;
                }
            }
        }
        s = wave_sum_u64(s);
        if (l == 0) sh.tilew[t][w] = s;
    });
    __syncthreads();
    for (int t = tid; t < ntiles; t += NTF) {
        u64 v = 0;
#pragma unroll
        for (int k = 0; k < NWF; ++k) v += sh.tilew[t][k];
        sh.tile[t] = v;
    }
    __syncthreads();
    const u32 n = sh.ncol;
    if (n > (u32)CAP) return false;
    u64 kp = (u64)VALID_MIN_OK << 32;  // every valid key
    if (topp) {
        // the top-p key among the collected tokens of bin b*
        kp = cut_collected(sh.maxk, sh.mass, n, above, P, M, c2, (int)bstar, (int)bstar, sh.cnt, sh.bc);
        // the kept tokens of bin b* (key >= the top-p key, mass >= Q) into their tiles
        for (u32 j = tid; j < n; j += NTF) {
            const u64 E = sh.mass[j];
            if (sh.maxk[j] >= kp && E >= Q) atomicAdd((unsigned long long*)&sh.tile[key_id(sh.maxk[j]) / TILE], (unsigned long long)E);
        }
        __syncthreads();
    }
    *kp_out = kp;
    return true;
}

template <int DT, bool COUNTS, bool MASK>
__device__ __forceinline__ void full_row(const void* __restrict__ logits, long long stride, int vocab, const int* __restrict__ counts,
                                         const u32* __restrict__ mask, const RowParamsDev* __restrict__ params,
                                         const float* __restrict__ uniforms, bool vec, int* __restrict__ out_ids,
                                         int* __restrict__ out_greedy, float* __restrict__ out_probs, float* __restrict__ out_logprobs,
                                         int* __restrict__ out_status, int r, Shared& sh) {
    const int tid = threadIdx.x, w = tid / WAVE, l = lane_id();
    const RowParamsDev p = params[r];
    const float u = uniforms[r];
    Row<DT, COUNTS, MASK> R;
    R.x = (const char*)logits + (size_t)r * (size_t)stride * (DT == GBS_DTYPE_F32 ? 4 : 2);
    R.c = COUNTS ? counts + (size_t)r * vocab : nullptr;
    R.m = MASK ? mask + (size_t)r * ((vocab + 31) / 32) : nullptr;
    R.vocab = vocab;
    R.vec = vec;
    R.rinv = 1.0f / p.repetition;
    R.rep = p.repetition;
    R.freq = p.frequency;
    R.pres = p.presence;
    const float clp = p.temperature > 0.0f ? temp_scale(p.temperature) : 1.44269504088896340736f;

    auto finish = [&](int id, int greedy, int status, float prob, float lp) {
        if (tid == 0) {
            out_ids[r] = status == GBS_ROW_OK ? id : -1;
            if (out_greedy) out_greedy[r] = status == GBS_ROW_OK ? greedy : -1;
            if (out_probs) out_probs[r] = status == GBS_ROW_OK ? prob : 0.f;
            if (out_logprobs) out_logprobs[r] = status == GBS_ROW_OK ? lp : __uint_as_float(0x7fc00000u);
            if (out_status) out_status[r] = status;
        }
    };
    if (params_invalid(p, u)) {
        finish(-1, -1, GBS_ROW_INVALID_PARAMS, 0.f, 0.f);
        return;
    }

    // ---- pass 0: maximum, NaN, allowed count, log-sum-exp
    Pass0Acc acc;
    stream_tiles(R, [&](int, int e, const float (&lv)[4]) { acc.add(lv, e, clp); });
    const u64 kmaxv = acc.key();
    const u32 nan = acc.nan, nallowed = acc.nallowed;
    const Lse lse = wave_lse(acc.lse, clp);
    if (l == 0) {
        sh.lse_m[w] = lse.m;
        sh.lse_s[w] = lse.s;
    }
    const u32 nan_any = (u32)block_sum((u64)nan, sh.red);
    const u64 n_allowed = block_sum((u64)nallowed, sh.red);
    const u64 top = block_max_u64(kmaxv, sh.red);
    Lse rl{-INFINITY, 0.f};
    for (int o = 0; o < NWF; ++o) rl = lse_merge(rl, Lse{sh.lse_m[o], sh.lse_s[o]}, clp);
    if (nan_any) {
        finish(-1, -1, GBS_ROW_NAN_LOGIT, 0.f, 0.f);
        return;
    }
    if (n_allowed == 0) {
        finish(-1, -1, GBS_ROW_NO_CANDIDATES, 0.f, 0.f);
        return;
    }
    const int greedy = (int)key_id(top);
    const float M = okey_to_f32(key_ok(top));
    auto logprob_of = [&](float lx) {
        if (isinf(M) || !isfinite(clp)) return __uint_as_float(0x7fc00000u);  // undefined: +inf maximum, 1/T beyond f32
        return ((lx - rl.m) * clp - log2f(rl.s)) * 0.6931471805599453f;
    };
    if (p.temperature == 0.0f) {
        finish(greedy, greedy, GBS_ROW_OK, 1.0f, logprob_of(M));
        return;
    }
    const float c2 = temp_scale(p.temperature);

    const u64 Q = p.min_p > 0.0f ? mul_ceil64(p.min_p, MASS_ONE) : 0ull;
    const int ntiles = (vocab + TILE - 1) / TILE;
    const bool topk_on = p.top_k > 0 && (u64)p.top_k < n_allowed;
    u64 kp = 0;
    // the binned cut fills the tiles' kept masses itself
    const bool binned = !topk_on && mass_fast_ok(M, c2) && binned_cut(R, M, c2, p.top_p, Q, &kp, sh);
    if (!binned) {
    // ---- top-k
    const u64 floor_key = (u64)VALID_MIN_OK << 32;
    u64 lb = floor_key;
    u64 zk = 0;
    bool have_zk = false;
    if (topk_on) {
        u64 above = 0;
        const u64 kk = radix_select(R, M, c2, floor_key, false, (u64)p.top_k, 0.0f, &above, nullptr, sh);
        lb = kk;
        zk = above + mass(okey_to_f32(key_ok(kk)), M, c2);
        have_zk = true;
    }
    // ---- top-p
    kp = lb;
    if (p.top_p > 0.0f && p.top_p < 1.0f) {
        u64 tot = 0;
        if (have_zk) kp = radix_select(R, M, c2, lb, true, mul_ceil64(p.top_p, zk), 0.0f, nullptr, nullptr, sh);
        else kp = radix_select(R, M, c2, lb, true, 0, p.top_p, nullptr, &tot, sh);
    }
    }
    // ---- draw: kept = key >= kp and mass >= Q, in ascending id order
    auto kept_mass = [&](float v, int i) -> u64 {
        if (!valid_l(v)) return 0ull;
        if (make_key(okey_f32(v), (u32)i) < kp) return 0ull;
        const u64 E = mass(v, M, c2);
        return E >= Q ? E : 0ull;
    };
    if (!binned) {
        stream_tiles(R, [&](int t, int e, const float (&lv)[4]) {
            u64 s = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) s += kept_mass(lv[q], e + q);
            s = block_sum(s, sh.red);
            if (tid == 0) sh.tile[t] = s;
        });
    }
    __syncthreads();
    u64 z = 0;
    for (int t = 0; t < ntiles; ++t) z += sh.tile[t];
    const u64 target = (u64)mul_floor(u, (u128)z, nullptr);
    int tsel = ntiles - 1;
    u64 before = 0;
    for (int t = 0; t < ntiles; ++t) {
        if (before + sh.tile[t] > target) {
            tsel = t;
            break;
        }
        before += sh.tile[t];
    }
    // the tile: thread sums, a block exclusive scan, the owning thread scans its 4 elements
    const int e = tsel * TILE + tid * 4;
    float lv[4];
    R.group(e, lv);
    u64 em[4], mine = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        em[q] = kept_mass(lv[q], e + q);
        mine += em[q];
    }
    const u64 incl = wave_scan_u64(mine);
    __syncthreads();
    if (l == WAVE - 1) sh.red[w] = incl;
    __syncthreads();
    u64 wbase = before;
    for (int o = 0; o < w; ++o) wbase += sh.red[o];
    const u64 excl = wbase + incl - mine;
    if (excl <= target && target < excl + mine) {
        // the first of the thread's four elements whose running mass exceeds the target (selections, no indexing)
        u64 acc = excl, ef = 0;
        int qf = -1;
        float lf = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc += em[q];
            const bool hit = qf < 0 && acc > target;
            qf = hit ? q : qf;
            ef = hit ? em[q] : ef;
            lf = hit ? lv[q] : lf;
        }
        sh.bc[5] = (u64)(e + qf);
        sh.bc[6] = ef;
        sh.bc[7] = __float_as_uint(lf);
    }
    __syncthreads();
    const int id = (int)sh.bc[5];
    const u64 ec = sh.bc[6];
    const float lx = __uint_as_float((u32)sh.bc[7]);
    finish(id, greedy, GBS_ROW_OK, (float)((double)ec / (double)z), logprob_of(lx));
}

// One block of NTF threads per row: the whole row in one block (batches of at least as many rows as CUs).
template <int DT, bool COUNTS, bool MASK>
__global__ void __launch_bounds__(NTF) sample_full_k(const void* __restrict__ logits, long long stride, int vocab,
                                                     const int* __restrict__ counts, const u32* __restrict__ mask,
                                                     const RowParamsDev* __restrict__ params, const float* __restrict__ uniforms, bool vec,
                                                     int* __restrict__ out_ids, int* __restrict__ out_greedy, float* __restrict__ out_probs,
                                                     float* __restrict__ out_logprobs, int* __restrict__ out_status,
                                                     const unsigned* __restrict__ flags) {
    __shared__ Shared sh;
    if (flags && flags[blockIdx.x] == 0u) return;
    full_row<DT, COUNTS, MASK>(logits, stride, vocab, counts, mask, params, uniforms, vec, out_ids, out_greedy, out_probs, out_logprobs,
                               out_status, (int)blockIdx.x, sh);
}

// The rows the split path marked (top-k with a cut, an infinite maximum or 1/T, no collection window, a window that
// missed the cut or held more than CAP tokens, flagged rows past the workspace's): one block each, the single-block
// path; the mark is cleared for the next launch.
template <int DT, bool COUNTS, bool MASK>
__global__ void __launch_bounds__(NTF) fs_fallback_k(const void* __restrict__ logits, long long stride, int vocab,
                                                     const int* __restrict__ counts, const u32* __restrict__ mask,
                                                     const RowParamsDev* __restrict__ params, const float* __restrict__ uniforms, bool vec,
                                                     int* __restrict__ out_ids, int* __restrict__ out_greedy, float* __restrict__ out_probs,
                                                     float* __restrict__ out_logprobs, int* __restrict__ out_status,
                                                     unsigned* __restrict__ marks) {
    __shared__ Shared sh;
    const int r = (int)blockIdx.x;
    if (marks[r] == 0u) return;
    full_row<DT, COUNTS, MASK>(logits, stride, vocab, counts, mask, params, uniforms, vec, out_ids, out_greedy, out_probs, out_logprobs,
                               out_status, r, sh);
    if (threadIdx.x == 0) marks[r] = 0u;
}

// ================================================================================================== the split path
// Batches with fewer rows than CUs: S blocks per row, block sp over whole tiles [sp * tpb, (sp + 1) * tpb). Three
// launches, each with a last-block hand-off per row (agent-scope stores and loads, an arrival counter):
//   fs_pass0_k    maximum, NaN flag, allowed count, LSE; the row's last block finishes every row that needs no cut (an
//                 invalid, NaN or empty row, T = 0) and marks the rows that need the radix path (top-k with a cut,
//                 an infinite maximum or 1/T). Not launched under per-row dispatch: the single-pass kernel has written
//                 the record of every row it flags.
//   fs_hist_k     the binned cut's mass histogram (rows with top-p); the last block sums the blocks' histograms and
//                 finds the crossing bin
//   fs_collect_k  kept masses per tile and the crossing bin's tokens; the last block finds the exact top-p key, the
//                 tile that holds the draw, and the token. A row marked for the radix path is taken by its first block
//                 (the single-block path, full_row), and so is a row whose crossing bin held more than CAP tokens, by its
//                 last block.
#ifndef GBS_FS_TARGET_BLOCKS
#define GBS_FS_TARGET_BLOCKS 256
#endif
constexpr int FS_TARGET_BLOCKS = GBS_FS_TARGET_BLOCKS;  // the split path's blocks (rows below the CU count)
#ifndef GBS_FS_DEFER_BLOCKS
#define GBS_FS_DEFER_BLOCKS 512
#endif
constexpr int FS_DEFER_BLOCKS = GBS_FS_DEFER_BLOCKS;  // the split path's blocks when it serves flagged rows (DEFER_ROWS)
constexpr int FS_MAX_SPLITS = 128;


struct FsPart0 {
    u64 key;
    u32 nan, nallowed;
    float m, s;
    int kgrid;  // the row's histogram grid top (pass 0; the same in every block of the row)
    u32 pad;
};

// The split path's workspace, carved from one base pointer (so that a kernel holds one pointer and three counts instead
// of a pointer per array): the control region (arrival counters, the per-row records), then per (row, block) partials.
constexpr size_t FS_CTL = SAMPLE_CTL_BYTES;  // the control region shared with the single-pass kernel

__host__ __device__ __forceinline__ size_t fs_align(size_t b) { return (b + 255) & ~(size_t)255; }

struct FsWs {
    char* base;
    int nrows, S, ntiles;

    __host__ __device__ size_t rs() const { return (size_t)nrows * S; }
    __host__ __device__ unsigned* cnt2() const { return (unsigned*)base + 2 * 65536; }  // per-row arrival counters
    // per-row marks of the rows the single-block path takes after the collection (zero between launches)
    __host__ __device__ unsigned* fallback() const { return (unsigned*)base + 65536; }
    __host__ __device__ FsRow* rec() const { return (FsRow*)(base + SAMPLE_FSROW_OFFSET); }  // [65536], indexed by row
    __host__ __device__ size_t o_p0() const { return FS_CTL; }
    __host__ __device__ size_t o_hist() const { return o_p0() + fs_align(rs() * sizeof(FsPart0)); }
    __host__ __device__ size_t o_units() const { return o_hist() + fs_align(rs() * NBINS * 8); }
    __host__ __device__ size_t o_ubound() const { return o_units() + fs_align(rs() * NUNITS * 8); }
    __host__ __device__ size_t o_zab() const { return o_ubound() + fs_align(rs() * NUNITS * sizeof(float2)); }
    __host__ __device__ size_t o_ckey() const { return o_zab() + fs_align(rs() * 4 * 8); }
    __host__ __device__ size_t o_cmass() const { return o_ckey() + fs_align(rs() * CAP * 8); }
    __host__ __device__ size_t o_ccount() const { return o_cmass() + fs_align(rs() * CAP * 8); }
    __host__ __device__ size_t o_tiles() const { return o_ccount() + fs_align(rs() * 4); }
    __host__ __device__ size_t bytes() const { return o_tiles() + fs_align((size_t)nrows * ntiles * 8); }
    // [rows][S]: pass 0's partials
    __host__ __device__ FsPart0* p0() const { return (FsPart0*)(base + o_p0()); }
    // [rows][S][NBINS]: fs_hist_k's mass histograms, or pass 0's counts (u32, first half)
    __host__ __device__ u64* hist() const { return (u64*)(base + o_hist()); }
    // [rows][S][NUNITS]: fs_hist_k's histograms summed per unit of y
    __host__ __device__ u64* units() const { return (u64*)(base + o_units()); }
    // [rows][S][NUNITS]: pass 0's per-unit bounds of the mass (relative to the grid top)
    __host__ __device__ float2* ubound() const { return (float2*)(base + o_ubound()); }
    // [rows][S][4]: the collection's exact total, mass above the window, window mass
    __host__ __device__ u64* zab() const { return (u64*)(base + o_zab()); }
    // [rows][S][CAP]: the collected keys and masses, and their counts [rows][S]
    __host__ __device__ u64* ckey() const { return (u64*)(base + o_ckey()); }
    __host__ __device__ u64* cmass() const { return (u64*)(base + o_cmass()); }
    __host__ __device__ u32* ccount() const { return (u32*)(base + o_ccount()); }
    // [rows][ntiles]: kept masses per tile
    __host__ __device__ u64* tiles() const { return (u64*)(base + o_tiles()); }
};


struct FsPlan {
    int S, tpb, ntiles;
    size_t bytes;
};

FsPlan fs_plan(int rows, int vocab, int target_blocks = FS_TARGET_BLOCKS) {
    FsPlan p;
    p.ntiles = (vocab + TILE - 1) / TILE;
    int want = (target_blocks + rows - 1) / rows;
    if (want > p.ntiles) want = p.ntiles;
    if (want > FS_MAX_SPLITS) want = FS_MAX_SPLITS;
    if (want < 1) want = 1;
    p.tpb = (p.ntiles + want - 1) / want;
    p.S = (p.ntiles + p.tpb - 1) / p.tpb;
    p.bytes = FsWs{nullptr, rows, p.S, p.ntiles}.bytes();
    return p;
}

FsWs fs_carve(void* ws, int rows, const FsPlan& p) { return FsWs{(char*)ws, rows, p.S, p.ntiles}; }

template <int DT, bool COUNTS, bool MASK>
__device__ __forceinline__ Row<DT, COUNTS, MASK> make_row(const void* logits, long long stride, int vocab, const int* counts,
                                                          const u32* mask, const RowParamsDev& p, bool vec, int r) {
    Row<DT, COUNTS, MASK> R;
    R.x = (const char*)logits + (size_t)r * (size_t)stride * (DT == GBS_DTYPE_F32 ? 4 : 2);
    R.c = COUNTS ? counts + (size_t)r * vocab : nullptr;
    R.m = MASK ? mask + (size_t)r * ((vocab + 31) / 32) : nullptr;
    R.vocab = vocab;
    R.vec = vec;
    R.rinv = 1.0f / p.repetition;
    R.rep = p.repetition;
    R.freq = p.frequency;
    R.pres = p.presence;
    return R;
}

__device__ __forceinline__ void fs_out(int r, int id, int greedy, int status, float prob, float lp, int* out_ids, int* out_greedy,
                                       float* out_probs, float* out_logprobs, int* out_status) {
    out_ids[r] = status == GBS_ROW_OK ? id : -1;
    if (out_greedy) out_greedy[r] = status == GBS_ROW_OK ? greedy : -1;
    if (out_probs) out_probs[r] = status == GBS_ROW_OK ? prob : 0.f;
    if (out_logprobs) out_logprobs[r] = status == GBS_ROW_OK ? lp : __uint_as_float(0x7fc00000u);
    if (out_status) out_status[r] = status;
}

__device__ __forceinline__ float fs_logprob(float lx, float M, float clp, float lse_m, float lse_s) {
    if (isinf(M) || !isfinite(clp)) return __uint_as_float(0x7fc00000u);  // undefined: +inf maximum, 1/T beyond f32
    return ((lx - lse_m) * clp - log2f(lse_s)) * 0.6931471805599453f;
}

__device__ __forceinline__ float fs_clp(const RowParamsDev& p) {
    return p.temperature > 0.0f ? temp_scale(p.temperature) : 1.44269504088896340736f;
}

// Under per-row dispatch the split path runs over the rows the single-pass kernel flagged: its workspace holds DEFER_ROWS
// of them (8 blocks each); a flagged row past those is taken whole by one block of fs_collect_k (full_row).
constexpr int DEFER_ROWS = 32;

// The row a block of the split path works on, and its place in the workspace. Without per-row dispatch (flags null)
// both are blockIdx.y. Under it the grid is (S, DEFER_ROWS + 1): blockIdx.y = i < DEFER_ROWS is the i-th flagged row
// (in row order), and the blocks of blockIdx.y = DEFER_ROWS share out the flagged rows past those (rank DEFER_ROWS +
// blockIdx.x, + S, ...), each taken whole by fs_collect_k. Returns the row (-1: none) and sets *wr to the workspace
// place. Every thread of the block calls it.
__device__ int fs_row(const unsigned* __restrict__ flags, int rows, int rank, int* s_row) {
    if (threadIdx.x == 0) *s_row = -1;
    __syncthreads();
    const int w = threadIdx.x / WAVE, l = lane_id();
    __shared__ int s_wc[NWF];
    int base = 0;  // flagged rows before this chunk
    for (int c0 = 0; c0 < rows; c0 += NTF) {
        const int i = c0 + (int)threadIdx.x;
        const bool f = i < rows && flags[i] != 0u;
        const u64 b = ballot(f);
        if (l == 0) s_wc[w] = __popcll(b);
        __syncthreads();
        int before = base;
        for (int o = 0; o < w; ++o) before += s_wc[o];
        if (f && before + mbcnt(b) == rank) *s_row = i;
        int tot = 0;
        for (int o = 0; o < NWF; ++o) tot += s_wc[o];
        __syncthreads();
        base += tot;
        if (base > rank) break;
    }
    __syncthreads();
    return *s_row;
}

// Pass 0 of the split form: the block's maximum key, NaN flag, allowed count and log-sum-exp over its tiles, into
// ws.p0()[row][sp] (each wave's totals by cross-lane moves, then wave 0 over the waves': one barrier). For rows with
// top-p it also counts the block's tokens on the row's histogram grid (block bins b = kgrid - 1 - floor(128 l c2),
// clamped to [0, NBINS - 1]): kgrid is a multiple of 128, GRID_MARGIN units of y above the largest value of the row's
// first tile, which every block of the row reads, so all of them share the grid and their units (128 bins) align.
// The counts go to the workspace with each unit's bounds of the mass, relative to 2^(kgrid / 128): bin b holds masses
// in [2^(-(b + 1) / 128), 2^(-b / 128)); bin 0 also holds every value above the grid (its count is kept apart), the
// last bin every value below it (lower bound 0). fs_collect_k makes the row's record and its collection window from
// them. Not launched under per-row dispatch.
constexpr int GRID_MARGIN = 8;

template <int DT, bool COUNTS, bool MASK>
__global__ void __launch_bounds__(NTF) fs_pass0_k(const void* __restrict__ logits, long long stride, int vocab,
                                                  const int* __restrict__ counts, const u32* __restrict__ mask,
                                                  const RowParamsDev* __restrict__ params, const float* __restrict__ uniforms, bool vec,
                                                  int tpb, FsWs ws) {
    __shared__ u64 s_k[NWF];
    __shared__ u32 s_nn[NWF], s_na[NWF];
    __shared__ float s_lm[NWF], s_ls[NWF], s_pm[NWF];
    __shared__ u32 s_cnt[NBINS];
    const int S = gridDim.x, sp = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x, w = tid / WAVE, l = lane_id();
    const RowParamsDev p = params[r];
    if (params_invalid(p, uniforms[r])) return;  // fs_collect_k writes the row's results
    const Row<DT, COUNTS, MASK> R = make_row<DT, COUNTS, MASK>(logits, stride, vocab, counts, mask, p, vec, r);
    const float clp = fs_clp(p);
    const int ntiles = (vocab + TILE - 1) / TILE;
    const int t0 = sp * tpb, t1 = min(ntiles, t0 + tpb);
    // the histogram: rows with top-p, a temperature and a finite 1/T (the others never use it)
    const bool hist = p.top_p > 0.0f && p.top_p < 1.0f && p.temperature > 0.0f && __builtin_isfinite(clp);
    const float c2x = clp * (float)BINS_PER_UNIT;
    float kg1 = 0.f;  // kgrid - 1
    int kgrid = 0;
    auto grid = [&]() -> bool {
        if (!hist) return true;
        for (int i = tid; i < NBINS; i += NTF) s_cnt[i] = 0;
        // the row's first tile: its largest allowed value
        float lv[4];
        R.group(tid * 4, lv);
        float pm = fmaxf(fmaxf(lv[0], lv[1]), fmaxf(lv[2], lv[3]));
        pm = pm > -INFINITY ? pm : -INFINITY;  // NaN: no value
#pragma unroll
        for (int m = 1; m < WAVE; m <<= 1) pm = fmaxf(pm, __uint_as_float(xor_lane(__float_as_uint(pm), m)));
        if (l == 0) s_pm[w] = pm;
        __syncthreads();
        float bm = s_pm[0];
        for (int o = 1; o < NWF; ++o) bm = fmaxf(bm, s_pm[o]);
        // units of y above: clamped so that kgrid stays far inside int (values beyond it only widen the window)
        const float u = fminf(fmaxf(floorf(bm * clp), -4194304.0f), 4194304.0f);
        kgrid = ((int)u + 1 + GRID_MARGIN) * BINS_PER_UNIT;
        kg1 = (float)(kgrid - 1);
        return true;
    };
    Pass0Acc acc;
    auto group0 = [&](int, int e, const float (&lv)[4]) {
        acc.add(lv, e, clp);
        if (hist) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (valid_l(lv[q])) {
                    const float bf = fminf(fmaxf(kg1 - floorf(lv[q] * c2x), 0.0f), (float)(NBINS - 1));
                    atomicAdd(&s_cnt[(u32)bf], 1u);
                }
            }
        }
    };
#if GBS_FS_STEPS
    stream_steps<SG, GBS_FS_AUX0>(R, t0, t1, group0, [](int, int) {}, grid);
#else
    grid();
    stream_tiles(R, t0, t1, group0);
#endif
    const u64 k = wave_max_u64(acc.key());
    const u32 nn = wave_or(acc.nan), na = wave_sum_u32(acc.nallowed);
    const Lse ls = wave_lse(acc.lse, clp);
    if (l == 0) {
        s_k[w] = k;
        s_nn[w] = nn;
        s_na[w] = na;
        s_lm[w] = ls.m;
        s_ls[w] = ls.s;
    }
    __syncthreads();
    const size_t slot = (size_t)r * S + sp;
    if (hist) {
        // the counts, and per unit (wave w: units w, w + NWF, ...; two bins per lane) the bounds of its mass
        u32* cnt = (u32*)(ws.hist() + slot * NBINS);
        for (int i = tid; i < NBINS; i += NTF) st_agent(&cnt[i], s_cnt[i]);
        for (int u = w; u < NUNITS; u += NWF) {
            const int b0 = u * BINS_PER_UNIT + 2 * l;
            const float c0 = (float)s_cnt[b0], c1 = (float)s_cnt[b0 + 1];
            const float e0 = exp2f(-(float)b0 / (float)BINS_PER_UNIT), e1 = exp2f(-(float)(b0 + 1) / (float)BINS_PER_UNIT),
                        e2 = exp2f(-(float)(b0 + 2) / (float)BINS_PER_UNIT);
            float lo = c0 * e1 + (b0 + 1 == NBINS - 1 ? 0.0f : c1 * e2);
            float hi = c0 * e0 + c1 * e1;
#pragma unroll
            for (int m = 1; m < WAVE; m <<= 1) {
                lo += __uint_as_float(xor_lane(__float_as_uint(lo), m));
                hi += __uint_as_float(xor_lane(__float_as_uint(hi), m));
            }
            if (l == 0) st_agent((u64*)&ws.ubound()[slot * NUNITS + u], ((u64)__float_as_uint(hi) << 32) | __float_as_uint(lo));
        }
    }
    if (w != 0) return;
    const bool in = l < NWF;
    const u64 bk = wave_max_u64(in ? s_k[l] : 0ull);
    const u32 bnn = wave_or(in ? s_nn[l] : 0u), bna = wave_sum_u32(in ? s_na[l] : 0u);
    const Lse bl = wave_lse(in ? Lse{s_lm[l], s_ls[l]} : Lse{-INFINITY, 0.f}, clp);
    if (l == 0) {
        FsPart0* pp = &ws.p0()[slot];
        st_agent(&pp->key, bk);
        st_agent(&pp->nan, bnn);
        st_agent(&pp->nallowed, bna);
        st_agent((u32*)&pp->m, __float_as_uint(bl.m));
        st_agent((u32*)&pp->s, __float_as_uint(bl.s));
        st_agent(&pp->kgrid, kgrid);
        st_agent(&pp->pad, hist ? s_cnt[0] : 0u);
    }
}

// Under per-row dispatch: the binned cut's exact mass histogram of the flagged rows (the single-pass kernel has stored
// their records). Rows with top-p that continue the cut: the block's bins and its sums per unit of y go to the
// workspace, where fs_collect_k finds the crossing bin.
template <int DT, bool COUNTS, bool MASK>
__global__ void __launch_bounds__(NTF) fs_hist_k(const void* __restrict__ logits, long long stride, int vocab,
                                                 const int* __restrict__ counts, const u32* __restrict__ mask,
                                                 const RowParamsDev* __restrict__ params, bool vec, int tpb, FsWs ws,
                                                 const unsigned* __restrict__ flags, int rows) {
    __shared__ u64 s_hist[NBINS];
    __shared__ int s_sel;
    const int S = gridDim.x, sp = blockIdx.x, wr = blockIdx.y;
    if (wr >= DEFER_ROWS) return;
    const int r = fs_row(flags, rows, wr, &s_sel);
    if (r < 0) return;
    const int tid = threadIdx.x, w = tid / WAVE, l = lane_id();
    const RowParamsDev p = params[r];
    if (!(p.top_p > 0.0f && p.top_p < 1.0f)) return;  // no top-p: no histogram
    const FsRow* row = &ws.rec()[r];
    if (ld_agent(&row->state) != FS_CUT) return;
    const u64 top = ld_agent(&row->top);
    const Row<DT, COUNTS, MASK> R = make_row<DT, COUNTS, MASK>(logits, stride, vocab, counts, mask, p, vec, r);
    const float M = okey_to_f32(key_ok(top));
    const float c2 = temp_scale(p.temperature);
    const int ntiles = (vocab + TILE - 1) / TILE;
    const int t0 = sp * tpb, t1 = min(ntiles, t0 + tpb);
    auto hist_group = [&](int, int, const float (&lv)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u64 E = mass_fast(lv[q], M, c2);
            if (E) atomicAdd((unsigned long long*)&s_hist[bin_of(lv[q], M, c2)], (unsigned long long)E);
        }
    };
    auto zero = [&]() {
        for (int i = tid; i < NBINS; i += NTF) s_hist[i] = 0;
        __syncthreads();
        return true;
    };
#if GBS_FS_STEPS
    stream_steps<SG, GBS_FS_AUXH>(R, t0, t1, hist_group, [](int, int) {}, zero);
#else
    zero();
    stream_tiles(R, t0, t1, hist_group);
#endif
    __syncthreads();
    // the block's histogram, and its sums per unit of y (wave w sums units w, w + NWF, ...; two bins per lane)
    u64* mine = ws.hist() + ((size_t)wr * S + sp) * NBINS;
    for (int i = tid; i < NBINS; i += NTF) st_agent(&mine[i], s_hist[i]);
    u64* my_units = ws.units() + ((size_t)wr * S + sp) * NUNITS;
    for (int u = w; u < NUNITS; u += NWF) {
        const u64 v = wave_sum_u64(s_hist[u * BINS_PER_UNIT + l] + s_hist[u * BINS_PER_UNIT + WAVE + l]);
        if (l == 0) st_agent(&my_units[u], v);
    }
}

// wave-wide inclusive prefix sum of doubles (DPP row shifts, then row broadcasts, as wave_scan_u64)
__device__ __forceinline__ double wave_scan_f64(double v) {
    auto mv = [](double x, int ctrl, int rm) { return __longlong_as_double((long long)dpp64((u64)__double_as_longlong(x), ctrl, rm)); };
    v += mv(v, 0x111, 0xF);
    v += mv(v, 0x112, 0xF);
    v += mv(v, 0x114, 0xF);
    v += mv(v, 0x118, 0xF);
    v += mv(v, 0x142, 0xA);
    v += mv(v, 0x143, 0xC);
    return v;
}

constexpr int WIN_UNITS = 4;      // the collection window's histogram units at most (more: the row takes the radix path)
constexpr u32 FS_WINDOW_FAIL = 3;  // block-local state: no window could be made; the row's first block takes the row

// The collection window of a row without per-row dispatch, from pass 0's counts on the row's grid: the bins [r_lo,
// r_hi] of bin_of() that certainly hold the top-p cut, i.e. the mass below them is at most Z - P and the mass below
// their top more than Z - P (Z ~ the log-sum-exp, a relative margin of 2^-14). Found from the bottom: per unit of y the
// bounds of its mass (the blocks' sums in block order, so every block of the row finds the same window), then the bins
// of the at most WIN_UNITS units that hold the window's ends. Every thread calls both; fs_window returns false when no
// window is found (state FS_WINDOW_FAIL in s_w[2]). s_w: r_lo, r_hi, state.
// Loads of the window's first stage, by threads WAVE .. WAVE + NUNITS (the caller's wave 0 loads the record meanwhile):
// per unit the blocks' bounds summed in block order, and the count of bin 0 and the grid.
__device__ __forceinline__ void fs_window_load(const FsWs& ws, int wr, int S, double* s_u) {
    const int i = (int)threadIdx.x - WAVE;
    if (i >= 0 && i < NUNITS) {
        double lo = 0.0, hi = 0.0;
        for (int o0 = 0; o0 < S; o0 += 8) {
            u64 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = o0 + j < S ? ld_prev((const u64*)&ws.ubound()[((size_t)wr * S + o0 + j) * NUNITS + i]) : 0ull;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                lo += (double)__uint_as_float((u32)v[j]);
                hi += (double)__uint_as_float((u32)(v[j] >> 32));
            }
        }
        s_u[2 * i] = lo;
        s_u[2 * i + 1] = hi;
    } else if (i == NUNITS) {
        u32 c0 = 0;
        c0 = sum_blocks<u32>(S, [&](int o) { return ld_prev(&ws.p0()[(size_t)wr * S + o].pad); });
        s_u[2 * NUNITS] = (double)c0;
        s_u[2 * NUNITS + 1] = (double)ld_prev(&ws.p0()[(size_t)wr * S].kgrid);
    }
}

// The window from the loaded first stage (s_u, after a barrier).
__device__ __attribute__((noinline)) bool fs_window(const u64* hist, int wr, int S, float M, float c2, float top_p, float lse_m,
                                                     float lse_s, const double* s_u, u32* s_fc, int* s_w, double* s_wd) {
    const int tid = threadIdx.x, l = lane_id();
    const double kgrid = s_u[2 * NUNITS + 1];
    const double F = exp2(kgrid / BINS_PER_UNIT - (double)M * (double)c2);  // the grid top's mass, relative to the maximum's
    const double Zf = (double)lse_s, T = (1.0 - (double)top_p) * Zf, d = Zf * 0x1p-14;
    const double Tlo = T - d > 0.0 ? T - d : 0.0, Thi = T + d;
    const bool lse_ok = lse_m == M && Zf > 0.0 && __builtin_isfinite(Zf) && F > 0.0 && __builtin_isfinite(F);
    if (tid < WAVE) {
        const bool in = l < NUNITS;
        double lo = in ? s_u[2 * l] * F : 0.0, hi = in ? s_u[2 * l + 1] * F : 0.0;
        if (l == 0) hi += s_u[2 * NUNITS] * (1.0 - F);  // bin 0: values above the grid, masses up to the maximum's
        const double ilo = wave_scan_f64(lo), ihi = wave_scan_f64(hi);
        const double tlo = __longlong_as_double((long long)readlane64((u64)__double_as_longlong(ilo), WAVE - 1));
        const double thi = __longlong_as_double((long long)readlane64((u64)__double_as_longlong(ihi), WAVE - 1));
        const double blo = tlo - ilo, bhi = thi - ihi;  // the mass below unit l (deeper units)
        const u64 ca = ballot(in && blo + lo > Thi), cb = ballot(in && bhi <= Tlo);
        const int ua = ca ? 63 - __builtin_clzll(ca) : 0;
        const int ub = cb ? (int)__builtin_ctzll(cb) : NUNITS - 1;
        const int ulo = ua < ub ? ua : ub, uhi = ua < ub ? ub : ua;
        if (l == 0) {
            s_w[0] = ulo;
            s_w[1] = uhi;
            s_w[2] = lse_ok && uhi - ulo < WIN_UNITS ? (int)FS_CUT : (int)FS_WINDOW_FAIL;
        }
        if (l == uhi) {
            s_wd[0] = blo;
            s_wd[1] = bhi;
        }
    }
    __syncthreads();
    if (s_w[2] != (int)FS_CUT) return false;
    const int ulo = s_w[0], uhi = s_w[1];
    const int nb = (uhi - ulo + 1) * BINS_PER_UNIT;
    for (int i = tid; i < nb; i += NTF) {
        u32 c = 0;
        c = sum_blocks<u32>(S, [&](int o) { return ld_prev(&((const u32*)(hist + ((size_t)wr * S + o) * NBINS))[ulo * BINS_PER_UNIT + i]); });
        s_fc[i] = c;
    }
    __syncthreads();
    if (tid < WAVE) {
        // lane l: bins base + l * PB .. + PB - 1 of the units ulo..uhi (PB = 2 per unit)
        constexpr int PBM = 2 * WIN_UNITS;
        const int PB = nb / WAVE, base = ulo * BINS_PER_UNIT;
        double blo[PBM], bhi[PBM], slo = 0.0, shi = 0.0;
#pragma unroll
        for (int q = 0; q < PBM; ++q) {
            blo[q] = bhi[q] = 0.0;
            if (q < PB) {
                const int b = base + l * PB + q;
                const double c = (double)s_fc[l * PB + q];
                blo[q] = b == NBINS - 1 ? 0.0 : c * (double)exp2f(-(float)(b + 1) / (float)BINS_PER_UNIT) * F;
                bhi[q] = b == 0 ? c : c * (double)exp2f(-(float)b / (float)BINS_PER_UNIT) * F;
                slo += blo[q];
                shi += bhi[q];
            }
        }
        const double ilo = wave_scan_f64(slo), ihi = wave_scan_f64(shi);
        const double tlo = __longlong_as_double((long long)readlane64((u64)__double_as_longlong(ilo), WAVE - 1));
        const double thi = __longlong_as_double((long long)readlane64((u64)__double_as_longlong(ihi), WAVE - 1));
        // the mass below this lane's last bin: the deeper lanes' and the units below uhi
        double below_lo = s_wd[0] + (tlo - ilo), below_hi = s_wd[1] + (thi - ihi);
        int a = -1, bb = 1 << 30;
#pragma unroll
        for (int q = PBM - 1; q >= 0; --q) {
            if (q < PB) {
                const int b = base + l * PB + q;
                if (below_hi <= Tlo) bb = b;  // the mass below bin b is at most Z - P
                if (a < 0 && below_lo + blo[q] > Thi) a = b;  // the mass from bin b down exceeds Z - P
                below_lo += blo[q];
                below_hi += bhi[q];
            }
        }
        // b_a: the deepest bin whose mass from it down exceeds Z - P (none: the top of the units); b_b: the highest bin
        // whose mass below is at most Z - P
        int ba = a, bbv = bb;
#pragma unroll
        for (int m = 1; m < WAVE; m <<= 1) {
            ba = max(ba, (int)xor_lane((u32)ba, m));
            bbv = min(bbv, (int)xor_lane((u32)bbv, m));
        }
        if (ba < 0) ba = base;
        if (bbv > base + nb - 1) bbv = base + nb - 1;
        const int wa = ba < bbv ? ba : bbv, wb = ba < bbv ? bbv : ba;
        if (l == 0) {
            // grid bins [wa, wb] to bins of bin_of(): -128 y lies in (D + wa, D + 1 + wb], D = 128 M c2 - kgrid; one bin of
            // margin each side for the rounding of the two computations of y
            const double D = (double)BINS_PER_UNIT * (double)M * (double)c2 - kgrid;
            const double rlo = wa == 0 ? 0.0 : floor(D + wa) - 1.0, rhi = wb == NBINS - 1 ? (double)(NBINS - 1) : floor(D + wb) + 2.0;
            s_w[0] = (int)fmin(fmax(rlo, 0.0), (double)(NBINS - 1));
            s_w[1] = (int)fmin(fmax(rhi, 0.0), (double)(NBINS - 1));
        }
    }
    __syncthreads();
    return true;
}

// The collection: every token's exact mass is summed (the row's total Z), the masses of the bins above the window
// (the mass above it, and per 4096-element tile the kept ones: mass >= the min-p floor) and of the window's bins;
// the window's tokens go to the workspace. The window: without per-row dispatch, from pass 0's counts (fs_window); under
// it, the exact crossing bin of fs_hist_k's histograms. Without per-row dispatch each block first makes the row's record
// from pass 0's S partials (block 0 writes the results of the rows that need no cut). The row's last block checks that
// the window holds the cut (mass above < P = ceil(top_p Z) <= mass above + window mass), finds the exact top-p key
// among the window's tokens, adds the kept ones to their tiles and draws. A row marked for the radix path (top-k with a
// cut, an infinite maximum or 1/T), or without a window, is taken by its first block (the single-block path,
// full_row); a row whose window held more than CAP tokens or missed the cut, by its last block.
template <int DT, bool COUNTS, bool MASK>
__global__ void __launch_bounds__(NTF) fs_collect_k(const void* __restrict__ logits, long long stride, int vocab,
                                                    const int* __restrict__ counts, const u32* __restrict__ mask,
                                                    const RowParamsDev* __restrict__ params, const float* __restrict__ uniforms,
                                                    bool vec, int tpb, FsWs ws, int* __restrict__ out_ids, int* __restrict__ out_greedy,
                                                    float* __restrict__ out_probs, float* __restrict__ out_logprobs,
                                                    int* __restrict__ out_status, const unsigned* __restrict__ flags, int rows) {
    // the collection's arrays live in the radix path's LDS record (the two never run at the same time)
    __shared__ Shared sh;
    u64* const s_key = sh.maxk;
    u64* const s_mass = sh.mass;
    u64 (*const s_tilew)[NWF] = sh.tilew;
    u64* const s_tile = sh.tile;
    u64* const s_red = sh.red;
    u64* const s_bc = sh.bc;
    u32& s_ncol = sh.ncol;
    __shared__ u32 s_off[FS_MAX_SPLITS + 1];
    __shared__ unsigned s_flag;
    __shared__ int s_sel;
    __shared__ u64 s_rec[4];            // the row's maximum key, state, log-sum-exp pair
    __shared__ u64 s_z[3];              // exact total, mass above the window, window mass
    __shared__ int s_w[3];              // the window's bins r_lo, r_hi; state
    __shared__ double s_u[2 * NUNITS + 2], s_wd[2];
    __shared__ u32 s_fc[WIN_UNITS * BINS_PER_UNIT];
    __shared__ u64 s_cx[3];
    const int S = gridDim.x, sp = blockIdx.x, wr = blockIdx.y;
    if (flags && wr >= DEFER_ROWS) {
        // the flagged rows past the workspace's, shared out over this row of blocks: each is marked for fs_fallback_k
        for (int k = DEFER_ROWS + sp;; k += S) {
            const int q = fs_row(flags, rows, k, &s_sel);
            if (q < 0) break;
            if (threadIdx.x == 0) ws.fallback()[q] = 1u;
        }
        return;
    }
    const int r = flags ? fs_row(flags, rows, wr, &s_sel) : wr;
    if (r < 0) return;
    const int tid = threadIdx.x, w = tid / WAVE, l = lane_id();
    const RowParamsDev p = params[r];
    const float u = uniforms[r];
    const float c2 = temp_scale(p.temperature);
    const bool topp = p.top_p > 0.0f && p.top_p < 1.0f;
    const u64 Q = p.min_p > 0.0f ? mul_ceil64(p.min_p, MASS_ONE) : 0ull;
    const int ntiles = (vocab + TILE - 1) / TILE;
    const int t0 = sp * tpb, t1 = min(ntiles, t0 + tpb);
    const Row<DT, COUNTS, MASK> R = make_row<DT, COUNTS, MASK>(logits, stride, vocab, counts, mask, p, vec, r);
    if (!flags && params_invalid(p, u)) {
        if (sp == 0 && tid == 0) fs_out(r, -1, -1, GBS_ROW_INVALID_PARAMS, 0.f, 0.f, out_ids, out_greedy, out_probs, out_logprobs, out_status);
        return;
    }
    // The row's record and window, while the first loads are in flight.
    float M = 0.f, lse_m = 0.f, lse_s = 0.f;
    u64 top = 0;
    int r_lo = NBINS, r_hi = NBINS - 1;  // the window's bins (none: every bin is above it)
    u32 state = FS_CUT;
    auto prepare = [&]() -> bool {
        if (tid == 0) {
            s_ncol = 0;
            s_z[0] = s_z[1] = s_z[2] = 0;
        }
        for (int i = tid; i < (t1 - t0) * NWF; i += NTF) s_tilew[i / NWF][i % NWF] = 0;
        if (flags) {
            // the record, and (rows with top-p) fs_hist_k's sums per unit of y over the blocks, in block order
            if (tid == 0) {
                const FsRow* row = &ws.rec()[r];
                s_rec[0] = ld_prev(&row->top);
                s_rec[1] = ld_prev(&row->state);
                s_rec[2] = ld_prev((const u32*)&row->lse_m);
                s_rec[3] = ld_prev((const u32*)&row->lse_s);
            } else if (topp && tid >= WAVE && tid < WAVE + NUNITS) {
                const u64* U = ws.units() + (size_t)wr * S * NUNITS + (tid - WAVE);
                u64 v = 0;
                v = sum_blocks<u64>(S, [&](int o) { return ld_prev(&U[(size_t)o * NUNITS]); });
                ((u64*)s_u)[tid - WAVE] = v;
            }
        } else if (tid >= WAVE) {
            if (topp) fs_window_load(ws, wr, S, s_u);
        } else {
            // the record from pass 0's partials (every block of the row makes the same one)
            const float clp = fs_clp(p);
            u64 k = 0;
            u32 nn = 0, na = 0;
            Lse rl{-INFINITY, 0.f};
            for (int o = l; o < S; o += WAVE) {
                const FsPart0 pt = ld_prev(&ws.p0()[(size_t)wr * S + o]);  // the whole partial in one round of loads
                k = pt.key > k ? pt.key : k;
                nn |= pt.nan;
                na += pt.nallowed;
                rl = lse_merge(rl, Lse{pt.m, pt.s}, clp);
            }
            k = wave_max_u64(k);
            nn = wave_or(nn);
            na = wave_sum_u32(na);
            rl = wave_lse(rl, clp);
            const float Mk = okey_to_f32(key_ok(k));
            u32 st = FS_CUT;
            if (nn || na == 0 || p.temperature == 0.0f) st = FS_DONE;
            else if ((p.top_k > 0 && (u32)p.top_k < na) || !mass_fast_ok(Mk, c2)) st = FS_RADIX;
            if (l == 0) {
                s_rec[0] = k;
                s_rec[1] = st;
                s_rec[2] = __float_as_uint(rl.m);
                s_rec[3] = __float_as_uint(rl.s);
                if (sp == 0) {
                    const int greedy = (int)key_id(k);
                    if (nn)
                        fs_out(r, -1, -1, GBS_ROW_NAN_LOGIT, 0.f, 0.f, out_ids, out_greedy, out_probs, out_logprobs, out_status);
                    else if (na == 0)
                        fs_out(r, -1, -1, GBS_ROW_NO_CANDIDATES, 0.f, 0.f, out_ids, out_greedy, out_probs, out_logprobs, out_status);
                    else if (p.temperature == 0.0f)
                        fs_out(r, greedy, greedy, GBS_ROW_OK, 1.0f, fs_logprob(Mk, Mk, clp, rl.m, rl.s), out_ids, out_greedy, out_probs,
                               out_logprobs, out_status);
                }
            }
        }
        __syncthreads();
        top = s_rec[0];
        state = (u32)s_rec[1];
        lse_m = __uint_as_float((u32)s_rec[2]);
        lse_s = __uint_as_float((u32)s_rec[3]);
        M = okey_to_f32(key_ok(top));
        if (state != FS_CUT || !topp) return state == FS_CUT;
        if (!flags) {
            if (!fs_window(ws.hist(), wr, S, M, c2, p.top_p, lse_m, lse_s, s_u, s_fc, s_w, s_wd)) {
                state = FS_WINDOW_FAIL;
                return false;
            }
            r_lo = s_w[0];
            r_hi = s_w[1];
            return true;
        }
        // under per-row dispatch: the crossing bin b* of fs_hist_k's exact histograms (the blocks' sums per unit of y
        // give the total, P and the unit where the cumulative mass from the top reaches P; that unit's 128 bins summed
        // over the blocks give b*)
        const u64* const s_units = (const u64*)s_u;
        u64* const s_fine = (u64*)s_fc;
        if (tid < WAVE) {
            const u64 v = l < NUNITS ? s_units[l] : 0ull;
            const u64 Z = wave_sum_u64(v);
            const u64 Pv = mul_ceil64(p.top_p, Z);
            const u64 incl = wave_scan_u64(v);
            const int f = min((int)__builtin_ctzll(ballot(incl >= Pv) | (1ull << 63)), NUNITS - 1);  // Pv <= Z: a unit reaches it
            if (l == f) {
                s_cx[0] = (u64)f;
                s_cx[1] = incl - v;  // the mass of the units above
                s_cx[2] = Pv;
            }
        }
        __syncthreads();
        const int ustar = (int)s_cx[0];
        if (tid < BINS_PER_UNIT) {
            const u64* H = ws.hist() + (size_t)wr * S * NBINS + (size_t)ustar * BINS_PER_UNIT + tid;
            u64 v = 0;
            v = sum_blocks<u64>(S, [&](int o) { return ld_prev(&H[(size_t)o * NBINS]); });
            s_fine[tid] = v;
        }
        __syncthreads();
        if (tid < WAVE) {
            // lane i holds bins 2i, 2i + 1 of the unit: the first bin where the cumulative mass reaches P
            const u64 a0 = s_fine[2 * l], a1 = s_fine[2 * l + 1];
            const u64 Pv = s_cx[2];
            const u64 incl = s_cx[1] + wave_scan_u64(a0 + a1);
            const u64 excl = incl - a0 - a1;
            const int f = (int)__builtin_ctzll(ballot(incl >= Pv) | (1ull << 63));
            if (l == f) s_cx[0] = (u64)(ustar * BINS_PER_UNIT + 2 * l + (excl + a0 >= Pv ? 0 : 1));
        }
        __syncthreads();
        r_lo = r_hi = (int)s_cx[0];
        return true;
    };
    // per token: the exact mass into the total; above the window (kept: mass >= the min-p floor) into the tile's
    // partial, and into the mass above when there is a floor (else the mass above is the tiles' sum); in the window
    // into the wave's part of the LDS collection (CAP / NWF keys per wave; a wave that overflows marks the block)
    constexpr u32 WCAP = CAP / NWF;
    u64 sacc = 0, zacc = 0, aacc = 0;
    u32 wcount = 0;  // the wave's collected tokens (wave-uniform)
    auto collect_group = [&](int t, int e, const float (&lv)[4]) {
        u64 s = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u64 E = mass_fast(lv[q], M, c2);  // 0 for -inf
            const int b = topp ? (int)bin_of(lv[q], M, c2) : 0;
            zacc += E;
            const bool above = b < r_lo;
            s += above && E >= Q ? E : 0ull;
            if (Q) aacc += above ? E : 0ull;
            const bool col = valid_l(lv[q]) && !above && b <= r_hi;
            const u64 mk = ballot(col);
            if (mk) {
                const u32 idx = wcount + mbcnt(mk);
                if (col && idx < WCAP) {
                    s_key[w * WCAP + idx] = make_key(okey_f32(lv[q]), (u32)(e + q));
                    s_mass[w * WCAP + idx] = E;
                }
                wcount += (u32)__popcll(mk);
            }
        }
        sacc += s;
    };
    auto collect_step = [&](int t, int q) {
        const u64 v = wave_sum_u64(sacc);
        if (l == 0) s_tilew[t - t0][q] = v;
        sacc = 0;
    };
#if GBS_FS_STEPS
    stream_steps<SG, GBS_FS_AUXC>(R, t0, t1, collect_group, collect_step, prepare);
#else
    if (prepare())
        stream_tiles(R, t0, t1, [&](int t, int e, const float (&lv)[4]) {
            collect_group(t, e, lv);
            collect_step(t, w);
        });
#endif
    if (state != FS_CUT) {
        // marked for the radix path, or no window: the row's first block marks it for fs_fallback_k
        if ((state == FS_RADIX || state == FS_WINDOW_FAIL) && sp == 0 && tid == 0) ws.fallback()[r] = 1u;
        return;
    }
    // the block's totals (exact total, mass above when there is a floor, window mass) and the waves' collections, packed
    // in wave order into the workspace (a block whose wave overflowed counts CAP + 1 tokens)
    __shared__ u32 s_wc[NWF];
    {
        u64 wm = 0;
        const u32 mine = wcount < WCAP ? wcount : WCAP;
        for (u32 i = l; i < mine; i += WAVE) wm += s_mass[w * WCAP + i];
        const u64 z = wave_sum_u64(zacc), a = wave_sum_u64(aacc);
        wm = wave_sum_u64(wm);
        if (l == 0) {
            atomicAdd((unsigned long long*)&s_z[0], (unsigned long long)z);
            atomicAdd((unsigned long long*)&s_z[1], (unsigned long long)a);
            atomicAdd((unsigned long long*)&s_z[2], (unsigned long long)wm);
            s_wc[w] = wcount;
        }
    }
    __syncthreads();
    for (int t = t0 + tid; t < t1; t += NTF) {
        u64 v = 0;
#pragma unroll
        for (int k = 0; k < NWF; ++k) v += s_tilew[t - t0][k];
        st_agent(&ws.tiles()[(size_t)wr * ntiles + t], v);
    }
    const size_t slot = (size_t)wr * S + sp;
    {
        u32 before = 0, nb = 0;
        bool over = false;
        for (int o = 0; o < NWF; ++o) {
            before += o < w ? s_wc[o] : 0u;
            nb += s_wc[o];
            over |= s_wc[o] > WCAP;
        }
        const u32 mine = wcount < WCAP ? wcount : WCAP;
        for (u32 i = l; i < mine; i += WAVE) {
            st_agent(&ws.ckey()[slot * CAP + before + i], s_key[w * WCAP + i]);
            st_agent(&ws.cmass()[slot * CAP + before + i], s_mass[w * WCAP + i]);
        }
        if (tid == 0) {
            st_agent(&ws.ccount()[slot], over ? (u32)CAP + 1u : nb);
            st_agent(&ws.zab()[slot * 4 + 0], s_z[0]);
            st_agent(&ws.zab()[slot * 4 + 1], s_z[1]);
            st_agent(&ws.zab()[slot * 4 + 2], s_z[2]);
        }
    }
    if (!arrive_last(&ws.cnt2()[r], (unsigned)S, &s_flag)) return;
    // ---- the row's last block. Wave 0 loads the totals, the blocks' counts and the tiles' kept masses and checks the
    // window; a collection of at most SMALL_N tokens is gathered and cut on wave 0 alone (no barriers), a larger one by
    // the whole block. Then every wave scans the draw's tile.
    constexpr u32 SMALL_N = 2 * WAVE;
    if (w == 0) {
        // lanes o and o + 64 (S <= 128): the blocks' counts and totals; the tiles (ntiles <= 128); all loads issued
        // before any is used
        const int o1 = l, o2 = l + WAVE;
        const u32 c1 = o1 < S ? ld_agent(&ws.ccount()[(size_t)wr * S + o1]) : 0u;
        const u32 c2v = o2 < S ? ld_agent(&ws.ccount()[(size_t)wr * S + o2]) : 0u;
        u64 zz[2][3];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int o = h ? o2 : o1;
            const u64* zb = &ws.zab()[((size_t)wr * S + o) * 4];
#pragma unroll
            for (int k = 0; k < 3; ++k) zz[h][k] = o < S ? ld_agent(&zb[k]) : 0ull;
        }
        const u64 tl1 = l < ntiles ? ld_agent(&ws.tiles()[(size_t)wr * ntiles + l]) : 0ull;
        const u64 tl2 = l + WAVE < ntiles ? ld_agent(&ws.tiles()[(size_t)wr * ntiles + l + WAVE]) : 0ull;
        if (l < ntiles) s_tile[l] = tl1;
        if (l + WAVE < ntiles) s_tile[l + WAVE] = tl2;
        // the blocks' offsets: an inclusive scan over o1 then o2
        const u64 i1 = wave_scan_u64(c1), t1c = readlane64(i1, WAVE - 1);
        const u64 i2 = t1c + wave_scan_u64(c2v);
        if (l == 0) s_off[0] = 0;
        if (o1 < S) s_off[o1 + 1] = (u32)i1;
        if (o2 < S) s_off[o2 + 1] = (u32)i2;
        const u64 nn = readlane64(i2, WAVE - 1);
        const u32 n = nn > (u64)CAP ? (u32)CAP + 1u : (u32)nn;
        const u64 Ztot = wave_sum_u64(zz[0][0] + zz[1][0]), wmass = wave_sum_u64(zz[0][2] + zz[1][2]);
        u64 above = wave_sum_u64(zz[0][1] + zz[1][1]);
        if (Q == 0 && topp) above = wave_sum_u64(tl1 + tl2);  // no floor: the mass above the window is the tiles' sum
        const u64 P = topp ? mul_ceil64(p.top_p, Ztot) : 0ull;
        const bool ok = n <= (u32)CAP && (!topp || (above < P && P <= above + wmass));
        if (!ok && l == 0) ws.fallback()[r] = 1u;  // more tokens than the collection holds, or a missed cut: fs_fallback_k
        if (l == 0) {
            s_bc[1] = ok ? (u64)n : ~0ull;
            s_bc[2] = above;
            s_bc[3] = P;
        }
    }
    __syncthreads();
    if (s_bc[1] == ~0ull) return;
    const u32 n = (u32)s_bc[1];
    const u64 above = s_bc[2], P = s_bc[3];
    // collected token i is block o's token i - s_off[o], s_off[o] <= i < s_off[o + 1] (a binary search)
    auto fetch = [&](u32 i, u64& k, u64& m) {
        int lo = 0, hi = S;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_off[mid] <= i) lo = mid;
            else hi = mid;
        }
        const size_t src = ((size_t)wr * S + lo) * CAP + (i - s_off[lo]);
        k = ld_agent(&ws.ckey()[src]);
        m = ld_agent(&ws.cmass()[src]);
    };
    u64 kp = (u64)VALID_MIN_OK << 32;  // every valid key
    if (n <= SMALL_N) {
        if (w == 0) {
            u64 kk[SMALL_N / WAVE], mm[SMALL_N / WAVE];
#pragma unroll
            for (int q = 0; q < (int)(SMALL_N / WAVE); ++q) {
                kk[q] = mm[q] = 0;
                const u32 i = q * WAVE + (u32)l;
                if (i < n) fetch(i, kk[q], mm[q]);
            }
#pragma unroll
            for (int q = 0; q < (int)(SMALL_N / WAVE); ++q) {
                const u32 i = q * WAVE + (u32)l;
                if (i < n) {
                    s_key[i] = kk[q];
                    s_mass[i] = mm[q];
                }
            }
            if (topp) {
                kp = cut_collected_wave(s_key, s_mass, n, above, P, M, c2, r_lo, r_hi, sh.cnt);
                add_kept_to_tiles_wave(s_key, s_mass, n, kp, Q, s_tile);
            }
        }
    } else {
        for (u32 i = tid; i < n; i += NTF) fetch(i, s_key[i], s_mass[i]);
        __syncthreads();
        kp = cut_collected(s_key, s_mass, n, above, P, M, c2, r_lo, r_hi, sh.cnt, s_bc);
        add_kept_to_tiles_wave(s_key, s_mass, n, kp, Q, s_tile, w, NWF);
        __syncthreads();
    }
    if (w == 0) {
        // the draw's tile: a scan of the tiles' kept masses, 64 at a time
        u64 zl = 0;
        for (int t = l; t < ntiles; t += WAVE) zl += s_tile[t];
        const u64 zt = wave_sum_u64(zl);
        const u64 tg = (u64)mul_floor(u, (u128)zt, nullptr);
        int ts = ntiles - 1;
        u64 bf = zt - s_tile[ntiles - 1];
        u64 run = 0;
        for (int c = 0; c < ntiles; c += WAVE) {
            const bool in = c + l < ntiles;
            const u64 v = in ? s_tile[c + l] : 0ull;
            const u64 incl = run + wave_scan_u64(v);
            const u64 hit = ballot(in && incl > tg);
            if (hit) {
                const int f = (int)__builtin_ctzll(hit);
                ts = c + f;
                bf = readlane64(incl - v, f);
                break;
            }
            run = readlane64(incl, WAVE - 1);
        }
        if (l == 0) {
            s_bc[0] = kp;
            s_bc[4] = zt;
            s_bc[5] = tg;
            s_bc[6] = (u64)ts;
            s_bc[7] = bf;
        }
    }
    __syncthreads();
    kp = s_bc[0];
    const u64 z = s_bc[4], target = s_bc[5], before = s_bc[7];
    const int tsel = (int)s_bc[6];
    auto kept_mass = [&](float v, int i) -> u64 {
        if (!valid_l(v)) return 0ull;
        if (make_key(okey_f32(v), (u32)i) < kp) return 0ull;
        const u64 E = mass(v, M, c2);
        return E >= Q ? E : 0ull;
    };
    const int e = tsel * TILE + tid * 4;
    float lv[4];
    R.group(e, lv);
    u64 em[4], mine = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        em[q] = kept_mass(lv[q], e + q);
        mine += em[q];
    }
    const u64 incl = wave_scan_u64(mine);
    if (l == WAVE - 1) s_red[w] = incl;
    __syncthreads();
    u64 wbase = before;
    for (int o = 0; o < w; ++o) wbase += s_red[o];
    const u64 excl = wbase + incl - mine;
    if (excl <= target && target < excl + mine) {
        // the first of the thread's four elements whose running mass exceeds the target (selections, no indexing)
        u64 acc = excl, ef = 0;
        int qf = -1;
        float lf = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc += em[q];
            const bool hit = qf < 0 && acc > target;
            qf = hit ? q : qf;
            ef = hit ? em[q] : ef;
            lf = hit ? lv[q] : lf;
        }
        s_bc[1] = (u64)(e + qf);
        s_bc[2] = ef;
        s_bc[3] = __float_as_uint(lf);
    }
    __syncthreads();
    if (tid == 0) {
        const float clp = fs_clp(p);
        fs_out(r, (int)s_bc[1], (int)key_id(top), GBS_ROW_OK, (float)((double)s_bc[2] / (double)z),
               fs_logprob(__uint_as_float((u32)s_bc[3]), M, clp, lse_m, lse_s), out_ids, out_greedy, out_probs, out_logprobs, out_status);
    }
}

}  // namespace


namespace gbs {

size_t sample_full_workspace_bytes(int rows, int vocab) {
    const FsPlan pl = fs_plan(rows, vocab);
    return pl.S >= 2 ? pl.bytes : 256;
}

size_t sample_full_deferred_workspace_bytes(int rows, int vocab) {
    return fs_plan(rows < DEFER_ROWS ? rows : DEFER_ROWS, vocab, FS_DEFER_BLOCKS).bytes;
}

int launch_sample_full(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts, const uint32_t* mask,
                       const void* params, const float* uniforms, int* out_ids, int* out_greedy, float* out_probs, float* out_logprobs,
                       int* out_status, void* ws, size_t ws_bytes, void* stream, const unsigned* row_flags) {
    const size_t esz = dtype == GBS_DTYPE_F32 ? 4 : 2;
    const bool vec = stride % 4 == 0 && aligned(logits, 4 * esz) && (!counts || (vocab % 4 == 0 && aligned(counts, 16)));
    const hipStream_t st = to_stream(stream);
    const RowParamsDev* p = (const RowParamsDev*)params;
    // under per-row dispatch the split path serves the flagged rows, its workspace sized for DEFER_ROWS of them
    const int wrows = row_flags ? (rows < DEFER_ROWS ? rows : DEFER_ROWS) : rows;
    const FsPlan pl = row_flags ? fs_plan(wrows, vocab, FS_DEFER_BLOCKS) : fs_plan(wrows, vocab);
    const bool split = pl.S >= 2 || row_flags;
    if (split && (!ws || !aligned(ws, 256) || ws_bytes < pl.bytes)) return GBS_ERR_INVALID;
    const FsWs w = split ? fs_carve(ws, wrows, pl) : FsWs{};
    auto run = [&]<int D, bool C, bool Mk>() {
        if (split) {
            const dim3 grid(pl.S, row_flags ? DEFER_ROWS + 1 : rows);
            // flagged rows: the single-pass kernel has written their records (maximum, log-sum-exp, state), so no pass 0
            // without per-row dispatch pass 0 (maximum, log-sum-exp, counts on the row's grid) and the collection; under
            // it the single-pass kernel has written the flagged rows' records, and the exact histogram gives the window
            if (!row_flags)
                hipLaunchKernelGGL((fs_pass0_k<D, C, Mk>), grid, dim3(NTF), 0, st, logits, (long long)stride, vocab, counts, mask, p, uniforms,
                                   vec, pl.tpb, w);
            else
                hipLaunchKernelGGL((fs_hist_k<D, C, Mk>), grid, dim3(NTF), 0, st, logits, (long long)stride, vocab, counts, mask, p, vec,
                                   pl.tpb, w, row_flags, rows);
            hipLaunchKernelGGL((fs_collect_k<D, C, Mk>), grid, dim3(NTF), 0, st, logits, (long long)stride, vocab, counts, mask, p,
                               uniforms, vec, pl.tpb, w, out_ids, out_greedy, out_probs, out_logprobs, out_status, row_flags, rows);
            hipLaunchKernelGGL((fs_fallback_k<D, C, Mk>), dim3(rows), dim3(NTF), 0, st, logits, (long long)stride, vocab, counts, mask,
                               p, uniforms, vec, out_ids, out_greedy, out_probs, out_logprobs, out_status, w.fallback());
        }
        else
            hipLaunchKernelGGL((sample_full_k<D, C, Mk>), dim3(rows), dim3(NTF), 0, st, logits, (long long)stride, vocab, counts, mask,
                               p, uniforms, vec, out_ids, out_greedy, out_probs, out_logprobs, out_status, row_flags);
    };
    const bool c = counts != nullptr, m = mask != nullptr;
    if (dtype == GBS_DTYPE_F32) {
        if (c && m) run.template operator()<GBS_DTYPE_F32, true, true>();
        else if (c) run.template operator()<GBS_DTYPE_F32, true, false>();
        else if (m) run.template operator()<GBS_DTYPE_F32, false, true>();
        else run.template operator()<GBS_DTYPE_F32, false, false>();
    } else if (dtype == GBS_DTYPE_BF16) {
        if (c && m) run.template operator()<GBS_DTYPE_BF16, true, true>();
        else if (c) run.template operator()<GBS_DTYPE_BF16, true, false>();
        else if (m) run.template operator()<GBS_DTYPE_BF16, false, true>();
        else run.template operator()<GBS_DTYPE_BF16, false, false>();
    } else {
        if (c && m) run.template operator()<GBS_DTYPE_F16, true, true>();
        else if (c) run.template operator()<GBS_DTYPE_F16, true, false>();
        else if (m) run.template operator()<GBS_DTYPE_F16, false, true>();
        else run.template operator()<GBS_DTYPE_F16, false, false>();
    }
    return launch_status();
}

}  // namespace gbs
