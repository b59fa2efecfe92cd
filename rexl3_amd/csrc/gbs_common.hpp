// Shared device code of libgbsample_hip.so (gfx950, wave64).
//
// Order keys. Every selection in this library ranks (value desc, id asc) through a u64 key that is larger for a better
// element: the value mapped to an order-preserving u32 in the high word, ~id in the low word. Keys are distinct, so any
// selection algorithm and any split of a row into chunks returns the same set in the same order.
//
// Wave lists. A wave keeps a sorted list of 64 keys in registers, lane i holding rank i. Candidates that beat the
// list's `count`-th key (a gate: anything at or below it cannot be in the answer) are appended to a wave-private LDS
// buffer by ballot + mbcnt compaction; 64 buffered keys at a time are sorted by a register bitonic network and merged
// into the list (max against the reversed group, then a bitonic clean-up), which raises the gate.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gbs_sample.h"

#define GBS_EXPORT extern "C" __attribute__((visibility("default")))

typedef uint64_t u64;
typedef uint32_t u32;
typedef uint16_t u16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace gbs {

constexpr int WAVE = 64;

static inline hipStream_t to_stream(void* s) { return (hipStream_t)s; }
static inline int launch_status() { return (int)hipGetLastError(); }
__host__ __device__ static inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// ------------------------------------------------------------------------------------------------ value -> order key

// f32 for the extended pipeline and the f32 top-k contract: -0 and +0 map to the same key. NaN is handled by the
// callers (the f32 top-k contract ranks it below -inf: key 0; the pipeline flags it).
__device__ __forceinline__ u32 okey_f32(float f) {
    const u32 u = __float_as_uint(f);
    if ((u << 1) == 0u) return 0x80000000u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// okey_f32 in four operations: adding +0 turns -0 into +0 (and changes no other value), then the sign-flip map
__device__ __forceinline__ u32 okey_f32_fast(float f) {
    const u32 u = __float_as_uint(f + 0.0f);
    return u ^ ((u32)((int)u >> 31) | 0x80000000u);
}

// inverse of okey_f32 (a zero comes back as +0)
__device__ __forceinline__ float okey_to_f32(u32 k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// the f32 top-k contract (reference crates/cuda/csrc/nemotron_glue.cu:191-203): NaN below -inf
__device__ __forceinline__ u32 okey_f32_nanlow(float f) {
    const u32 u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0u;
    return okey_f32(f);
}

// 16-bit floats (reference crates/cuda/csrc/glue.cu:529-534 for bf16, crates/cuda/csrc/glm_glue.cu:105-110 for fp16):
// NaN -> -inf, -0 -> +0, then the sign-flip map into 16 bits.
template <bool F16>
__device__ __forceinline__ u32 okey_16(u32 h) {
    constexpr u32 inf = F16 ? 0x7C00u : 0x7F80u;
    constexpr u32 ninf = F16 ? 0xFC00u : 0xFF80u;
    h &= 0xFFFFu;
    if ((h & 0x7FFFu) > inf) h = ninf;
    else if ((h & 0x7FFFu) == 0u) h = 0u;
    return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
}

template <bool F16>
__device__ __forceinline__ float okey16_to_f32(u32 k) {
    const u32 h = (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
    if (F16) return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
    return __uint_as_float(h << 16);
}

__device__ __forceinline__ u64 make_key(u32 ok, u32 id) { return ((u64)ok << 32) | (u64)(~id); }
__device__ __forceinline__ u32 key_id(u64 k) { return ~(u32)k; }
__device__ __forceinline__ u32 key_ok(u64 k) { return (u32)(k >> 32); }

// ------------------------------------------------------------------------------------------------ wave primitives

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ u64 shfl_xor64(u64 v, int m) {
    const u32 lo = (u32)__shfl_xor((int)(u32)v, m, WAVE);
    const u32 hi = (u32)__shfl_xor((int)(u32)(v >> 32), m, WAVE);
    return ((u64)hi << 32) | lo;
}

// v of lane (lane ^ m), m a power of two below 64, without LDS: DPP within 16-lane rows (quad_perm for 1 and 2, row
// rotations for 4 and 8), v_permlane16_swap / v_permlane32_swap across rows. m must be a compile-time constant after
// unrolling.
__device__ __forceinline__ u32 xor_lane(u32 v, int m) {
    const int l = (int)__lane_id();
    switch (m) {
        case 1: return (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
        case 2: return (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
        case 4: {
            const u32 down = (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false);  // row_ror:4  -> lane - 4
            const u32 up = (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x12C, 0xF, 0xF, false);    // row_ror:12 -> lane + 4
            return (l & 4) ? down : up;
        }
        case 8: return (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
        case 16: {
            const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
            return (l & 16) ? (u32)r[0] : (u32)r[1];
        }
        default: {
            const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
            return (l & 32) ? (u32)r[0] : (u32)r[1];
        }
    }
}

__device__ __forceinline__ u64 xor_lane64(u64 v, int m) {
    return ((u64)xor_lane((u32)(v >> 32), m) << 32) | xor_lane((u32)v, m);
}

__device__ __forceinline__ u64 shfl64(u64 v, int src) {
    const u32 lo = (u32)__shfl((int)(u32)v, src, WAVE);
    const u32 hi = (u32)__shfl((int)(u32)(v >> 32), src, WAVE);
    return ((u64)hi << 32) | lo;
}

__device__ __forceinline__ u64 readlane64(u64 v, int lane) {
    const u32 lo = (u32)__builtin_amdgcn_readlane((int)(u32)v, lane);
    const u32 hi = (u32)__builtin_amdgcn_readlane((int)(u32)(v >> 32), lane);
    return ((u64)hi << 32) | lo;
}

__device__ __forceinline__ u32 readlane32(u32 v, int lane) { return (u32)__builtin_amdgcn_readlane((int)v, lane); }

__device__ __forceinline__ u64 ballot(bool p) { return __ballot(p); }

// lanes below this one with their bit set
__device__ __forceinline__ int mbcnt(u64 m) {
    return (int)__builtin_amdgcn_mbcnt_hi((u32)(m >> 32), __builtin_amdgcn_mbcnt_lo((u32)m, 0u));
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// descending bitonic sort of one key per lane (lane 0 ends with the largest)
__device__ __forceinline__ u64 wave_sort_desc(u64 v) {
    const int l = lane_id();
#pragma unroll
    for (int k = 2; k <= WAVE; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const u64 o = xor_lane64(v, j);
            const bool lower = (l & j) == 0;
            const bool desc = (l & k) == 0;
            const bool keep_max = (lower == desc);
            v = keep_max ? (v > o ? v : o) : (v < o ? v : o);
        }
    }
    return v;
}

// ascending bitonic sort of one u64 per lane (lane 0 ends with the smallest)
__device__ __forceinline__ u64 wave_sort_asc(u64 v) {
    const int l = lane_id();
#pragma unroll
    for (int k = 2; k <= WAVE; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const u64 o = xor_lane64(v, j);
            const bool lower = (l & j) == 0;
            const bool asc = (l & k) == 0;
            const bool keep_min = (lower == asc);
            v = keep_min ? (v < o ? v : o) : (v > o ? v : o);
        }
    }
    return v;
}

// ascending bitonic sort of one u32 per lane (lane 0 ends with the smallest)
__device__ __forceinline__ u32 wave_sort_asc32(u32 v) {
    const int l = lane_id();
#pragma unroll
    for (int k = 2; k <= WAVE; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const u32 o = xor_lane(v, j);
            const bool lower = (l & j) == 0;
            const bool asc = (l & k) == 0;
            const bool keep_min = (lower == asc);
            v = keep_min ? (v < o ? v : o) : (v > o ? v : o);
        }
    }
    return v;
}

// descending bitonic clean-up of a bitonic sequence
__device__ __forceinline__ u64 wave_bitonic_desc(u64 v) {
    const int l = lane_id();
#pragma unroll
    for (int j = WAVE / 2; j > 0; j >>= 1) {
        const u64 o = xor_lane64(v, j);
        const bool lower = (l & j) == 0;
        v = lower ? (v > o ? v : o) : (v < o ? v : o);
    }
    return v;
}

// the 64 largest of a descending list and an ascending list (one key per lane each), descending
__device__ __forceinline__ u64 wave_merge_desc_asc(u64 a_desc, u64 b_asc) { return wave_bitonic_desc(a_desc > b_asc ? a_desc : b_asc); }

// v of lane 63 - lane: mirror within each 16-lane row (DPP), then swap row halves and neighbouring rows (permlanes)
__device__ __forceinline__ u32 reverse_lane(u32 v) {
    const int l = (int)__lane_id();
    u32 m = (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false);  // row_mirror
    const auto a = __builtin_amdgcn_permlane32_swap(m, m, false, false);
    m = (l & 32) ? (u32)a[0] : (u32)a[1];
    const auto b = __builtin_amdgcn_permlane16_swap(m, m, false, false);
    return (l & 16) ? (u32)b[0] : (u32)b[1];
}

__device__ __forceinline__ u64 reverse_lane64(u64 v) { return ((u64)reverse_lane((u32)(v >> 32)) << 32) | reverse_lane((u32)v); }

// the 64 largest of two descending lists, descending
__device__ __forceinline__ u64 wave_merge_desc(u64 a, u64 b_desc) {
    const u64 br = reverse_lane64(b_desc);
    return wave_bitonic_desc(a > br ? a : br);
}

// the k-th largest (1 <= k <= 64) of one u32 per lane: the largest r with at least k lanes holding a value >= r
__device__ __forceinline__ u32 wave_kth_largest(u32 v, int k) {
    u32 r = 0;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const u32 c = r | (1u << b);
        if (__popcll(ballot(v >= c)) >= k) r = c;
    }
    return r;
}

__device__ __forceinline__ u64 wave_sum_u64(u64 v) {
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) v += xor_lane64(v, m);
    return v;
}

// u64 of the DPP-shifted lane (0 where the control selects no lane or the row is masked off)
__device__ __forceinline__ u64 dpp64(u64 v, int ctrl, int row_mask) {
    u32 lo, hi;
    switch (ctrl) {  // the control must be a constant: one case per use
        case 0x111: lo = __builtin_amdgcn_update_dpp(0, (int)(u32)v, 0x111, 0xF, 0xF, true); hi = __builtin_amdgcn_update_dpp(0, (int)(u32)(v >> 32), 0x111, 0xF, 0xF, true); break;
        case 0x112: lo = __builtin_amdgcn_update_dpp(0, (int)(u32)v, 0x112, 0xF, 0xF, true); hi = __builtin_amdgcn_update_dpp(0, (int)(u32)(v >> 32), 0x112, 0xF, 0xF, true); break;
        case 0x114: lo = __builtin_amdgcn_update_dpp(0, (int)(u32)v, 0x114, 0xF, 0xF, true); hi = __builtin_amdgcn_update_dpp(0, (int)(u32)(v >> 32), 0x114, 0xF, 0xF, true); break;
        case 0x118: lo = __builtin_amdgcn_update_dpp(0, (int)(u32)v, 0x118, 0xF, 0xF, true); hi = __builtin_amdgcn_update_dpp(0, (int)(u32)(v >> 32), 0x118, 0xF, 0xF, true); break;
        case 0x142: lo = __builtin_amdgcn_update_dpp(0, (int)(u32)v, 0x142, 0xA, 0xF, false); hi = __builtin_amdgcn_update_dpp(0, (int)(u32)(v >> 32), 0x142, 0xA, 0xF, false); break;
        default: lo = __builtin_amdgcn_update_dpp(0, (int)(u32)v, 0x143, 0xC, 0xF, false); hi = __builtin_amdgcn_update_dpp(0, (int)(u32)(v >> 32), 0x143, 0xC, 0xF, false); break;
    }
    (void)row_mask;
    return ((u64)hi << 32) | lo;
}

// inclusive prefix sum over lanes: DPP row shifts within 16-lane rows, then row broadcasts across rows
__device__ __forceinline__ u64 wave_scan_u64(u64 v) {
    v += dpp64(v, 0x111, 0xF);  // row_shr:1
    v += dpp64(v, 0x112, 0xF);  // row_shr:2
    v += dpp64(v, 0x114, 0xF);  // row_shr:4
    v += dpp64(v, 0x118, 0xF);  // row_shr:8
    v += dpp64(v, 0x142, 0xA);  // row_bcast:15 into rows 1 and 3
    v += dpp64(v, 0x143, 0xC);  // row_bcast:31 into rows 2 and 3
    return v;
}

__device__ __forceinline__ u64 wave_max_u64(u64 v) {
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) {
        const u64 o = xor_lane64(v, m);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ u32 wave_or(u32 v) {
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) v |= xor_lane(v, m);
    return v;
}

// ------------------------------------------------------------------------------------------------ wave top list

// A wave's gated top list. `buf` is the wave's private LDS buffer of at least BUF keys.
template <int BUF>
struct WaveTop {
    u64 list;  // rank lane_id()
    u64 thr;   // key of rank count - 1 (wave-uniform); keys <= thr are dropped
    u32 gate;  // order values below the gate cannot pass: (thr >> 32) + (low word of thr all ones)
    int n;     // buffered keys (wave-uniform)
    int count;
    u64* buf;

    float gate_f;  // the float whose order value is `gate`: for a non-NaN v, okey(v) >= gate <=> v >= gate_f

    static constexpr int INSERT_MAX = 6;  // survivors of a flush inserted one by one rather than sorted
    __device__ __forceinline__ void set_thr(u64 t) {
        thr = t;
        const u32 hi = (u32)(t >> 32);
        gate = ((u32)t == 0xFFFFFFFFu && hi != 0xFFFFFFFFu) ? hi + 1u : hi;
        gate_f = okey_to_f32(gate);
    }

    // offer element `id` of value `v` (f32 order, NaN never passes): one float compare per element; the order key is
    // built only for the elements that pass
    __device__ __forceinline__ void offer_f(float v, u32 id) {
        const bool pass = v >= gate_f;
        const u64 m = ballot(pass);
        if (m) {
            if (pass) buf[n + mbcnt(m)] = make_key(okey_f32_fast(v), id);
            n += __popcll(m);
        }
    }

    // Optional sharing of the gate: every wave's `count`-th key is a lower bound of the count-th key of its whole row,
    // so waves publish it to a block-wide LDS slot (atomic max) and raise their own gate to the largest published value.
    u64* s_shared;  // LDS, block-wide (may be null)
    // Block bound: every wave publishes the order values of its TOPN best keys into its own LDS row. These are
    // distinct elements of the block (each wave sees its own elements), so the count-th largest of all published
    // values has at least `count` elements of the row at or above it: a lower bound of the row's count-th key that
    // tracks the block as a whole, however unevenly its best elements fall on the waves.
    static constexpr int TOPN = 8;
    u32* s_top;  // LDS, nw * TOPN entries, zero at start (may be null)
    int top_w, top_n;

    __device__ __forceinline__ void set_top(u32* t, int w, int nw) {
        s_top = t;
        top_w = w;
        top_n = nw * TOPN;
        if (top_n > 2 * WAVE) s_top = nullptr;
    }

    // raise the gate to the block bound of the published values (all lanes of the wave call it): the count-th largest
    // published value, by one wave sort when they fit one per lane, else by a bitwise search of the counts
    __device__ __forceinline__ void block_bound() {
        const int l = lane_id();
        const u32 v0 = l < top_n ? s_top[l] : 0u;
        u32 r = 0;
        if (top_n <= WAVE) {
            const u64 sv = wave_sort_desc(((u64)v0 << 32) | (u64)l);
            r = count <= WAVE ? (u32)(readlane64(sv, count - 1) >> 32) : 0u;
        } else {
            const u32 v1 = l + WAVE < top_n ? s_top[l + WAVE] : 0u;
#pragma unroll
            for (int b = 31; b >= 0; --b) {
                const u32 c = r | (1u << b);
                if (__popcll(ballot(v0 >= c)) + __popcll(ballot(v1 >= c)) >= count) r = c;
            }
        }
        if (r > 0u) {
            const u64 t = ((u64)r << 32) - 1ull;
            if (t > thr) {
                set_thr(t);
                if (l == 0 && s_shared) __hip_atomic_fetch_max(s_shared, t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
    }

    __device__ __forceinline__ void publish_top() {
        if (!s_top) return;
        if (lane_id() < TOPN) s_top[top_w * TOPN + lane_id()] = (u32)(list >> 32);
        wave_lds_sync();
        block_bound();
    }

    __device__ __forceinline__ void init(u64* b, int cnt, u64 floor_key, u64* sh = nullptr) {
        list = 0;
        set_thr(floor_key);
        n = 0;
        count = cnt;
        buf = b;
        s_shared = sh;
        s_top = nullptr;
        top_w = 0;
        top_n = 0;
        pend_l = 0;
    }

    __device__ __forceinline__ void publish() {
        if (lane_id() == 0 && s_shared) __hip_atomic_fetch_max(s_shared, thr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }

    // Read the shared bound (relaxed; a stale value is still a valid bound) into `pend_l`; apply_shared() raises the
    // gate with it one step later, so the LDS read never makes the wave wait.
    u64 pend_l = 0;

    __device__ __forceinline__ void prefetch_shared() {
        if (s_shared) pend_l = __hip_atomic_load(s_shared, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }

    __device__ __forceinline__ void apply_shared() {
        const u64 t = readlane64(pend_l, 0);
        if (t > thr) set_thr(t);
    }

    // offer one key per lane (any lane may offer a key that fails the gate)
    __device__ __forceinline__ void offer(u64 k) {
        const bool pass = k > thr;
        const u64 m = ballot(pass);
        if (m) {
            if (pass) buf[n + mbcnt(m)] = k;
            n += __popcll(m);
        }
    }

    // offer element `id` of order value `ok`. The cheap 32-bit gate lets ties of the gate value through; the merge is
    // exact, so a key that passes needlessly only costs a slot.
    __device__ __forceinline__ void offer_ok(u32 ok, u32 id, bool valid = true) {
        const bool pass = valid && ok >= gate;
        const u64 m = ballot(pass);
        if (m) {
            if (pass) buf[n + mbcnt(m)] = make_key(ok, id);
            n += __popcll(m);
        }
    }

    // merge buffered keys, 64 at a time; `all` also merges a partial group
    // Insert one key (wave-uniform, above thr) into the descending list: its rank is the number of entries above it;
    // the entries from that rank on move down one lane (the last one drops out).
    __device__ __forceinline__ void insert(u64 k) {
        const int l = lane_id();
        const int pos = __popcll(ballot(list > k));
        const u32 lo = (u32)__builtin_amdgcn_update_dpp(0, (int)(u32)list, 0x138, 0xF, 0xF, false);  // wave_shr:1
        const u32 hi = (u32)__builtin_amdgcn_update_dpp(0, (int)(u32)(list >> 32), 0x138, 0xF, 0xF, false);
        const u64 below = ((u64)hi << 32) | lo;
        list = l < pos ? list : (l == pos ? k : below);
    }

    // merge buffered keys, 64 at a time; `all` also merges a partial group. Keys the gate has passed by since they
    // were buffered are dropped first; a few survivors are inserted one by one, more are sorted and merged.
    __device__ __forceinline__ void flush(bool all) {
        if (n < WAVE && !(all && n > 0)) return;
        wave_lds_sync();
        const int l = lane_id();
        while (n >= WAVE || (all && n > 0)) {
            const int take = n < WAVE ? n : WAVE;
            const int base = n - take;
            u64 g = l < take ? buf[base + l] : 0ull;
            n = base;
            u64 km = ballot(g > thr);
            if (km == 0ull) continue;
            if (__popcll(km) <= INSERT_MAX) {
                do {
                    const int src = (int)__builtin_ctzll(km);
                    km &= km - 1ull;
                    const u64 k = readlane64(g, src);
                    if (k > thr) {
                        insert(k);
                        const u64 t = readlane64(list, count - 1);
                        if (t > thr) set_thr(t);
                    }
                } while (km);
            } else {
                g = wave_sort_asc(g > thr ? g : 0ull);
                list = wave_merge_desc_asc(list, g);
                const u64 t = readlane64(list, count - 1);
                if (t > thr) set_thr(t);
            }
        }
        publish();
        if (!all) publish_top();
        wave_lds_sync();
    }

    // offer element `id` of value `v` whose gate test `v >= gate_f` was already taken: `pass` is this lane's result,
    // `m` the wave's ballot of it
    __device__ __forceinline__ void offer_tested(u64 m, bool pass, float v, u32 id) {
        if (m) {
            if (pass) buf[n + mbcnt(m)] = make_key(okey_f32_fast(v), id);
            n += __popcll(m);
        }
    }

    // Raise the gate from a sample: `ok` is one order value (key high word) per lane, of elements that will all be
    // offered. At least `count` of them are >= their count-th largest, so every key below that value is out.
    __device__ __forceinline__ void seed(u32 ok) {
        const u32 r = wave_kth_largest(ok, count);
        if (r > 0u) {
            const u64 t = ((u64)r << 32) - 1ull;
            if (t > thr) {
                set_thr(t);
                publish();
            }
        }
        if (s_top) {
            // the TOPN largest sample values are TOPN distinct elements of this wave
            const u64 sv = wave_sort_desc(((u64)ok << 32) | (u64)lane_id());
            if (lane_id() < TOPN) s_top[top_w * TOPN + lane_id()] = (u32)(sv >> 32);
        }
    }

    __device__ __forceinline__ void merge_sorted(u64 g_desc) {
        list = wave_merge_desc(list, g_desc);
        const u64 t = readlane64(list, count - 1);
        if (t > thr) set_thr(t);
    }
};

// ------------------------------------------------------------------------------------------------ cross-block hand-off
//
// Blocks of one row hand their partial results to the row's last block through device memory. The partials are
// written and read as relaxed atomics at agent scope (write-through, and reads that bypass the XCD-local L2), and each
// writer waits for its stores to complete before the block counts its arrival. This needs no L2 write-back or
// invalidation: a release/acquire fence at agent scope would write back and invalidate the whole L2 of the XCD in
// every block, which costs more than the streaming itself.

template <typename T>
__device__ __forceinline__ void st_agent(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ T ld_agent(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void st_agent_f2(float2* p, float2 v) {
    st_agent((u64*)p, ((u64)__float_as_uint(v.y) << 32) | __float_as_uint(v.x));
}

__device__ __forceinline__ float2 ld_agent_f2(const float2* p) {
    const u64 b = ld_agent((const u64*)p);
    return make_float2(__uint_as_float((u32)b), __uint_as_float((u32)(b >> 32)));
}

// Count this block's arrival at `counter` after its agent-scope stores have completed; true in every thread of the
// block that arrives last. The last block resets the counter to 0 for the next launch.
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned expected, unsigned* s_flag) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // every store of this thread has completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev == expected - 1;
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = last ? 1u : 0u;
    }
    __syncthreads();
    return *s_flag != 0u;
}

// The top 64 of the NW waves' descending lists, in wave 0 (other waves: unspecified), by a pairwise tree in LDS:
// ceil(log2(NW)) merge levels instead of NW - 1 merges on one wave. All threads of the block call it; s_list must not be
// in use by another wave when it is called.
template <int NW>
__device__ __forceinline__ u64 block_tree_merge(u64 acc, u64 (*s_list)[WAVE]) {
    const int w = threadIdx.x / WAVE, l = lane_id();
    s_list[w][l] = acc;
    __syncthreads();
#pragma unroll
    for (int a = NW; a > 1; a = (a + 1) / 2) {
        const int h = (a + 1) / 2;  // waves [0, a - h) take the list of wave w + h
        if (w < a - h) {
            acc = wave_merge_desc(acc, s_list[w + h][l]);
            if (h > 1) s_list[w][l] = acc;
        }
        if (h > 1) __syncthreads();
    }
    return acc;
}

// The last block's merge of `nl` descending 64-key lists at lists[i * 64 + lane] (agent-scope reads): each wave merges
// every NW-th list with the next list's load in flight, then wave 0 merges the waves' results. Returns the merged
// list in wave 0 (other waves: unspecified). All threads of the block call it. s_list: NW x 64 keys of LDS.
template <int NW>
__device__ __forceinline__ u64 block_merge_lists(const u64* lists, int nl, u64 (*s_list)[WAVE]) {
    const int w = threadIdx.x / WAVE, l = lane_id();
    // wave w's first four lists (w, w + NW, ...) are loaded at once, further ones one ahead of their merge
    constexpr int PRE = 4;
    u64 v[PRE];
#pragma unroll
    for (int k = 0; k < PRE; ++k) v[k] = w + k * NW < nl ? ld_agent(&lists[(size_t)(w + k * NW) * WAVE + l]) : 0ull;
    u64 acc = v[0];
#pragma unroll
    for (int k = 1; k < PRE; ++k)
        if (w + k * NW < nl) acc = wave_merge_desc(acc, v[k]);
    for (int o = w + PRE * NW; o < nl; o += NW) acc = wave_merge_desc(acc, ld_agent(&lists[(size_t)o * WAVE + l]));
    __syncthreads();
    return block_tree_merge<NW>(acc, s_list);
}

}  // namespace gbs
