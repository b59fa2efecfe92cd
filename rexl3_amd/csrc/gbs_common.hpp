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
            const u64 o = shfl_xor64(v, j);
            const bool lower = (l & j) == 0;
            const bool desc = (l & k) == 0;
            const bool keep_max = (lower == desc);
            v = keep_max ? (v > o ? v : o) : (v < o ? v : o);
        }
    }
    return v;
}

// the 64 largest of two descending lists (one key per lane each), descending
__device__ __forceinline__ u64 wave_merge_desc(u64 a, u64 b_desc) {
    const int l = lane_id();
    const u64 br = shfl64(b_desc, WAVE - 1 - l);
    u64 v = a > br ? a : br;  // bitonic
#pragma unroll
    for (int j = WAVE / 2; j > 0; j >>= 1) {
        const u64 o = shfl_xor64(v, j);
        const bool lower = (l & j) == 0;
        v = lower ? (v > o ? v : o) : (v < o ? v : o);
    }
    return v;
}

// ascending bitonic sort of one u64 per lane
__device__ __forceinline__ u64 wave_sort_asc(u64 v) {
    const int l = lane_id();
#pragma unroll
    for (int k = 2; k <= WAVE; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const u64 o = shfl_xor64(v, j);
            const bool lower = (l & j) == 0;
            const bool asc = (l & k) == 0;
            const bool keep_min = (lower == asc);
            v = keep_min ? (v < o ? v : o) : (v > o ? v : o);
        }
    }
    return v;
}

__device__ __forceinline__ u64 wave_sum_u64(u64 v) {
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) v += shfl_xor64(v, m);
    return v;
}

// inclusive prefix sum over lanes
__device__ __forceinline__ u64 wave_scan_u64(u64 v) {
    const int l = lane_id();
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const u64 o = shfl64(v, l >= d ? l - d : l);
        if (l >= d) v += o;
    }
    return v;
}

__device__ __forceinline__ u32 wave_or(u32 v) {
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) v |= (u32)__shfl_xor((int)v, m, WAVE);
    return v;
}

// ------------------------------------------------------------------------------------------------ wave top list

// A wave's gated top list. `buf` is the wave's private LDS buffer of at least BUF keys.
template <int BUF>
struct WaveTop {
    u64 list;  // rank lane_id()
    u64 thr;   // key of rank count - 1 (wave-uniform); keys <= thr are dropped
    int n;     // buffered keys (wave-uniform)
    int count;
    u64* buf;

    __device__ __forceinline__ void init(u64* b, int cnt, u64 floor_key) {
        list = 0;
        thr = floor_key;
        n = 0;
        count = cnt;
        buf = b;
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

    // merge buffered keys, 64 at a time; `all` also merges a partial group
    __device__ __forceinline__ void flush(bool all) {
        if (n < WAVE && !(all && n > 0)) return;
        wave_lds_sync();
        const int l = lane_id();
        while (n >= WAVE || (all && n > 0)) {
            const int take = n < WAVE ? n : WAVE;
            const int base = n - take;
            u64 g = l < take ? buf[base + l] : 0ull;
            n = base;
            g = wave_sort_desc(g);
            list = wave_merge_desc(list, g);
            const u64 t = readlane64(list, count - 1);
            thr = t > thr ? t : thr;
        }
        wave_lds_sync();
    }

    __device__ __forceinline__ void merge_sorted(u64 g_desc) {
        list = wave_merge_desc(list, g_desc);
        const u64 t = readlane64(list, count - 1);
        thr = t > thr ? t : thr;
    }
};

// ------------------------------------------------------------------------------------------------ cross-block hand-off

// Release this block's global writes and count its arrival at `counter`; true in every thread of the block that
// arrives last (which then sees every other block's writes). The last block resets the counter to 0.
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned expected, unsigned* s_flag) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev == expected - 1;
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = last ? 1u : 0u;
    }
    __syncthreads();
    const bool last = *s_flag != 0u;
    if (last) __threadfence();
    return last;
}

}  // namespace gbs
