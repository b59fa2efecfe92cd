// Exact integer arithmetic of the extended pipeline, device side. The definitions (the per-element penalty, the mass
// of a token, the exact products with an f32 fraction) are the pipeline's specification; each helper states it.
#pragma once
#include <hip/hip_fp16.h>
#include "gbs_common.hpp"

namespace gbs {
namespace modeu {

typedef unsigned __int128 u128;

constexpr u32 NEG_INF_KEY = 0x007fffffu;  // okey_f32(-inf)
constexpr u64 MASS_ONE = 1ull << 44;      // the mass of the row maximum

struct RowParamsDev {
    float temperature, top_p, min_p, repetition, presence, frequency;
    int top_k, reserved;
};
static_assert(sizeof(RowParamsDev) == 32, "GbsRowParams is 32 bytes");

__device__ __forceinline__ bool params_invalid(const RowParamsDev& p, float u) {
    bool bad = !(isfinite(p.temperature) && p.temperature >= 0.0f);
    bad |= !(p.top_p >= 0.0f && p.top_p <= 1.0f);
    bad |= !(p.min_p >= 0.0f && p.min_p <= 1.0f);
    bad |= !(isfinite(p.repetition) && p.repetition > 0.0f);
    bad |= !isfinite(p.presence) || !isfinite(p.frequency);
    bad |= p.top_k < 0;
    bad |= !(u >= 0.0f && u < 1.0f);
    return bad;
}

// penalties: if c > 0, l = (x > 0 ? x * rinv : x * rep) - ((float)c * freq + pres), each operation rounded to f32
__device__ __forceinline__ float penalize(float x, int c, float rinv, float rep, float freq, float pres) {
    if (c > 0) {
        float l = x > 0.0f ? x * rinv : x * rep;
        const float a = (float)c * freq;
        const float b = a + pres;
        return l - b;
    }
    return x;
}

// 2^f, f in [-0.5, 0.5]: degree-7 Taylor series of exp(f ln 2), Horner form in fused multiply-adds
__host__ __device__ __forceinline__ float pow2_frac(float f) {
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

// The integer mass of a token of logit l in a row of maximum M at c2 = log2(e) / T:
// 2^44 if l == M; else y = (l - M) * c2; 0 unless y >= -64; n = rint(y), f = y - n; m = (u32)(2^f * 2^24);
// mass = m * 2^(n + 20), truncated.
__device__ __forceinline__ u64 mass(float l, float M, float c2) {
    if (l == M) return MASS_ONE;
    const float d = l - M;
    const float y = d * c2;
    if (!(y >= -64.0f)) return 0ull;
    const float n = rintf(y);
    const float f = y - n;
    const float p = pow2_frac(f);
    const u32 m = (u32)(p * 16777216.0f);
    const int sh = (int)n + 20;
    if (sh >= 0) return (u64)m << sh;
    if (sh <= -32) return 0ull;
    return (u64)(m >> (-sh));
}

// 2^24 * pow2_frac(f), bit for bit: every coefficient of the Horner form scaled by 2^24 (a power of two, so each fused
// multiply-add rounds to exactly 2^24 times the unscaled one; no value comes near the subnormal or overflow range).
__host__ __device__ __forceinline__ float pow2_frac_2p24(float f) {
    float p = 1.52527338e-05f * 16777216.0f;
    p = fmaf(p, f, 1.54035304e-04f * 16777216.0f);
    p = fmaf(p, f, 1.33335581e-03f * 16777216.0f);
    p = fmaf(p, f, 9.61812911e-03f * 16777216.0f);
    p = fmaf(p, f, 5.55041087e-02f * 16777216.0f);
    p = fmaf(p, f, 2.40226507e-01f * 16777216.0f);
    p = fmaf(p, f, 6.93147181e-01f * 16777216.0f);
    p = fmaf(p, f, 16777216.0f);
    return p;
}

// mass() without branches or selections, for streaming sums. Preconditions: c2 and M finite, and l <= M or l = -inf
// (M is the maximum of the values it is applied to). Bit-identical to mass() there:
//  - y = (l - M) * c2 <= 0 is clamped at -51 (a NaN y cannot occur: l - M is never inf - inf). Every y < -25.5 has
//    mass 0 under mass() (n <= -26, and m < 2^25 is shifted right by >= 26 bits, or y < -64), and so has the clamped
//    y = -51: m = 2^24 shifted right by 31 bits.
//  - Otherwise n = rint(y) in [-51, 0], m = (u32)(2^24 * 2^f) < 2^25, and (m * 2^32) >> (12 - n) with a shift in
//    [12, 63] is m << (n + 20) for n + 20 >= 0 and m >> -(n + 20) below, as mass() computes.
//  - l == M gives y = 0 (c2 finite): n = 0, f = 0, m = 2^24 exactly, and 2^56 >> 12 = 2^44 = MASS_ONE.
__host__ __device__ __forceinline__ u64 mass_fast(float l, float M, float c2) {
    const float y = fmaxf((l - M) * c2, -51.0f);
    const float n = rintf(y);
    const u32 m = (u32)pow2_frac_2p24(y - n);
    const u32 s = (u32)(12 - (int)n);
    return ((u64)m << 32) >> s;
}

// whether mass_fast may stand for mass() over a row of maximum M at c2 (one test per row)
__host__ __device__ __forceinline__ bool mass_fast_ok(float M, float c2) { return __builtin_isfinite(M) && __builtin_isfinite(c2); }

__device__ __forceinline__ float temp_scale(float t) { return 1.44269504088896340736f / t; }

// floor(x * z) for finite x >= 0 (x < 2^23), exactly; *exact = the product was an integer
__device__ __forceinline__ u128 mul_floor(float x, u128 z, bool* exact) {
    const u32 b = __float_as_uint(x);
    const u32 e = (b >> 23) & 0xFFu;
    u64 m = b & 0x7FFFFFu;
    int sh;
    if (e == 0) sh = 149;
    else {
        m |= 0x800000u;
        sh = 150 - (int)e;
    }
    if (m == 0 || z == 0) {
        if (exact) *exact = true;
        return 0;
    }
    const u128 lo = (u128)m * (u64)z;
    const u128 hi = (u128)m * (u64)(z >> 64);
    u64 w0 = (u64)lo;
    const u128 mid = (lo >> 64) + (u64)hi;
    u64 w1 = (u64)mid;
    u64 w2 = (u64)((hi >> 64) + (mid >> 64));
    bool ex = true;
    int s = sh;
    while (s >= 64) {
        ex &= w0 == 0;
        w0 = w1;
        w1 = w2;
        w2 = 0;
        s -= 64;
    }
    if (s > 0) {
        ex &= (w0 & ((1ull << s) - 1)) == 0;
        w0 = (w0 >> s) | (w1 << (64 - s));
        w1 = (w1 >> s) | (w2 << (64 - s));
    }
    if (exact) *exact = ex;
    return ((u128)w1 << 64) | w0;
}

__device__ __forceinline__ u64 mul_ceil64(float x, u64 z) {
    bool ex;
    const u64 f = (u64)mul_floor(x, (u128)z, &ex);
    return f + (ex ? 0ull : 1ull);
}

// (max, sum of 2^((l - max) * c)) pairs: the online log-sum-exp, base 2
// The two 16-bit logits of a 32-bit word (low half first), widened exactly to f32: bf16 by a shift, fp16 by the
// conversion instruction (every fp16 value, NaN and infinities included, is an f32 value).
template <int DT>
__device__ __forceinline__ void widen2(u32 w, float& a, float& b) {
    if constexpr (DT == GBS_DTYPE_BF16) {
        a = __uint_as_float(w << 16);
        b = __uint_as_float(w & 0xFFFF0000u);
    } else {
        a = __half2float(__ushort_as_half((unsigned short)(w & 0xFFFFu)));
        b = __half2float(__ushort_as_half((unsigned short)(w >> 16)));
    }
}

template <int DT>
__device__ __forceinline__ float widen1(u32 h) {
    if constexpr (DT == GBS_DTYPE_BF16) return __uint_as_float(h << 16);
    else return __half2float(__ushort_as_half((unsigned short)h));
}

struct Lse {
    float m, s;
};

__device__ __forceinline__ Lse lse_merge(Lse a, Lse b, float c) {
    if (b.m == -INFINITY) return a;
    if (a.m == -INFINITY) return b;
    const float M = fmaxf(a.m, b.m);
    return Lse{M, a.s * exp2f((a.m - M) * c) + b.s * exp2f((b.m - M) * c)};
}

// The wave's total of per-lane online log-sum-exp pairs, in every lane: the maximum first, then each lane's sum
// rescaled to it once and summed (cross-lane moves by DPP and permlane swaps, no LDS). A lane at -inf adds 0.
__device__ __forceinline__ Lse wave_lse(Lse a, float c) {
    float M = a.m;
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) M = fmaxf(M, __uint_as_float(xor_lane(__float_as_uint(M), m)));
    float s = a.m == -INFINITY ? 0.0f : a.s * exp2f((a.m - M) * c);
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) s += __uint_as_float(xor_lane(__float_as_uint(s), m));
    return Lse{M, s};
}

}  // namespace modeu
}  // namespace gbs
