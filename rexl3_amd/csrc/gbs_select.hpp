// Block-level exact selection over a chunk of one logits row (f32 / bf16 / fp16), shared by the top-k drop-ins and
// the fused keyed sampler. See gbs_common.hpp for the key order and the wave lists.
#pragma once
#include "gbs_common.hpp"

namespace gbs {
namespace sel {

constexpr int NT = 256;
constexpr int NW = NT / WAVE;
constexpr int BUF = 2 * WAVE;  // < 64 keys left after a flush + one key per lane

enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

template <int DT>
__device__ __forceinline__ u32 elem_key(const void* row, int e) {
    if (DT == DT_F32) return okey_f32_nanlow(((const float*)row)[e]);
    if (DT == DT_BF16) return okey_16<false>(((const u16*)row)[e]);
    return okey_16<true>(((const u16*)row)[e]);
}

// four order keys (high words) of elements e..e+3; `vec` = 16-byte (f32) / 8-byte (16-bit) loads are legal
template <int DT>
__device__ __forceinline__ void load_group(const void* row, int e, int hi, bool vec, u32 (&k)[4], bool (&in)[4]) {
    if (vec && e + 4 <= hi) {
        if (DT == DT_F32) {
            const float4 v = *(const float4*)((const float*)row + e);
            k[0] = okey_f32_nanlow(v.x); k[1] = okey_f32_nanlow(v.y); k[2] = okey_f32_nanlow(v.z); k[3] = okey_f32_nanlow(v.w);
        } else {
            const uint2 v = *(const uint2*)((const u16*)row + e);
            k[0] = okey_16<DT == DT_F16>(v.x); k[1] = okey_16<DT == DT_F16>(v.x >> 16);
            k[2] = okey_16<DT == DT_F16>(v.y); k[3] = okey_16<DT == DT_F16>(v.y >> 16);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) in[q] = true;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            in[q] = e + q < hi;
            k[q] = in[q] ? elem_key<DT>(row, e + q) : 0u;
        }
    }
}

// Streams [lo, hi) of `row` (block-cyclic 4-element groups) through the block's wave lists; leaves the block's best 64
// (sorted, best first) in wave 0's `list`. `count` <= 64.
template <int DT>
__device__ void block_select(const void* row, int lo, int hi, bool vec, int count, WaveTop<BUF>& wt, u64 (*s_list)[WAVE]) {
    const int tid = threadIdx.x;
    const int w = tid / WAVE;
    const int step = NT * 4;
    int e = lo + tid * 4;
    u32 k[4], kn[4];
    bool in[4], inn[4];
    load_group<DT>(row, e, hi, vec, k, in);
    // every lane of a wave runs the same number of steps: lanes past the end offer nothing
    const int wave_first = lo + w * WAVE * 4;
    const int nsteps = wave_first < hi ? (hi - wave_first + step - 1) / step : 0;
    for (int s = 0; s < nsteps; ++s) {
        const int en = e + step;
        load_group<DT>(row, en, hi, vec, kn, inn);
#pragma unroll
        for (int q = 0; q < 4; ++q) wt.offer(in[q] ? make_key(k[q], (u32)(e + q)) : 0ull), wt.flush(false);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            k[q] = kn[q];
            in[q] = inn[q];
        }
        e = en;
    }
    wt.flush(true);
    s_list[w][lane_id()] = wt.list;
    __syncthreads();
    if (w == 0) {
        for (int o = 1; o < NW; ++o) wt.merge_sorted(s_list[o][lane_id()]);
    }
}

}  // namespace sel
}  // namespace gbs
