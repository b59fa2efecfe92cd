// Block-level exact selection over a chunk of one logits row (f32 / bf16 / fp16), shared by the top-k drop-ins and
// the fused keyed sampler. See gbs_common.hpp for the key order and the wave lists.
#pragma once
#include <type_traits>

#include "gbs_common.hpp"

namespace gbs {
namespace sel {

constexpr int NT = 256;
constexpr int NW = NT / WAVE;
constexpr int BUF = WAVE * (4 + 1);  // < 64 keys left after a flush + 4 keys per lane of one group

enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

template <int DT>
__device__ __forceinline__ u32 elem_key(const void* row, int e) {
    if (DT == DT_F32) return okey_f32_nanlow(((const float*)row)[e]);
    if (DT == DT_BF16) return okey_16<false>(((const u16*)row)[e]);
    return okey_16<true>(((const u16*)row)[e]);
}

constexpr int SEL_GROUPS = 4;  // 4-element groups per lane per step of the main loop

template <int DT>
struct SelRaw {
    typename std::conditional<DT == DT_F32, u32x4, u32x2>::type x[SEL_GROUPS];
};

template <int DT>
__device__ __forceinline__ void sel_load(const void* row, int e, SelRaw<DT>& r) {
#pragma unroll
    for (int j = 0; j < SEL_GROUPS; ++j) {
        const int eg = e + j * NT * 4;
        if constexpr (DT == DT_F32) r.x[j] = __builtin_nontemporal_load((const u32x4*)((const float*)row + eg));
        else r.x[j] = __builtin_nontemporal_load((const u32x2*)((const u16*)row + eg));
    }
}

template <int DT>
__device__ __forceinline__ void sel_keys(const SelRaw<DT>& r, int j, u32 (&k)[4]) {
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

// Streams [lo, hi) of `row` through the block's wave lists; leaves the block's best 64 (sorted, best first) in wave 0's
// `list`. Main loop: SEL_GROUPS 4-element groups per lane per step, every one in bounds, the next step's loads issued
// before the current step is ranked; then a guarded tail of one group per lane per round. `count` <= 64.
template <int DT>
__device__ void block_select(const void* row, int lo, int hi, bool vec, int count, WaveTop<BUF>& wt, u64 (*s_list)[WAVE]) {
    const int tid = threadIdx.x;
    int e0 = lo;
    if (vec) {
        const int step = NT * 4 * SEL_GROUPS;
        const int nfull = (hi - lo) / step;
        if (nfull > 0) {
            SelRaw<DT> b0, b1;
            int e = lo + tid * 4;
            sel_load<DT>(row, e, b0);
            {
                u32 m = 0;
#pragma unroll
                for (int j = 0; j < SEL_GROUPS; ++j) {
                    u32 k[4];
                    sel_keys<DT>(b0, j, k);
#pragma unroll
                    for (int q = 0; q < 4; ++q) m = k[q] > m ? k[q] : m;
                }
                wt.seed(m);
            }
            // one step: every key of the step, one gate test per key folded into one scalar mask, one branch into
            // the (rare) offer path
            auto step_fn = [&](const SelRaw<DT>& B, int e) {
                u32 k[SEL_GROUPS * 4];
#pragma unroll
                for (int j = 0; j < SEL_GROUPS; ++j) {
                    u32 kj[4];
                    sel_keys<DT>(B, j, kj);
#pragma unroll
                    for (int q = 0; q < 4; ++q) k[j * 4 + q] = kj[q];
                }
                const u32 g = wt.gate;
                u64 anyp = 0;
#pragma unroll
                for (int i = 0; i < SEL_GROUPS * 4; ++i) anyp |= ballot(k[i] >= g);
                if (anyp) {
#pragma unroll
                    for (int j = 0; j < SEL_GROUPS; ++j) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) wt.offer_ok(k[j * 4 + q], (u32)(e + j * NT * 4 + q));
                        wt.flush(false);
                    }
                }
            };
            // two register buffers in turn: no buffer copy forces its loads to complete early
            for (int s = 0; s < nfull; s += 2) {
                sel_load<DT>(row, s + 1 < nfull ? e + step : e, b1);
                step_fn(b0, e);
                if (s + 1 >= nfull) break;
                sel_load<DT>(row, s + 2 < nfull ? e + 2 * step : e, b0);
                step_fn(b1, e + step);
                e += 2 * step;
            }
        }
        e0 = lo + nfull * step;
    }
    const int rounds = (hi - e0 + NT * 4 - 1) / (NT * 4);
    for (int r = 0; r < rounds; ++r) {
        const int eg = e0 + r * NT * 4 + tid * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) wt.offer_ok(eg + q < hi ? elem_key<DT>(row, eg + q) : 0u, (u32)(eg + q), eg + q < hi);
        wt.flush(false);
    }
    wt.flush(true);
    wt.list = block_tree_merge<NW>(wt.list, s_list);
}

}  // namespace sel
}  // namespace gbs
