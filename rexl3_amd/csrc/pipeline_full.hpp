// Internal (not exported) launcher of the extended pipeline's full-distribution path (pipeline_full.hip).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace gbs {
// The control region at the start of every gbs_sample_rows workspace, at offsets that depend only on the row (room for
// 65536 rows): three u32 arrival counters per row, zero between launches (the single-pass kernel's split form uses the
// first, the full path all three), then one u32 per row that the single-pass kernel sets, under per-row dispatch, for
// the rows it leaves to the full path, then the full path's per-row record (FsRow), which the single-pass kernel fills
// for the rows it flags. Partial results come after it.
constexpr size_t SAMPLE_DEFER_OFFSET = (size_t)3 * 65536 * 4;
constexpr size_t SAMPLE_FSROW_OFFSET = (size_t)4 * 65536 * 4;

// The full path's per-row record: the row's maximum key, its log-sum-exp pair, and the state of the binned cut
// (FS_CUT: the cut continues; FS_DONE: the row's results are written; FS_RADIX: the single-block kernel takes the row),
// its crossing bin, the mass above it and P. Pass 0 writes it, or the single-pass kernel for the rows it flags.
enum : uint32_t { FS_CUT = 0, FS_DONE = 1, FS_RADIX = 2 };
struct FsRow {
    uint64_t top;
    float lse_m, lse_s;
    uint32_t nallowed, state, bstar, pad;
    uint64_t above, P;
};
constexpr uint32_t FS_NBINS = 52 * 128;  // the binned cut's bins (bstar = FS_NBINS: no cut, every bin kept)
constexpr size_t SAMPLE_CTL_BYTES = SAMPLE_FSROW_OFFSET + (size_t)65536 * sizeof(FsRow);

// workspace bytes of the full-distribution path, the control region included (a cleared workspace serves launches of
// any shape, as the fast path's)
size_t sample_full_workspace_bytes(int rows, int vocab);
// the full path's workspace when it serves the rows flagged by per-row dispatch
size_t sample_full_deferred_workspace_bytes(int rows, int vocab);
// `row_flags` (may be null): only the rows whose flag is non-zero are sampled, the others are left as they are
int launch_sample_full(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts, const uint32_t* mask,
                       const void* params, const float* uniforms, int* out_ids, int* out_greedy, float* out_probs, float* out_logprobs,
                       int* out_status, void* ws, size_t ws_bytes, void* stream, const unsigned* row_flags = nullptr);
}
