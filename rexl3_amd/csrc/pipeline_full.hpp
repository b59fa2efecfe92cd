// Internal (not exported) launcher of the extended pipeline's full-distribution path (pipeline_full.hip).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace gbs {
// The control region at the start of every gbs_sample_rows workspace, at offsets that depend only on the row (room for
// 65536 rows): three u32 arrival counters per row, zero between launches (the single-pass kernel's split form uses the
// first, the full path all three), then one u32 per row that the single-pass kernel sets, under per-row dispatch, for
// the rows it leaves to the full path. Partial results come after it.
constexpr size_t SAMPLE_CTL_BYTES = (size_t)4 * 65536 * 4;
constexpr size_t SAMPLE_DEFER_OFFSET = (size_t)3 * 65536 * 4;

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
