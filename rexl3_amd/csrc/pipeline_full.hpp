// Internal (not exported) launcher of the extended pipeline's full-distribution path (pipeline_full.hip).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace gbs {
// workspace bytes of the full-distribution path (a cleared workspace serves launches of any shape, as the fast path's)
size_t sample_full_workspace_bytes(int rows, int vocab);
int launch_sample_full(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts, const uint32_t* mask,
                       const void* params, const float* uniforms, int* out_ids, int* out_greedy, float* out_probs, float* out_logprobs,
                       int* out_status, void* ws, size_t ws_bytes, void* stream);
}
