// Internal (not exported) launcher of the extended pipeline's full-distribution path (pipeline_full.hip).
#pragma once
#include <stdint.h>

namespace gbs {
int launch_sample_full(const void* logits, int dtype, int rows, int stride, int vocab, const int32_t* counts, const uint32_t* mask,
                       const void* params, const float* uniforms, int* out_ids, int* out_greedy, float* out_probs, float* out_logprobs,
                       int* out_status, void* stream);
}
