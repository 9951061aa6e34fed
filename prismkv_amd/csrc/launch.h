// Host-side launchers shared between translation units of the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prismkv {

// Route pass 1 (moment scoring, route.hip): logits [G][4][3008] and chunk
// statistics [G][94][4][2] for `groups` KV groups, enqueued on `stream`.
void launch_route_score(const uint16_t* q, const float* moments, const int* counts, float* logits, float* stats,
                        int groups, hipStream_t stream);

}  // namespace prismkv
