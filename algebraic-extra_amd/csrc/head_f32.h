// Float32 fused-head path (head_f32.hip), dispatched from the head's C entry
// points when the hidden states are float32.
#pragma once

#include "common.h"

namespace algx {

int64_t head_f32_fwd_workspace(int N, int V);
int64_t head_f32_bwd_workspace(int N, int V);
int32_t head_f32_fwd(const float* h, const float* E, const int32_t* targets, float* stat,
                     float* zt, float* partial, int N, int d, int V, int kind, int log2n,
                     float inv_c, float clamp, hipStream_t s);
int32_t head_f32_bwd(const float* h, const float* E, const int32_t* targets, const float* stat,
                     const float* scale, float* dh, float* dE, float* dz, int N, int d, int V,
                     int kind, int log2n, float inv_c, float clamp, hipStream_t s);

}  // namespace algx
