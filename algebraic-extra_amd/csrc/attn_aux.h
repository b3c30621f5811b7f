// Host-side launchers shared by the attention entry points.
#pragma once

#include "attn_common.h"

namespace algx {

int32_t guard_words();
// q_s = cast(q * q_scale); with a guard buffer also the range-guard word.
int32_t launch_prepare(const void* q, const void* k, const void* v, const float* sink, void* q_s,
                       int32_t* guard, int B, int H, int T, int D, int dtype, float q_scale,
                       float bound, float vmax, hipStream_t s);
// Guard word from `nblocks` triples of partial maxima (|q_s|^2, |k|^2, |v|).
int32_t launch_guard_finish(const float* partial, int nblocks, const float* sink, int H,
                            float bound, float vmax, int32_t* guard, hipStream_t s);
// Row pre-pass of the backward: di (and the sink gradient), and the dQ
// accumulator cleared when dq_acc is given.
int32_t launch_bwd_pre(const void* dout, const void* o, const float* o_precise,
                       const float* stat, const float* sink, float* di, float* dq_acc,
                       float* dsink, int B, int H, int T, int D, int dtype, const KVariant& low,
                       const KVariant& high, const int32_t* guard, hipStream_t s);
int32_t launch_dq_finish(const float* acc, void* dq, int64_t n, int dtype, const KVariant& low,
                         const KVariant& high, const int32_t* guard, float q_scale,
                         hipStream_t s);

// Generic kernels: any T, D in {16, 32, 64}, bf16 or f32, every variant.
int32_t launch_fwd_generic(const void* q_s, const void* k, const void* v, const float* sink,
                           void* o, float* o_precise, float* stat, int B, int H, int T, int D,
                           int dtype, const KVariant& var, const int32_t* guard, int want_low,
                           hipStream_t s);
int32_t launch_bwd_generic(const void* q, const void* k, const void* v, const float* stat,
                           const float* di, const void* dout, void* dq, void* dk, void* dv,
                           int B, int H, int T, int D, int dtype, float q_scale,
                           const KVariant& var, const int32_t* guard, int want_low,
                           hipStream_t s);

// MFMA kernels: bf16, D = 64, T % 128 == 0.
bool mfma_supported(int T, int D, int dtype);
// One launch per call: with a guard word the kernel runs `lo` or `hi` for the
// whole grid; without one it runs `lo`.
int32_t launch_fwd_mfma(const void* q_s, const void* k, const void* v, const float* sink,
                        void* o, float* o_precise, float* stat, int B, int H, int T,
                        const KVariant& lo, const KVariant& hi, const int32_t* guard,
                        hipStream_t s);
// Pre-scale, guard and forward in one pass over q (MFMA shapes): the low
// variant runs over the whole grid writing q_s and, guarded, one triple of
// partial maxima per workgroup (fwd_fused_partials of them); a second launch
// reduces them to the guard word and, out of range only, runs the high
// variant. dq_zero (or null): the backward's dQ accumulator, cleared in the
// same pass.
int64_t fwd_fused_partials(int B, int H, int T);
int32_t launch_fwd_fused(const void* q, const void* k, const void* v, const float* sink,
                         void* q_s, void* o, float* o_precise, float* stat, int32_t* guard,
                         float* partial, float* dq_zero, int B, int H, int T, float q_scale,
                         float bound, float vmax, const KVariant& lo, const KVariant& hi,
                         hipStream_t s);
int32_t launch_bwd_mfma(const void* q_s, const void* k, const void* v, const float* stat,
                        const float* di, const void* dout, float* dq_acc, void* dk, void* dv,
                        int B, int H, int T, const KVariant& lo, const KVariant& hi,
                        const int32_t* guard, hipStream_t s);

}  // namespace algx
