// Attention kernel-side variant and the per-element weight math shared by
// the generic (scalar) and the MFMA kernels.
#pragma once

#include "common.h"

namespace algx {

// Kernel form of algx_attn_variant (flash.py:59-73).
struct KVariant {
  int kind;      // ALGX_SOFTMAX / ALGX_ASINH
  int log2n;     // n = 2^log2n
  int shift;     // running-max accumulation (asinh) -- softmax always shifts
  int fast;      // fast rho
  int inv_stat;  // unshifted statistic 1/l
  int bounded;   // no score clamp
  int precise;   // write float32 output too
  float clamp;
  float slope;   // n for asinh, 1 for softmax (flash.py:430, :441)
  int poly;      // bounded radical (radical.py:26-38)
};

// rho and its slope factor r of the variant (flash.py:91-92).
__device__ __forceinline__ float rho_of(const KVariant& v, float x, float& r) {
  return v.poly ? rho_poly(x, r) : rho_var(x, v.fast, r);
}

constexpr float kNeg = -1e4f;           // flash.py:55
constexpr float kLog2e = 1.4426950408889634f;

// Backward weight p and d(logit)/ds factor r for one score (flash.py:339-361).
// Returns p; writes ds-multiplier (r or 1) to rr and whether the clamp kink
// zeroes the score gradient to keep.
__device__ __forceinline__ float bwd_weight(const KVariant& v, float s, float stat, float& rr,
                                            bool& keep) {
  keep = true;
  if (v.kind == ALGX_SOFTMAX) {
    rr = 1.0f;
    return __expf(s - stat);
  }
  float x = s;
  if (!v.shift && !v.bounded) {
    x = __builtin_fminf(s, v.clamp);
    keep = s < v.clamp;
  }
  float r;
  float rh = rho_of(v, x, r);
  rr = r;
  return v.inv_stat ? pow2n(rh, v.log2n) * stat : pow2n(rh * stat, v.log2n);
}

// Initial row state from the sink (flash.py:197-214): (m, l).
__device__ __forceinline__ void sink_init(const KVariant& v, bool has_sink, float b, float& m,
                                          float& l) {
  if (v.kind == ALGX_ASINH && !v.shift) {
    m = 0.0f;
    if (has_sink) {
      float x = v.bounded ? b : __builtin_fminf(b, v.clamp);
      float r;
      l = pow2n(rho_of(v, x, r), v.log2n);
    } else {
      l = 0.0f;
    }
    return;
  }
  m = has_sink ? b : kNeg;
  l = has_sink ? 1.0f : 0.0f;
}

// Final statistic (flash.py:275-280).
__device__ __forceinline__ float final_stat(const KVariant& v, float m, float l) {
  if (v.kind == ALGX_SOFTMAX) return m + __logf(l);
  if (!v.shift) return v.inv_stat ? 1.0f / l : inv_root(l, v.log2n);
  float r;
  return rho_exact(-m, r) * inv_root(l, v.log2n);
}

// Sink probability mass and slope (flash.py:694-705): contribution to dsink
// of one row is -mass * di * slope.
__device__ __forceinline__ float sink_grad_term(const KVariant& v, float b, float stat, float di) {
  if (v.kind == ALGX_SOFTMAX) return -__expf(b - stat) * di;
  const bool clipped = !v.shift && !v.bounded;
  const float bb = clipped ? __builtin_fminf(b, v.clamp) : b;
  float r;
  const float rh = v.poly ? rho_poly(bb, r) : rho_exact(bb, r);
  const float mass = v.inv_stat ? pow2n(rh, v.log2n) * stat : pow2n(rh * stat, v.log2n);
  float slope = v.slope * r;
  if (clipped && !(b < v.clamp)) slope = 0.0f;
  return -mass * di * slope;
}

}  // namespace algx
