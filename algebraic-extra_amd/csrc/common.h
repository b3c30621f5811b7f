// Shared device helpers for the algx gfx950 kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "algx.h"

namespace algx {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- errors
void set_error(const std::string& msg);
int32_t fail(const std::string& msg);
// Returns 0 after a launch that succeeded, else records the HIP error.
int32_t check_launch(const char* what);
// Fills n floats on stream s with a kernel (no memset node).
int32_t fill_f32(float* p, int64_t n, float value, hipStream_t s);

// HIP events armed by algx_set_probe for one kernel. A probed launch hands
// them to hipExtLaunchKernel, which records them as part of the kernel's own
// dispatch: timing inserts no extra packets (and no cache fences) between
// kernels, so the probed kernel runs as it does unprobed.
struct Probe {
  hipEvent_t start = nullptr, stop = nullptr;
  bool active() const { return start != nullptr; }
};
Probe probe_for(int which);

template <typename F, typename... Args>
void launch_k(const Probe& p, F kernel, dim3 grid, dim3 block, hipStream_t s, Args... args) {
  if (p.active())
    hipExtLaunchKernelGGL(kernel, grid, block, 0, s, p.start, p.stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
}

// ------------------------------------------------------------- scalar math
__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }

// Rounds through the storage type (identity for float32 storage).
template <typename T> __device__ __forceinline__ float round_to(float x) { return to_f(from_f<T>(x)); }

__device__ __forceinline__ float rsq(float x) { return __builtin_amdgcn_rsqf(x); }

// rho(x) = x + sqrt(1+x^2) without the reciprocal branch (flash.py:84-87).
__device__ __forceinline__ float rho_fast(float x, float& r) {
  float rad = __builtin_fmaf(x, x, 1.0f);
  r = rsq(rad);
  return __builtin_fmaf(rad, r, x);
}
// Stable rho: |x| + sqrt(1+x^2), reciprocal for x < 0 (flash.py:76-80).
__device__ __forceinline__ float rho_exact(float x, float& r) {
  float rad = __builtin_fmaf(x, x, 1.0f);
  r = rsq(rad);
  float t = __builtin_fmaf(rad, r, __builtin_fabsf(x));
  return x >= 0.0f ? t : __builtin_amdgcn_rcpf(t);
}
__device__ __forceinline__ float rho_var(float x, bool fast, float& r) {
  return fast ? rho_fast(x, r) : rho_exact(x, r);
}
// Bounded radical (radical.py:13-38): on |x| <= 1, x + sqrt(1+t) and
// r = 1/sqrt(1+t) as degree-4 polynomials in t = x^2 (Horner, the
// reference's float32 coefficients); outside, the stable exact radical. The
// reference picks the polynomial for a whole score tile whose max |x| is at
// most 1; here each score picks it for itself.
__device__ __forceinline__ float rho_poly(float x, float& r) {
  if (__builtin_fabsf(x) <= 1.0f) {
    const float t = x * x;
    float s = -.010264432643176741f;
    s = __builtin_fmaf(s, t, .04451694257534509f);
    s = __builtin_fmaf(s, t, -.11935047485233699f);
    s = __builtin_fmaf(s, t, .49927168521732207f);
    s = __builtin_fmaf(s, t, 1.0000227161113386f);
    float q = .05025262090029994f;
    q = __builtin_fmaf(q, t, -.1841886600636537f);
    q = __builtin_fmaf(q, t, .3364554110926816f);
    q = __builtin_fmaf(q, t, -.49515903732516475f);
    q = __builtin_fmaf(q, t, .9998514827226793f);
    r = q;
    return x + s;
  }
  return rho_exact(x, r);
}
// x^(2^log2n) by repeated squaring == int_pow for powers of two (flash.py:95-104).
__device__ __forceinline__ float pow2n(float x, int log2n) {
  for (int i = 0; i < log2n; ++i) x = x * x;
  return x;
}
// l^(-1/n): rsqrt followed by n/2 - 1 rsqrt-steps (flash.py:107-114).
__device__ __forceinline__ float inv_root(float l, int log2n) {
  float y = rsq(l);
  for (int k = 1; k < log2n; ++k) y = y * rsq(y);
  return y;
}

__host__ __device__ inline int ilog2(int n) {
  int k = 0;
  while ((1 << k) < n) ++k;
  return k;
}

// Selects the variant a guarded launch runs: guard == NULL -> low.
__device__ __forceinline__ bool guard_in_range(const int32_t* guard) {
  return guard == nullptr || guard[0] != 0;
}

}  // namespace algx
