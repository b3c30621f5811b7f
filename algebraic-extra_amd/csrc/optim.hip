// Muon's elementwise steps around Newton-Schulz (optimizers.py:200-204) as
// single passes over float32 parameter state:
//
// * momentum: m <- mu m + (1 - mu) g, look = (1 - mu) g + mu m (the updated
//   m): the Nesterov look-ahead that Newton-Schulz orthogonalises. Reads g, m;
//   writes m, look (16 bytes per element, where four separate tensor ops move
//   40).
// * apply: p <- p * decay - step * o for the orthogonalised update o (bf16 or
//   float32), step = lr times the aspect factor of newton_schulz_5. Reads p,
//   o; writes p.
//
// Each thread owns 4 consecutive elements (one 16-byte float32 vector); the
// last partial vector is done element by element.
#include "common.h"

namespace algx {

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void muon_momentum_kernel(const float* __restrict__ g,
                                                                 float* __restrict__ m,
                                                                 float* __restrict__ look,
                                                                 int64_t n, float mu) {
  const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
  if (i >= n) return;
  const float a = 1.0f - mu;
  if (i + 4 <= n) {
    const f32x4 gv = *reinterpret_cast<const f32x4*>(g + i);
    const f32x4 mv = *reinterpret_cast<const f32x4*>(m + i);
    f32x4 mn, lk;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mn[e] = mu * mv[e] + a * gv[e];
      lk[e] = a * gv[e] + mu * mn[e];
    }
    *reinterpret_cast<f32x4*>(m + i) = mn;
    *reinterpret_cast<f32x4*>(look + i) = lk;
  } else {
    for (int64_t j = i; j < n; ++j) {
      const float mn = mu * m[j] + a * g[j];
      m[j] = mn;
      look[j] = a * g[j] + mu * mn;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void muon_apply_kernel(float* __restrict__ p,
                                                              const T* __restrict__ o, int64_t n,
                                                              float decay, float step) {
  const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
  if (i >= n) return;
  if (i + 4 <= n) {
    f32x4 pv = *reinterpret_cast<const f32x4*>(p + i);
    float ov[4];
    if (sizeof(T) == 2) {
      const bf16x4 ob = *reinterpret_cast<const bf16x4*>(o + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = (float)ob[e];
    } else {
      const f32x4 of = *reinterpret_cast<const f32x4*>(o + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = of[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) pv[e] = pv[e] * decay - step * ov[e];
    *reinterpret_cast<f32x4*>(p + i) = pv;
  } else {
    for (int64_t j = i; j < n; ++j) p[j] = p[j] * decay - step * to_f(o[j]);
  }
}

int64_t blocks_of(int64_t n) { return (n + 4 * kThreads - 1) / (4 * kThreads); }

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int32_t algx_muon_momentum(const float* g, float* m, float* look, int64_t n, float mu,
                                      void* stream) {
  if (n < 0) return fail("muon_momentum: negative size");
  if (n == 0) return 0;
  if (g == nullptr || m == nullptr || look == nullptr) return fail("muon_momentum: null pointer");
  if (!aligned16(g) || !aligned16(m) || !aligned16(look))
    return fail("muon_momentum: pointers must be 16-byte aligned");
  if (blocks_of(n) >= ((int64_t)1 << 31)) return fail("muon_momentum: too many elements");
  hipLaunchKernelGGL(muon_momentum_kernel, dim3((uint32_t)blocks_of(n)), dim3(kThreads), 0,
                     (hipStream_t)stream, g, m, look, n, mu);
  return check_launch("muon_momentum");
}

extern "C" int32_t algx_muon_apply(float* p, const void* o, int64_t n, int32_t o_dtype,
                                   float decay, float step, void* stream) {
  if (n < 0) return fail("muon_apply: negative size");
  if (o_dtype != ALGX_BF16 && o_dtype != ALGX_F32) return fail("muon_apply: o must be bf16 or f32");
  if (n == 0) return 0;
  if (p == nullptr || o == nullptr) return fail("muon_apply: null pointer");
  if (!aligned16(p) || ((uintptr_t)o & (o_dtype == ALGX_BF16 ? 7 : 15)))
    return fail("muon_apply: p must be 16-byte and o 8-byte (bf16) or 16-byte (f32) aligned");
  if (blocks_of(n) >= ((int64_t)1 << 31)) return fail("muon_apply: too many elements");
  hipStream_t s = (hipStream_t)stream;
  if (o_dtype == ALGX_BF16)
    hipLaunchKernelGGL(muon_apply_kernel<bf16>, dim3((uint32_t)blocks_of(n)), dim3(kThreads), 0,
                       s, p, (const bf16*)o, n, decay, step);
  else
    hipLaunchKernelGGL(muon_apply_kernel<float>, dim3((uint32_t)blocks_of(n)), dim3(kThreads), 0,
                       s, p, (const float*)o, n, decay, step);
  return check_launch("muon_apply");
}
