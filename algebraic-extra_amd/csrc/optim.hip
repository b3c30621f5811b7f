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
// * adamw: the Adam-family leaves' step (optimizers.py:222-226): m, v, the
//   bias-corrected update and the decayed parameter in one pass (reads p, g,
//   m, v; writes p, m, v: 28 bytes per element).
// * ns_normalize: X / sqrt(sum(X^2) + eps) per matrix, cast to the
//   Newton-Schulz input type (optimizers.py:44-45): per-block sums of squares
//   of each matrix, then one pass that reduces its matrix's partials (fixed
//   order, so every block forms the same norm) and writes the scaled copy.
//
// momentum / apply: each thread owns 4 consecutive elements (one 16-byte
// float32 vector); the last partial vector is done element by element.
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

__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, float b1,
                                           float b2, float c1, float c2, float eps, float decay,
                                           float lr) {
  m = b1 * m + (1.0f - b1) * g;
  v = b2 * v + (1.0f - b2) * (g * g);
  const float u = (m / c1) / (__builtin_sqrtf(v / c2) + eps);
  p = p * decay - lr * u;
}

__global__ __launch_bounds__(kThreads) void adamw_kernel(float* __restrict__ p,
                                                         const float* __restrict__ g,
                                                         float* __restrict__ m,
                                                         float* __restrict__ v, int64_t n, float b1,
                                                         float b2, float c1, float c2, float eps,
                                                         float decay, float lr) {
  const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
  if (i >= n) return;
  if (i + 4 <= n) {
    f32x4 pv = *reinterpret_cast<const f32x4*>(p + i);
    const f32x4 gv = *reinterpret_cast<const f32x4*>(g + i);
    f32x4 mv = *reinterpret_cast<const f32x4*>(m + i);
    f32x4 vv = *reinterpret_cast<const f32x4*>(v + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float pe = pv[e], me = mv[e], ve = vv[e];
      adamw_elem(pe, gv[e], me, ve, b1, b2, c1, c2, eps, decay, lr);
      pv[e] = pe;
      mv[e] = me;
      vv[e] = ve;
    }
    *reinterpret_cast<f32x4*>(p + i) = pv;
    *reinterpret_cast<f32x4*>(m + i) = mv;
    *reinterpret_cast<f32x4*>(v + i) = vv;
  } else {
    for (int64_t j = i; j < n; ++j) adamw_elem(p[j], g[j], m[j], v[j], b1, b2, c1, c2, eps, decay, lr);
  }
}

constexpr int kMaxNormBlocks = 256;  // partial sums per matrix

// Block (b, k): sum of squares of elements [b * span, (b + 1) * span) of
// matrix k, a fixed-order tree over the block's threads. VEC: 16-byte loads
// (mn and span multiples of 4, x 16-byte aligned).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void ns_sumsq_kernel(const float* __restrict__ x,
                                                            float* __restrict__ partial,
                                                            int64_t mn, int64_t span) {
  const int64_t k = blockIdx.y;
  const float* xk = x + k * mn;
  const int64_t lo = blockIdx.x * span;
  const int64_t hi = min(mn, lo + span);
  float s0 = 0.0f, s1 = 0.0f;
  if (VEC) {
    int64_t i = lo + 4 * threadIdx.x;
    // four 16-byte loads in flight per thread (hi - i is a multiple of 4)
    for (; i + 12 * kThreads < hi; i += 16 * kThreads) {
      f32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const f32x4*>(xk + i + 4 * kThreads * u);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        s0 = __builtin_fmaf(v[u][0], v[u][0], s0);
        s1 = __builtin_fmaf(v[u][1], v[u][1], s1);
        s0 = __builtin_fmaf(v[u][2], v[u][2], s0);
        s1 = __builtin_fmaf(v[u][3], v[u][3], s1);
      }
    }
    for (; i < hi; i += 4 * kThreads) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(xk + i);
      s0 = __builtin_fmaf(v[0], v[0], s0);
      s1 = __builtin_fmaf(v[1], v[1], s1);
      s0 = __builtin_fmaf(v[2], v[2], s0);
      s1 = __builtin_fmaf(v[3], v[3], s1);
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) s0 = __builtin_fmaf(xk[i], xk[i], s0);
  }
  __shared__ float red[kThreads];
  red[threadIdx.x] = s0 + s1;
  __syncthreads();
#pragma unroll
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[k * gridDim.x + blockIdx.x] = red[0];
}

// Block (b, k): norm of matrix k from its nb partials (the same fixed-order
// tree in every block of the matrix), then out = x / norm over the block's
// span, cast to T. VEC: 16-byte loads and 4-element stores.
template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void ns_scale_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ partial,
                                                            int nb, T* __restrict__ out,
                                                            int64_t mn, int64_t span, float eps) {
  const int64_t k = blockIdx.y;
  __shared__ float red[kMaxNormBlocks];
  red[threadIdx.x] = threadIdx.x < nb ? partial[k * nb + threadIdx.x] : 0.0f;
  __syncthreads();
#pragma unroll
  for (int w = kMaxNormBlocks / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  const float norm = __builtin_sqrtf(red[0] + eps);
  const float* xk = x + k * mn;
  T* ok = out + k * mn;
  const int64_t lo = blockIdx.x * span;
  const int64_t hi = min(mn, lo + span);
  if (VEC) {
    auto put = [&](int64_t i, const f32x4& v) {
      if (sizeof(T) == 2) {
        bf16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (bf16)(v[e] / norm);
        *reinterpret_cast<bf16x4*>(ok + i) = o;
      } else {
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = v[e] / norm;
        *reinterpret_cast<f32x4*>(ok + i) = o;
      }
    };
    int64_t i = lo + 4 * threadIdx.x;
    // four 16-byte loads in flight per thread (hi - i is a multiple of 4)
    for (; i + 12 * kThreads < hi; i += 16 * kThreads) {
      f32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const f32x4*>(xk + i + 4 * kThreads * u);
#pragma unroll
      for (int u = 0; u < 4; ++u) put(i + 4 * kThreads * u, v[u]);
    }
    for (; i < hi; i += 4 * kThreads) put(i, *reinterpret_cast<const f32x4*>(xk + i));
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) ok[i] = from_f<T>(xk[i] / norm);
  }
}

int64_t blocks_of(int64_t n) { return (n + 4 * kThreads - 1) / (4 * kThreads); }

// Blocks per matrix of the normalisation: ~2048 blocks over the batch, at
// most kMaxNormBlocks per matrix and at least 4096 elements per block.
int norm_blocks(int64_t K, int64_t mn) {
  int64_t nb = (2048 + K - 1) / K;
  const int64_t cap = (mn + 4095) / 4096;
  if (nb > cap) nb = cap;
  if (nb > kMaxNormBlocks) nb = kMaxNormBlocks;
  return (int)(nb < 1 ? 1 : nb);
}

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

extern "C" int64_t algx_ns_normalize_workspace_bytes(int64_t K, int64_t MN) {
  if (K <= 0 || MN <= 0) return 0;
  return K * norm_blocks(K, MN) * (int64_t)sizeof(float);
}

extern "C" int32_t algx_ns_normalize(const float* x, void* out, int64_t K, int64_t MN,
                                     int32_t out_dtype, float eps, void* workspace,
                                     void* stream) {
  if (K < 0 || MN < 0) return fail("ns_normalize: negative size");
  if (out_dtype != ALGX_BF16 && out_dtype != ALGX_F32)
    return fail("ns_normalize: out must be bf16 or f32");
  if (!(eps >= 0.0f)) return fail("ns_normalize: eps must be non-negative");
  if (K == 0 || MN == 0) return 0;
  if (K > 65535) return fail("ns_normalize: at most 65535 matrices");
  if (x == nullptr || out == nullptr || workspace == nullptr) return fail("ns_normalize: null pointer");
  const int nb = norm_blocks(K, MN);
  const bool vec = MN % 4 == 0 && aligned16(x) && ((uintptr_t)out & (out_dtype == ALGX_BF16 ? 7 : 15)) == 0;
  int64_t span = (MN + nb - 1) / nb;
  if (vec) span = (span + 3) / 4 * 4;
  hipStream_t s = (hipStream_t)stream;
  float* partial = (float*)workspace;
  const dim3 grid((uint32_t)nb, (uint32_t)K);
  if (vec)
    hipLaunchKernelGGL(ns_sumsq_kernel<true>, grid, dim3(kThreads), 0, s, x, partial, MN, span);
  else
    hipLaunchKernelGGL(ns_sumsq_kernel<false>, grid, dim3(kThreads), 0, s, x, partial, MN, span);
  if (int32_t rc = check_launch("ns_sumsq")) return rc;
  static_assert(kMaxNormBlocks == kThreads, "one partial per thread in the norm reduction");
  if (out_dtype == ALGX_BF16) {
    if (vec)
      hipLaunchKernelGGL((ns_scale_kernel<bf16, true>), grid, dim3(kThreads), 0, s, x, partial, nb,
                         (bf16*)out, MN, span, eps);
    else
      hipLaunchKernelGGL((ns_scale_kernel<bf16, false>), grid, dim3(kThreads), 0, s, x, partial, nb,
                         (bf16*)out, MN, span, eps);
  } else {
    if (vec)
      hipLaunchKernelGGL((ns_scale_kernel<float, true>), grid, dim3(kThreads), 0, s, x, partial, nb,
                         (float*)out, MN, span, eps);
    else
      hipLaunchKernelGGL((ns_scale_kernel<float, false>), grid, dim3(kThreads), 0, s, x, partial, nb,
                         (float*)out, MN, span, eps);
  }
  return check_launch("ns_scale");
}

extern "C" int32_t algx_adamw_step(float* p, const float* g, float* m, float* v, int64_t n,
                                  float b1, float b2, float c1, float c2, float eps, float decay,
                                  float lr, void* stream) {
  if (n < 0) return fail("adamw_step: negative size");
  if (n == 0) return 0;
  if (p == nullptr || g == nullptr || m == nullptr || v == nullptr) return fail("adamw_step: null pointer");
  if (!aligned16(p) || !aligned16(g) || !aligned16(m) || !aligned16(v))
    return fail("adamw_step: pointers must be 16-byte aligned");
  if (blocks_of(n) >= ((int64_t)1 << 31)) return fail("adamw_step: too many elements");
  hipLaunchKernelGGL(adamw_kernel, dim3((uint32_t)blocks_of(n)), dim3(kThreads), 0,
                     (hipStream_t)stream, p, g, m, v, n, b1, b2, c1, c2, eps, decay, lr);
  return check_launch("adamw_step");
}
