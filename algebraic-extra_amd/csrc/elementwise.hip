// The model's elementwise algebraic ops around the attention path
// (algebraic.py:76-117): RMS normalisation of d_model-wide rows with an
// optional float32 gain (rms_norm; no gain is the parameter-free AVN) and the
// algebraic linear unit alu(x) = x/2 (1 + bx / sqrt(1 + b^2 x^2)) with its
// custom VJP, plus the model's gated product gate * alu(up) fused into one
// pass (model.py:186-191).
//
// All of it is HBM-bound: one pass over the operands with 16-byte accesses.
// A norm row belongs to one wave (its D/8 bf16 or D/4 f32 chunks spread over
// the 64 lanes), so the row sums are wave reductions. dgain is reduced per
// workgroup into a workspace row and finished per column in a fixed order
// (deterministic).
#include <initializer_list>

#include "common.h"

namespace algx {

namespace {

constexpr int kFwdThreads = 256;
constexpr int kBwdThreads = 1024;
constexpr int kBwdWaves = kBwdThreads / 64;
constexpr int kMaxD = 2048;
constexpr int kMaxBwdBlocks = 512;
constexpr int kEltThreads = 256;

template <typename T> struct Vec;
template <> struct Vec<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct Vec<float> { typedef f32x4 type; static constexpr int n = 4; };

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Gain values of this lane's chunks (1 where there is no gain).
template <int CPL, int EPL>
__device__ __forceinline__ void load_gain(const float* gain, int lane, int nch,
                                          float (&g)[CPL][EPL]) {
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      g[c][e] = (gain != nullptr && ch < nch) ? gain[ch * EPL + e] : 1.0f;
  }
}

// y = cast((x * tau) * gain), tau = rsqrt(mean(x^2) + eps) (algebraic.py:76-83).
// One row per wave; CPL = 16-byte chunks per lane. With a residual r the row
// is first x = cast(x + r) (the block's residual add, model.py:177, :191),
// written to xsum, and normalised.
template <typename T, int CPL>
__global__ __launch_bounds__(kFwdThreads) void rmsnorm_fwd_kernel(const T* __restrict__ x,
                                                                  const float* __restrict__ gain,
                                                                  T* __restrict__ y, int64_t rows,
                                                                  int D, float eps,
                                                                  const T* __restrict__ r,
                                                                  T* __restrict__ xsum) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  const int lane = threadIdx.x & 63;
  const int nch = D / EPL;
  float g[CPL][EPL];
  load_gain<CPL, EPL>(gain, lane, nch, g);
  const int64_t stride = (int64_t)gridDim.x * (kFwdThreads / 64);
  const float inv_d = 1.0f / (float)D;
  for (int64_t row = (int64_t)blockIdx.x * (kFwdThreads / 64) + (threadIdx.x >> 6); row < rows;
       row += stride) {
    const T* xr = x + row * D;
    VT in[CPL];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        in[c] = *reinterpret_cast<const VT*>(xr + ch * EPL);
        if (r != nullptr) {
          const VT rv = *reinterpret_cast<const VT*>(r + row * D + ch * EPL);
#pragma unroll
          for (int e = 0; e < EPL; ++e) in[c][e] = from_f<T>(to_f(in[c][e]) + to_f(rv[e]));
          *reinterpret_cast<VT*>(xsum + row * D + ch * EPL) = in[c];
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float f = to_f(in[c][e]);
          ss = __builtin_fmaf(f, f, ss);
        }
      }
    }
    const float tau = rsq(wave_sum(ss) * inv_d + eps);
    T* yr = y + row * D;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        VT out;
#pragma unroll
        for (int e = 0; e < EPL; ++e) out[e] = from_f<T>((to_f(in[c][e]) * tau) * g[c][e]);
        *reinterpret_cast<VT*>(yr + ch * EPL) = out;
      }
    }
  }
}

// Input VJP of rms_norm (autodiff of algebraic.py:76-83 through mean/rsqrt):
//   dx = tau * gain * dy - x * tau^3 * sum(dy * gain * x) / D
// and, given `partial` ([gridDim.x][D] float32), each workgroup's share of
//   dgain = sum_rows dy * x * tau.
// With dres (the gradient reaching the normalised input along the residual
// stream) the output is cast(cast(dx) + dres): autograd's sum of the two
// gradients of the residual sum, rounded as it rounds.
template <typename T, int CPL>
__global__ __launch_bounds__(kBwdThreads) void rmsnorm_bwd_kernel(
    const T* __restrict__ x, const float* __restrict__ gain, const T* __restrict__ dy,
    T* __restrict__ dx, float* __restrict__ partial, int64_t rows, int D, float eps,
    const T* __restrict__ dres) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  // One row of column sums per wave, as wide as the widest row this
  // instantiation takes (64 KB at CPL * EPL = 16).
  __shared__ float red[kBwdWaves][64 * CPL * EPL];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nch = D / EPL;
  float g[CPL][EPL], dg[CPL][EPL];
  load_gain<CPL, EPL>(gain, lane, nch, g);
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int e = 0; e < EPL; ++e) dg[c][e] = 0.0f;
  const int64_t stride = (int64_t)gridDim.x * kBwdWaves;
  const float inv_d = 1.0f / (float)D;
  for (int64_t row = (int64_t)blockIdx.x * kBwdWaves + w; row < rows; row += stride) {
    VT xi[CPL], gi[CPL];
    float ss = 0.0f, dot = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        xi[c] = *reinterpret_cast<const VT*>(x + row * D + ch * EPL);
        gi[c] = *reinterpret_cast<const VT*>(dy + row * D + ch * EPL);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float xf = to_f(xi[c][e]);
          ss = __builtin_fmaf(xf, xf, ss);
          dot = __builtin_fmaf(to_f(gi[c][e]) * g[c][e], xf, dot);
        }
      }
    }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    const float tau = rsq(ss * inv_d + eps);
    const float cfac = tau * tau * tau * dot * inv_d;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        VT out;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float xf = to_f(xi[c][e]), df = to_f(gi[c][e]);
          out[e] = from_f<T>(tau * g[c][e] * df - cfac * xf);
          dg[c][e] = __builtin_fmaf(df, xf * tau, dg[c][e]);
        }
        if (dres != nullptr) {
          const VT rv = *reinterpret_cast<const VT*>(dres + row * D + ch * EPL);
#pragma unroll
          for (int e = 0; e < EPL; ++e) out[e] = from_f<T>(to_f(out[e]) + to_f(rv[e]));
        }
        *reinterpret_cast<VT*>(dx + row * D + ch * EPL) = out;
      }
    }
  }
  if (partial == nullptr) return;
  // Workgroup share of dgain: the waves' column sums added in wave order.
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nch)
#pragma unroll
      for (int e = 0; e < EPL; ++e) red[w][ch * EPL + e] = dg[c][e];
  }
  __syncthreads();
  for (int col = threadIdx.x; col < D; col += kBwdThreads) {
    float s = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kBwdWaves; ++ww) s += red[ww][col];
    partial[(int64_t)blockIdx.x * D + col] = s;
  }
}

// dgain[col] = sum of the workgroup partials: 64 columns per workgroup of
// 1024 threads, 16 interleaved slices of the partial rows per column (many
// independent loads in flight), combined in slice order (deterministic).
__global__ __launch_bounds__(1024) void rmsnorm_gain_finish(const float* __restrict__ partial,
                                                            int nparts, int D,
                                                            float* __restrict__ dgain) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, slice = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float s0 = 0.0f, s1 = 0.0f;
  if (col < D) {
    int r = slice;
    for (; r + 16 < nparts; r += 32) {
      s0 += partial[(int64_t)r * D + col];
      s1 += partial[(int64_t)(r + 16) * D + col];
    }
    if (r < nparts) s0 += partial[(int64_t)r * D + col];
  }
  red[slice][lane] = s0 + s1;
  __syncthreads();
  if (slice == 0 && col < D) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += red[i][lane];
    dgain[col] = s;
  }
}

// alu in float32 (algebraic.py:86-93): u = bz r, r = rsqrt(1 + (bz)^2),
// alu = z/2 (1 + u) with 1 + u taken as r^2 / (1 - u) for bz < 0 so the
// negative tail keeps its relative precision.
__device__ __forceinline__ float alu_parts(float z, float beta, float& u, float& r) {
  const float bz = beta * z;
  r = rsq(__builtin_fmaf(bz, bz, 1.0f));
  u = bz * r;
  const float one_plus_u =
      bz < 0.0f ? (r * r) * __builtin_amdgcn_rcpf(1.0f - u) : 1.0f + u;
  return 0.5f * z * one_plus_u;
}
// d alu / dz = (1 + u)/2 + u r^2 / 2 (algebraic.py:109-111), with its one
// fused multiply-add written out: hipcc contracts a * b + c wherever it finds
// one, and which products it finds depends on what the caller shares with
// alu_parts, so an implicit form rounds differently in the fused and the plain
// backward kernels. (1 + u)/2 = 1/2 + u/2 exactly.
__device__ __forceinline__ float alu_deriv(float u, float r) {
  const float h = 0.5f * u;
  return __builtin_fmaf(h, r * r, 0.5f + h);
}

// GLU = 0: y = cast(alu(a)).
// GLU = 1: y = cast(b * cast(alu(a))), a = up, b = gate (model.py:186-191).
template <typename T, int GLU>
__global__ __launch_bounds__(kEltThreads) void alu_fwd_kernel(const T* __restrict__ a,
                                                              const T* __restrict__ b,
                                                              T* __restrict__ y, int64_t n,
                                                              float beta) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  const int64_t nvec = n / EPL;
  for (int64_t i = (int64_t)blockIdx.x * kEltThreads + threadIdx.x; i < nvec;
       i += (int64_t)gridDim.x * kEltThreads) {
    const VT av = reinterpret_cast<const VT*>(a)[i];
    VT bv;
    if (GLU) bv = reinterpret_cast<const VT*>(b)[i];
    VT out;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float u, r;
      const float act = round_to<T>(alu_parts(to_f(av[e]), beta, u, r));
      out[e] = from_f<T>(GLU ? to_f(bv[e]) * act : act);
    }
    reinterpret_cast<VT*>(y)[i] = out;
  }
  // n % EPL trailing elements, one per thread of the first workgroup.
  const int64_t t = nvec * EPL + threadIdx.x;
  if (blockIdx.x == 0 && t < n) {
    float u, r;
    const float act = round_to<T>(alu_parts(to_f(a[t]), beta, u, r));
    y[t] = from_f<T>(GLU ? to_f(b[t]) * act : act);
  }
}

// GLU = 0: da = cast(dy * alu'(a)) (algebraic.py:108-112).
// GLU = 1, out = b * act with act = cast(alu(a)):
//   db = cast(dy * act), da = cast(cast(dy * b) * alu'(a)).
template <typename T, int GLU>
__global__ __launch_bounds__(kEltThreads) void alu_bwd_kernel(const T* __restrict__ a,
                                                              const T* __restrict__ b,
                                                              const T* __restrict__ dy,
                                                              T* __restrict__ da,
                                                              T* __restrict__ db, int64_t n,
                                                              float beta) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  const int64_t nvec = n / EPL;
  for (int64_t i = (int64_t)blockIdx.x * kEltThreads + threadIdx.x; i < nvec;
       i += (int64_t)gridDim.x * kEltThreads) {
    const VT av = reinterpret_cast<const VT*>(a)[i];
    const VT gv = reinterpret_cast<const VT*>(dy)[i];
    VT bv;
    if (GLU) bv = reinterpret_cast<const VT*>(b)[i];
    VT oa, ob;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float u, r;
      const float g = to_f(gv[e]);
      if (GLU) {
        const float act = round_to<T>(alu_parts(to_f(av[e]), beta, u, r));
        const float gact = round_to<T>(g * to_f(bv[e]));
        oa[e] = from_f<T>(gact * alu_deriv(u, r));
        ob[e] = from_f<T>(g * act);
      } else {
        const float bz = beta * to_f(av[e]);
        r = rsq(__builtin_fmaf(bz, bz, 1.0f));
        u = bz * r;
        oa[e] = from_f<T>(g * alu_deriv(u, r));
      }
    }
    reinterpret_cast<VT*>(da)[i] = oa;
    if (GLU) reinterpret_cast<VT*>(db)[i] = ob;
  }
  const int64_t t = nvec * EPL + threadIdx.x;
  if (blockIdx.x == 0 && t < n) {
    float u, r;
    const float act = round_to<T>(alu_parts(to_f(a[t]), beta, u, r));
    const float g = to_f(dy[t]);
    if (GLU) {
      da[t] = from_f<T>(round_to<T>(g * to_f(b[t])) * alu_deriv(u, r));
      db[t] = from_f<T>(g * act);
    } else {
      da[t] = from_f<T>(g * alu_deriv(u, r));
    }
  }
}

int fwd_blocks(int64_t rows) {
  const int64_t per = kFwdThreads / 64;
  int64_t nb = (rows + per - 1) / per;
  return (int)(nb > 8192 ? 8192 : nb);
}

int bwd_blocks(int64_t rows) {
  int64_t nb = (rows + kBwdWaves - 1) / kBwdWaves;
  return (int)(nb > kMaxBwdBlocks ? kMaxBwdBlocks : nb);
}

// One 16-byte vector per thread and no grid-stride loop (up to 2^30 groups):
// workgroups then sweep the operands in address order, which streams from HBM
// faster than a capped grid striding over the whole range.
int elt_blocks(int64_t nvec) {
  int64_t nb = (nvec + kEltThreads - 1) / kEltThreads;
  return (int)(nb > (1 << 30) ? (1 << 30) : nb);
}

int epl_of(int dtype) { return dtype == ALGX_BF16 ? 8 : 4; }

int32_t check_norm(const void* x, int64_t rows, int32_t D, int32_t dtype, float eps) {
  if (dtype != ALGX_BF16 && dtype != ALGX_F32) return fail("rms_norm: dtype must be bf16 or f32");
  if (rows < 0) return fail("rms_norm: negative row count");
  if (D <= 0 || D > kMaxD || D % epl_of(dtype))
    return fail("rms_norm: D must be a multiple of 8 (bf16) or 4 (f32), at most 2048");
  if (!(eps > 0.0f)) return fail("rms_norm: eps must be positive");
  if (rows > 0 && x == nullptr) return fail("rms_norm: null input");
  return 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int32_t check_alu(const void* a, int64_t n, int32_t dtype) {
  if (dtype != ALGX_BF16 && dtype != ALGX_F32) return fail("alu: dtype must be bf16 or f32");
  if (n < 0) return fail("alu: negative element count");
  if (n > 0 && a == nullptr) return fail("alu: null input");
  return 0;
}

// The 16-byte vector accesses need 16-byte aligned operands.
int32_t check_aligned(std::initializer_list<const void*> ps, const char* what) {
  for (const void* p : ps)
    if (!aligned16(p)) return fail(std::string(what) + ": operands must be 16-byte aligned");
  return 0;
}

template <typename T, int CPL>
void launch_norm_fwd(const void* x, const float* gain, void* y, int64_t rows, int D, float eps,
                     const void* r, void* xsum, hipStream_t s) {
  launch_k(probe_for(ALGX_PROBE_RMSNORM_FWD), rmsnorm_fwd_kernel<T, CPL>, dim3(fwd_blocks(rows)),
           dim3(kFwdThreads), s, (const T*)x, gain, (T*)y, rows, D, eps, (const T*)r, (T*)xsum);
}

template <typename T, int CPL>
void launch_norm_bwd(const void* x, const float* gain, const void* dy, void* dx, float* partial,
                     int64_t rows, int D, float eps, const void* dres, hipStream_t s) {
  launch_k(probe_for(ALGX_PROBE_RMSNORM_BWD), rmsnorm_bwd_kernel<T, CPL>, dim3(bwd_blocks(rows)),
           dim3(kBwdThreads), s, (const T*)x, gain, (const T*)dy, (T*)dx, partial, rows, D, eps,
           (const T*)dres);
}

}  // namespace
}  // namespace algx

using namespace algx;

namespace {

int32_t norm_fwd_impl(const void* x, const void* r, const float* gain, void* xsum, void* y,
                      int64_t rows, int32_t D, int32_t dtype, float eps, hipStream_t s) {
  if (int32_t rc = check_norm(x, rows, D, dtype, eps)) return rc;
  if (rows == 0) return 0;
  if (y == nullptr) return fail("rms_norm: null output");
  if (r != nullptr && xsum == nullptr) return fail("rms_norm: the residual sum needs xsum");
  if (int32_t rc = check_aligned({x, y}, "rms_norm")) return rc;
  if (r != nullptr)
    if (int32_t rc = check_aligned({r, xsum}, "rms_norm")) return rc;
  // Chunks per lane: ceil(D / (16-byte elements) / 64).
  const int cpl = (D / epl_of(dtype) + 63) / 64;
  if (dtype == ALGX_BF16) {
    switch (cpl) {
      case 1: launch_norm_fwd<bf16, 1>(x, gain, y, rows, D, eps, r, xsum, s); break;
      case 2: launch_norm_fwd<bf16, 2>(x, gain, y, rows, D, eps, r, xsum, s); break;
      case 3: launch_norm_fwd<bf16, 3>(x, gain, y, rows, D, eps, r, xsum, s); break;
      default: launch_norm_fwd<bf16, 4>(x, gain, y, rows, D, eps, r, xsum, s); break;
    }
  } else {
    switch (cpl) {
      case 1: launch_norm_fwd<float, 1>(x, gain, y, rows, D, eps, r, xsum, s); break;
      case 2: launch_norm_fwd<float, 2>(x, gain, y, rows, D, eps, r, xsum, s); break;
      case 3: launch_norm_fwd<float, 3>(x, gain, y, rows, D, eps, r, xsum, s); break;
      case 4: launch_norm_fwd<float, 4>(x, gain, y, rows, D, eps, r, xsum, s); break;
      case 5: case 6: launch_norm_fwd<float, 6>(x, gain, y, rows, D, eps, r, xsum, s); break;
      default: launch_norm_fwd<float, 8>(x, gain, y, rows, D, eps, r, xsum, s); break;
    }
  }
  return check_launch("rms_norm_fwd");
}

int32_t norm_bwd_impl(const void* x, const float* gain, const void* dy, const void* dres,
                      void* dx, float* dgain, void* workspace, int64_t rows, int32_t D,
                      int32_t dtype, float eps, hipStream_t s) {
  if (int32_t rc = check_norm(x, rows, D, dtype, eps)) return rc;
  if ((gain == nullptr) != (dgain == nullptr))
    return fail("rms_norm: dgain is required exactly when gain is given");
  if (rows == 0) return dgain != nullptr ? fill_f32(dgain, D, 0.0f, s) : 0;
  if (dy == nullptr || dx == nullptr) return fail("rms_norm: null dy/dx");
  if (gain != nullptr && workspace == nullptr) return fail("rms_norm: null workspace");
  if (int32_t rc = check_aligned({x, dy, dx}, "rms_norm")) return rc;
  if (dres != nullptr)
    if (int32_t rc = check_aligned({dres}, "rms_norm")) return rc;
  float* partial = gain != nullptr ? (float*)workspace : nullptr;
  const int cpl = (D / epl_of(dtype) + 63) / 64;
  if (dtype == ALGX_BF16) {
    switch (cpl) {
      case 1: launch_norm_bwd<bf16, 1>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
      case 2: launch_norm_bwd<bf16, 2>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
      case 3: launch_norm_bwd<bf16, 3>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
      default: launch_norm_bwd<bf16, 4>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
    }
  } else {
    switch (cpl) {
      case 1: launch_norm_bwd<float, 1>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
      case 2: launch_norm_bwd<float, 2>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
      case 3: launch_norm_bwd<float, 3>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
      case 4: launch_norm_bwd<float, 4>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
      case 5: case 6: launch_norm_bwd<float, 6>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
      default: launch_norm_bwd<float, 8>(x, gain, dy, dx, partial, rows, D, eps, dres, s); break;
    }
  }
  if (int32_t rc = check_launch("rms_norm_bwd")) return rc;
  if (gain == nullptr) return 0;
  rmsnorm_gain_finish<<<(D + 63) / 64, 1024, 0, s>>>(partial, bwd_blocks(rows), D, dgain);
  return check_launch("rms_norm_gain_finish");
}

}  // namespace

extern "C" int32_t algx_rms_norm_fwd(const void* x, const float* gain, void* y, int64_t rows,
                                     int32_t D, int32_t dtype, float eps, void* stream) {
  return norm_fwd_impl(x, nullptr, gain, nullptr, y, rows, D, dtype, eps, (hipStream_t)stream);
}

extern "C" int32_t algx_add_rms_norm_fwd(const void* x, const void* r, const float* gain,
                                         void* xsum, void* y, int64_t rows, int32_t D,
                                         int32_t dtype, float eps, void* stream) {
  if (rows > 0 && r == nullptr) return fail("add_rms_norm: null residual");
  return norm_fwd_impl(x, r, gain, xsum, y, rows, D, dtype, eps, (hipStream_t)stream);
}

extern "C" int64_t algx_rms_norm_bwd_workspace_bytes(int64_t rows, int32_t D, int32_t dtype) {
  (void)dtype;
  if (rows <= 0 || D <= 0) return 0;
  return (int64_t)bwd_blocks(rows) * D * (int64_t)sizeof(float);
}

extern "C" int32_t algx_rms_norm_bwd(const void* x, const float* gain, const void* dy, void* dx,
                                     float* dgain, void* workspace, int64_t rows, int32_t D,
                                     int32_t dtype, float eps, void* stream) {
  return norm_bwd_impl(x, gain, dy, nullptr, dx, dgain, workspace, rows, D, dtype, eps,
                       (hipStream_t)stream);
}

extern "C" int32_t algx_add_rms_norm_bwd(const void* xsum, const float* gain, const void* dy,
                                         const void* dres, void* dx, float* dgain,
                                         void* workspace, int64_t rows, int32_t D, int32_t dtype,
                                         float eps, void* stream) {
  if (rows > 0 && dres == nullptr) return fail("add_rms_norm: null residual gradient");
  return norm_bwd_impl(xsum, gain, dy, dres, dx, dgain, workspace, rows, D, dtype, eps,
                       (hipStream_t)stream);
}

namespace {

template <typename T>
int32_t alu_fwd_any(const void* up, const void* gate, void* y, int64_t n, float beta,
                    hipStream_t s) {
  const int64_t nvec = (n + Vec<T>::n - 1) / Vec<T>::n;
  const Probe probe = probe_for(ALGX_PROBE_ALU_FWD);
  if (gate == nullptr)
    launch_k(probe, alu_fwd_kernel<T, 0>, dim3(elt_blocks(nvec)), dim3(kEltThreads), s,
             (const T*)up, (const T*)nullptr, (T*)y, n, beta);
  else
    launch_k(probe, alu_fwd_kernel<T, 1>, dim3(elt_blocks(nvec)), dim3(kEltThreads), s,
             (const T*)up, (const T*)gate, (T*)y, n, beta);
  return check_launch("alu_fwd");
}

template <typename T>
int32_t alu_bwd_any(const void* up, const void* gate, const void* dy, void* dup, void* dgate,
                    int64_t n, float beta, hipStream_t s) {
  const int64_t nvec = (n + Vec<T>::n - 1) / Vec<T>::n;
  const Probe probe = probe_for(ALGX_PROBE_ALU_BWD);
  if (gate == nullptr)
    launch_k(probe, alu_bwd_kernel<T, 0>, dim3(elt_blocks(nvec)), dim3(kEltThreads), s,
             (const T*)up, (const T*)nullptr, (const T*)dy, (T*)dup, (T*)nullptr, n, beta);
  else
    launch_k(probe, alu_bwd_kernel<T, 1>, dim3(elt_blocks(nvec)), dim3(kEltThreads), s,
             (const T*)up, (const T*)gate, (const T*)dy, (T*)dup, (T*)dgate, n, beta);
  return check_launch("alu_bwd");
}

}  // namespace

extern "C" int32_t algx_alu_fwd(const void* x, void* y, int64_t n, int32_t dtype, float beta,
                                void* stream) {
  if (int32_t rc = check_alu(x, n, dtype)) return rc;
  if (n == 0) return 0;
  if (y == nullptr) return fail("alu: null output");
  if (int32_t rc = check_aligned({x, y}, "alu")) return rc;
  hipStream_t s = (hipStream_t)stream;
  return dtype == ALGX_BF16 ? alu_fwd_any<bf16>(x, nullptr, y, n, beta, s)
                            : alu_fwd_any<float>(x, nullptr, y, n, beta, s);
}

extern "C" int32_t algx_alu_bwd(const void* x, const void* dy, void* dx, int64_t n, int32_t dtype,
                                float beta, void* stream) {
  if (int32_t rc = check_alu(x, n, dtype)) return rc;
  if (n == 0) return 0;
  if (dy == nullptr || dx == nullptr) return fail("alu: null dy/dx");
  if (int32_t rc = check_aligned({x, dy, dx}, "alu")) return rc;
  hipStream_t s = (hipStream_t)stream;
  return dtype == ALGX_BF16 ? alu_bwd_any<bf16>(x, nullptr, dy, dx, nullptr, n, beta, s)
                            : alu_bwd_any<float>(x, nullptr, dy, dx, nullptr, n, beta, s);
}

extern "C" int32_t algx_alu_glu_fwd(const void* gate, const void* up, void* out, int64_t n,
                                    int32_t dtype, float beta, void* stream) {
  if (int32_t rc = check_alu(up, n, dtype)) return rc;
  if (n == 0) return 0;
  if (gate == nullptr || out == nullptr) return fail("alu_glu: null gate/output");
  if (int32_t rc = check_aligned({gate, up, out}, "alu_glu")) return rc;
  hipStream_t s = (hipStream_t)stream;
  return dtype == ALGX_BF16 ? alu_fwd_any<bf16>(up, gate, out, n, beta, s)
                            : alu_fwd_any<float>(up, gate, out, n, beta, s);
}

extern "C" int32_t algx_alu_glu_bwd(const void* gate, const void* up, const void* dout,
                                    void* dgate, void* dup, int64_t n, int32_t dtype, float beta,
                                    void* stream) {
  if (int32_t rc = check_alu(up, n, dtype)) return rc;
  if (n == 0) return 0;
  if (gate == nullptr || dout == nullptr || dgate == nullptr || dup == nullptr)
    return fail("alu_glu: null gate/dout/dgate/dup");
  if (int32_t rc = check_aligned({gate, up, dout, dgate, dup}, "alu_glu")) return rc;
  hipStream_t s = (hipStream_t)stream;
  return dtype == ALGX_BF16 ? alu_bwd_any<bf16>(up, gate, dout, dup, dgate, n, beta, s)
                            : alu_bwd_any<float>(up, gate, dout, dup, dgate, n, beta, s);
}

// ---------------------------------------------------------------------------
// Gated feed-forward on the packed projection [gate | up] (rows x 2 cols):
// the model's gate and up GEMMs (model.py:184-185) as one GEMM against
// [w_g | w_u], and the gated product read straight from its output rows.
// ACT = ALGX_GLU_ALU: gate * alu(up) exactly as algx_alu_glu_*;
// ACT = ALGX_GLU_SILU: gate * silu(up), silu(x) = x * sigmoid(x)
// (standard.py:12-13) with sigmoid rounded to dtype before the product as the
// reference's bf16 ops round; its VJP uses sigma + x sigma (1 - sigma) in
// float32.
namespace algx {
namespace {

__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

template <typename T, int ACT>
__global__ __launch_bounds__(kEltThreads) void glu_packed_fwd_kernel(const T* __restrict__ gu,
                                                                     T* __restrict__ y,
                                                                     int64_t nvec, int nvr,
                                                                     int cols, float beta) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  const int64_t i = (int64_t)blockIdx.x * kEltThreads + threadIdx.x;
  if (i >= nvec) return;
  const int64_t r = i / nvr;
  const int c = (int)(i - r * nvr) * EPL;
  const VT gv = *reinterpret_cast<const VT*>(gu + r * 2 * cols + c);
  const VT uv = *reinterpret_cast<const VT*>(gu + r * 2 * cols + cols + c);
  VT out;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float up = to_f(uv[e]);
    float act;
    if (ACT == ALGX_GLU_ALU) {
      float u, rr;
      act = round_to<T>(alu_parts(up, beta, u, rr));
    } else {
      act = round_to<T>(up * round_to<T>(sigmoid_f(up)));
    }
    out[e] = from_f<T>(to_f(gv[e]) * act);
  }
  *reinterpret_cast<VT*>(y + r * cols + c) = out;
}

template <typename T, int ACT>
__global__ __launch_bounds__(kEltThreads) void glu_packed_bwd_kernel(const T* __restrict__ gu,
                                                                     const T* __restrict__ dy,
                                                                     T* __restrict__ dgu,
                                                                     int64_t nvec, int nvr,
                                                                     int cols, float beta) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  const int64_t i = (int64_t)blockIdx.x * kEltThreads + threadIdx.x;
  if (i >= nvec) return;
  const int64_t r = i / nvr;
  const int c = (int)(i - r * nvr) * EPL;
  const VT gv = *reinterpret_cast<const VT*>(gu + r * 2 * cols + c);
  const VT uv = *reinterpret_cast<const VT*>(gu + r * 2 * cols + cols + c);
  const VT dv = *reinterpret_cast<const VT*>(dy + r * cols + c);
  VT dg, du;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float up = to_f(uv[e]), g = to_f(dv[e]);
    const float gact = round_to<T>(g * to_f(gv[e]));
    float act, deriv;
    if (ACT == ALGX_GLU_ALU) {
      float u, rr;
      act = round_to<T>(alu_parts(up, beta, u, rr));
      deriv = alu_deriv(u, rr);
    } else {
      const float sg = sigmoid_f(up);
      act = round_to<T>(up * round_to<T>(sg));
      deriv = __builtin_fmaf(up * sg, 1.0f - sg, sg);
    }
    dg[e] = from_f<T>(g * act);
    du[e] = from_f<T>(gact * deriv);
  }
  *reinterpret_cast<VT*>(dgu + r * 2 * cols + c) = dg;
  *reinterpret_cast<VT*>(dgu + r * 2 * cols + cols + c) = du;
}

int32_t check_packed(const void* gu, int64_t rows, int32_t cols, int32_t act, int32_t dtype) {
  if (dtype != ALGX_BF16 && dtype != ALGX_F32) return fail("glu_packed: dtype must be bf16 or f32");
  if (act != ALGX_GLU_ALU && act != ALGX_GLU_SILU) return fail("glu_packed: unknown activation");
  if (rows < 0 || cols <= 0 || cols % epl_of(dtype))
    return fail("glu_packed: cols must be a positive multiple of 8 (bf16) or 4 (f32)");
  if (rows > 0 && gu == nullptr) return fail("glu_packed: null input");
  return 0;
}

template <typename T>
void glu_packed_fwd_any(const void* gu, void* y, int64_t rows, int cols, int act, float beta,
                        hipStream_t s) {
  const int nvr = cols / Vec<T>::n;
  const int64_t nvec = rows * nvr;
  const dim3 grid((unsigned)((nvec + kEltThreads - 1) / kEltThreads));
  const Probe probe = probe_for(ALGX_PROBE_ALU_FWD);
  if (act == ALGX_GLU_ALU)
    launch_k(probe, glu_packed_fwd_kernel<T, ALGX_GLU_ALU>, grid, dim3(kEltThreads), s,
             (const T*)gu, (T*)y, nvec, nvr, cols, beta);
  else
    launch_k(probe, glu_packed_fwd_kernel<T, ALGX_GLU_SILU>, grid, dim3(kEltThreads), s,
             (const T*)gu, (T*)y, nvec, nvr, cols, beta);
}

template <typename T>
void glu_packed_bwd_any(const void* gu, const void* dy, void* dgu, int64_t rows, int cols, int act,
                        float beta, hipStream_t s) {
  const int nvr = cols / Vec<T>::n;
  const int64_t nvec = rows * nvr;
  const dim3 grid((unsigned)((nvec + kEltThreads - 1) / kEltThreads));
  const Probe probe = probe_for(ALGX_PROBE_ALU_BWD);
  if (act == ALGX_GLU_ALU)
    launch_k(probe, glu_packed_bwd_kernel<T, ALGX_GLU_ALU>, grid, dim3(kEltThreads), s,
             (const T*)gu, (const T*)dy, (T*)dgu, nvec, nvr, cols, beta);
  else
    launch_k(probe, glu_packed_bwd_kernel<T, ALGX_GLU_SILU>, grid, dim3(kEltThreads), s,
             (const T*)gu, (const T*)dy, (T*)dgu, nvec, nvr, cols, beta);
}

}  // namespace
}  // namespace algx

extern "C" int32_t algx_glu_packed_fwd(const void* gu, void* y, int64_t rows, int32_t cols,
                                       int32_t act, int32_t dtype, float beta, void* stream) {
  if (int32_t rc = check_packed(gu, rows, cols, act, dtype)) return rc;
  if (rows == 0) return 0;
  if (y == nullptr) return fail("glu_packed: null output");
  if (int32_t rc = check_aligned({gu, y}, "glu_packed")) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ALGX_BF16) glu_packed_fwd_any<bf16>(gu, y, rows, cols, act, beta, s);
  else glu_packed_fwd_any<float>(gu, y, rows, cols, act, beta, s);
  return check_launch("glu_packed_fwd");
}

extern "C" int32_t algx_glu_packed_bwd(const void* gu, const void* dy, void* dgu, int64_t rows,
                                       int32_t cols, int32_t act, int32_t dtype, float beta,
                                       void* stream) {
  if (int32_t rc = check_packed(gu, rows, cols, act, dtype)) return rc;
  if (rows == 0) return 0;
  if (dy == nullptr || dgu == nullptr) return fail("glu_packed: null dy/dgu");
  if (int32_t rc = check_aligned({gu, dy, dgu}, "glu_packed")) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ALGX_BF16) glu_packed_bwd_any<bf16>(gu, dy, dgu, rows, cols, act, beta, s);
  else glu_packed_bwd_any<float>(gu, dy, dgu, rows, cols, act, beta, s);
  return check_launch("glu_packed_bwd");
}
