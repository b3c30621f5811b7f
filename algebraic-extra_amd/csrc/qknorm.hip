// QK RMS normalisation over rows of 64 values with a float32 gain.
//
// Forward: y = cast(x * rsqrt(mean(x^2) + eps) * gain)  (algebraic.py:76-83)
// Backward: dx = tau*g*dy - tau^3 * x * sum(dy*g*x)/D   (native VJP, qk_norm.py:42-43)
//           dgain = sum_rows dy * x * tau               (qk_norm.py:20-26, :55)
//
// Single pass over HBM: each row is split over LPR lanes that each move one
// 16-byte vector (8 bf16 or 4 f32); the row sum of squares is combined with
// xor-shuffles inside the LPR-lane group. dgain is reduced per block into a
// workspace row and summed by a finishing kernel with one block per column
// (deterministic).
#include "common.h"

namespace algx {

namespace {

constexpr int kD = 64;
constexpr int kThreads = 256;
constexpr int kMaxBlocks = 2048;

template <typename T> struct Vec;
template <> struct Vec<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct Vec<float> { typedef f32x4 type; static constexpr int n = 4; };

template <int LPR> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < LPR; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void qknorm_fwd_kernel(const T* __restrict__ x,
                                                              const float* __restrict__ gain,
                                                              T* __restrict__ y, int64_t rows,
                                                              float eps) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  constexpr int LPR = kD / EPL;
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane % LPR, rw = lane / LPR;
  float g[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) g[i] = gain[sub * EPL + i];
  const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * (kThreads / 64) * RPW;
  for (int64_t row = wave * RPW + rw; row < rows; row += stride) {
    VT in = *reinterpret_cast<const VT*>(x + row * kD + sub * EPL);
    float xs[EPL];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      xs[i] = to_f(in[i]);
      ss = __builtin_fmaf(xs[i], xs[i], ss);
    }
    ss = group_sum<LPR>(ss);
    const float tau = rsq(ss * (1.0f / kD) + eps);
    VT out;
#pragma unroll
    for (int i = 0; i < EPL; ++i) out[i] = from_f<T>((xs[i] * tau) * g[i]);
    *reinterpret_cast<VT*>(y + row * kD + sub * EPL) = out;
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void qknorm_bwd_kernel(
    const T* __restrict__ x, const float* __restrict__ gain, const T* __restrict__ dy,
    T* __restrict__ dx, float* __restrict__ partial, int64_t rows, float eps) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  constexpr int LPR = kD / EPL;
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane % LPR, rw = lane / LPR;
  float g[EPL], dg[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    g[i] = gain[sub * EPL + i];
    dg[i] = 0.0f;
  }
  const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * (kThreads / 64) * RPW;
  for (int64_t row = wave * RPW + rw; row < rows; row += stride) {
    VT xin = *reinterpret_cast<const VT*>(x + row * kD + sub * EPL);
    VT din = *reinterpret_cast<const VT*>(dy + row * kD + sub * EPL);
    float xs[EPL], ds[EPL];
    float ss = 0.0f, dot = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      xs[i] = to_f(xin[i]);
      ds[i] = to_f(din[i]);
      ss = __builtin_fmaf(xs[i], xs[i], ss);
      dot = __builtin_fmaf(ds[i] * g[i], xs[i], dot);
    }
    ss = group_sum<LPR>(ss);
    dot = group_sum<LPR>(dot);
    const float tau = rsq(ss * (1.0f / kD) + eps);
    const float c = tau * tau * tau * dot * (1.0f / kD);
    VT out;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      out[i] = from_f<T>(tau * g[i] * ds[i] - c * xs[i]);
      dg[i] = __builtin_fmaf(ds[i], xs[i] * tau, dg[i]);
    }
    *reinterpret_cast<VT*>(dx + row * kD + sub * EPL) = out;
  }
  // Reduce dg over the row groups of the wave, then over the block's waves.
  __shared__ float red[kThreads / 64][kD];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    float v = dg[i];
#pragma unroll
    for (int m = LPR; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
    dg[i] = v;
  }
  if (rw == 0) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) red[threadIdx.x >> 6][sub * EPL + i] = dg[i];
  }
  __syncthreads();
  if (threadIdx.x < kD) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s += red[w][threadIdx.x];
    partial[(int64_t)blockIdx.x * kD + threadIdx.x] = s;
  }
}

__global__ __launch_bounds__(kThreads) void qknorm_gain_finish(const float* __restrict__ partial,
                                                               int nblocks,
                                                               float* __restrict__ dgain) {
  // One block per gain column: every thread sums a strided slice of the block
  // partials with independent loads in flight, then a fixed-order tree in LDS
  // finishes the column (deterministic for a given grid).
  __shared__ float red[kThreads];
  const int col = blockIdx.x;
  float s0 = 0.0f, s1 = 0.0f;
  int b = threadIdx.x;
  for (; b + kThreads < nblocks; b += 2 * kThreads) {
    s0 += partial[(int64_t)b * kD + col];
    s1 += partial[(int64_t)(b + kThreads) * kD + col];
  }
  if (b < nblocks) s0 += partial[(int64_t)b * kD + col];
  red[threadIdx.x] = s0 + s1;
  __syncthreads();
#pragma unroll
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) dgain[col] = red[0];
}

int blocks_for(int64_t rows, int dtype) {
  const int rpw = dtype == ALGX_BF16 ? 8 : 4;
  int64_t per_block = (int64_t)(kThreads / 64) * rpw;
  int64_t want = (rows + per_block - 1) / per_block;
  // At least ~2 rows per wave keeps loads in flight; cap the grid.
  want = (want + 1) / 2;
  if (want < 1) want = 1;
  return (int)(want > kMaxBlocks ? kMaxBlocks : want);
}

int32_t check_args(const void* x, const float* gain, int64_t rows, int32_t D, int32_t dtype,
                   float eps) {
  if (D != kD) return fail("qknorm: D must be 64");
  if (dtype != ALGX_BF16 && dtype != ALGX_F32) return fail("qknorm: dtype must be bf16 or f32");
  if (rows < 0) return fail("qknorm: negative row count");
  if (!(eps > 0.0f)) return fail("qknorm: eps must be positive");
  if (rows > 0 && (x == nullptr || gain == nullptr)) return fail("qknorm: null pointer");
  return 0;
}

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int32_t algx_qknorm_fwd(const void* x, const float* gain, void* y, int64_t rows,
                                   int32_t D, int32_t dtype, float eps, void* stream) {
  if (int32_t rc = check_args(x, gain, rows, D, dtype, eps)) return rc;
  if (rows == 0) return 0;
  if (y == nullptr) return fail("qknorm: null output");
  hipStream_t s = (hipStream_t)stream;
  const int nb = blocks_for(rows, dtype);
  const Probe probe = probe_for(ALGX_PROBE_QKNORM_FWD);
  if (dtype == ALGX_BF16)
    launch_k(probe, qknorm_fwd_kernel<bf16>, dim3(nb), dim3(kThreads), s, (const bf16*)x, gain,
             (bf16*)y, rows, eps);
  else
    launch_k(probe, qknorm_fwd_kernel<float>, dim3(nb), dim3(kThreads), s, (const float*)x, gain,
             (float*)y, rows, eps);
  return check_launch("qknorm_fwd");
}

extern "C" int64_t algx_qknorm_bwd_workspace_bytes(int64_t rows, int32_t D, int32_t dtype) {
  (void)D;
  return (int64_t)blocks_for(rows, dtype) * kD * sizeof(float);
}

extern "C" int32_t algx_qknorm_bwd(const void* x, const float* gain, const void* dy, void* dx,
                                   float* dgain, void* workspace, int64_t rows, int32_t D,
                                   int32_t dtype, float eps, void* stream) {
  if (int32_t rc = check_args(x, gain, rows, D, dtype, eps)) return rc;
  if (dgain == nullptr || workspace == nullptr) return fail("qknorm: null dgain/workspace");
  hipStream_t s = (hipStream_t)stream;
  if (rows == 0) {
    return fill_f32(dgain, kD, 0.0f, s);
  }
  if (dy == nullptr || dx == nullptr) return fail("qknorm: null dy/dx");
  const int nb = blocks_for(rows, dtype);
  float* partial = (float*)workspace;
  {
    const Probe probe = probe_for(ALGX_PROBE_QKNORM_BWD);
    if (dtype == ALGX_BF16)
      launch_k(probe, qknorm_bwd_kernel<bf16>, dim3(nb), dim3(kThreads), s, (const bf16*)x, gain,
               (const bf16*)dy, (bf16*)dx, partial, rows, eps);
    else
      launch_k(probe, qknorm_bwd_kernel<float>, dim3(nb), dim3(kThreads), s, (const float*)x,
               gain, (const float*)dy, (float*)dx, partial, rows, eps);
  }
  if (int32_t rc = check_launch("qknorm_bwd")) return rc;
  qknorm_gain_finish<<<kD, kThreads, 0, s>>>(partial, nb, dgain);
  return check_launch("qknorm_gain_finish");
}
