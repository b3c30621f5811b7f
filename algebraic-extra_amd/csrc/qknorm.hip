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
//
// One launch covers one tensor or a pair (the attention's q and k, each with
// its own gain): the first nb0 blocks stream tensor 0, the rest tensor 1, so
// the pair moves as one 134 MB (forward) / 201 MB (backward) stream instead of
// two half-size ones.
#include "common.h"

namespace algx {

namespace {

constexpr int kD = 64;
constexpr int kThreads = 256;
constexpr int kMaxBlocks = 2048;
constexpr int kUnroll = 2;  // rows per lane group in flight per loop iteration

template <typename T> struct Vec;
template <> struct Vec<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct Vec<float> { typedef f32x4 type; static constexpr int n = 4; };

template <int LPR> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < LPR; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Tensors of one launch: blocks [0, nb0) take tensor 0, [nb0, gridDim.x)
// tensor 1 (nb0 == gridDim.x for a single tensor).
template <typename T>
struct NormPair {
  const T* x[2];
  const float* gain[2];
  const T* dy[2];
  T* out[2];  // y (forward) or dx (backward)
  int nb0;
};

template <typename T>
__global__ __launch_bounds__(kThreads) void qknorm_fwd_kernel(NormPair<T> P, int64_t rows,
                                                              float eps) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  constexpr int LPR = kD / EPL;
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane % LPR, rw = lane / LPR;
  const int t = blockIdx.x >= P.nb0 ? 1 : 0;
  const int blk = blockIdx.x - t * P.nb0, nblk = t ? gridDim.x - P.nb0 : P.nb0;
  const T* __restrict__ x = P.x[t];
  T* __restrict__ y = P.out[t];
  float g[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) g[i] = P.gain[t][sub * EPL + i];
  const int64_t wave = (int64_t)blk * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t stride = (int64_t)nblk * (kThreads / 64) * RPW;
  // kUnroll rows per lane group and iteration, all loads issued first. A row
  // past the end reads row 0 and is not stored; the LPR lanes of a group
  // share a row, so the group shuffles never see a divergent lane.
  for (int64_t row0 = wave * RPW + rw; row0 < rows; row0 += kUnroll * stride) {
    VT in[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t row = row0 + u * stride;
      in[u] = *reinterpret_cast<const VT*>(x + (row < rows ? row : 0) * kD + sub * EPL);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t row = row0 + u * stride;
      float xs[EPL];
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        xs[i] = to_f(in[u][i]);
        ss = __builtin_fmaf(xs[i], xs[i], ss);
      }
      ss = group_sum<LPR>(ss);
      const float tau = rsq(ss * (1.0f / kD) + eps);
      VT out;
#pragma unroll
      for (int i = 0; i < EPL; ++i) out[i] = from_f<T>((xs[i] * tau) * g[i]);
      if (row < rows) *reinterpret_cast<VT*>(y + row * kD + sub * EPL) = out;
    }
  }
}

// partial: one dgain row per block (tensor 0's blocks first).
template <typename T>
__global__ __launch_bounds__(kThreads) void qknorm_bwd_kernel(NormPair<T> P,
                                                              float* __restrict__ partial,
                                                              int64_t rows, float eps) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  constexpr int LPR = kD / EPL;
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane % LPR, rw = lane / LPR;
  const int t = blockIdx.x >= P.nb0 ? 1 : 0;
  const int blk = blockIdx.x - t * P.nb0, nblk = t ? gridDim.x - P.nb0 : P.nb0;
  const T* __restrict__ x = P.x[t];
  const T* __restrict__ dy = P.dy[t];
  T* __restrict__ dx = P.out[t];
  float g[EPL], dg[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    g[i] = P.gain[t][sub * EPL + i];
    dg[i] = 0.0f;
  }
  const int64_t wave = (int64_t)blk * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t stride = (int64_t)nblk * (kThreads / 64) * RPW;
  // As the forward: kUnroll rows per iteration, loads first; a row past the
  // end reads row 0, adds nothing to dgain and is not stored.
  for (int64_t row0 = wave * RPW + rw; row0 < rows; row0 += kUnroll * stride) {
    VT xin[kUnroll], din[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t row = row0 + u * stride;
      const int64_t off = (row < rows ? row : 0) * kD + sub * EPL;
      xin[u] = *reinterpret_cast<const VT*>(x + off);
      din[u] = *reinterpret_cast<const VT*>(dy + off);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t row = row0 + u * stride;
      const bool live = row < rows;
      float xs[EPL], ds[EPL];
      float ss = 0.0f, dot = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        xs[i] = to_f(xin[u][i]);
        ds[i] = live ? to_f(din[u][i]) : 0.0f;
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
      if (live) *reinterpret_cast<VT*>(dx + row * kD + sub * EPL) = out;
    }
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

// Block c of tensor t (blockIdx.x = 64 t + c) finishes dgain column c of
// tensor t from that tensor's nblocks partial rows.
__global__ __launch_bounds__(kThreads) void qknorm_gain_finish(const float* __restrict__ partial,
                                                               int nblocks0, int nblocks1,
                                                               float* __restrict__ dgain0,
                                                               float* __restrict__ dgain1) {
  // One block per gain column: every thread sums a strided slice of the block
  // partials with independent loads in flight, then a fixed-order tree in LDS
  // finishes the column (deterministic for a given grid).
  __shared__ float red[kThreads];
  const int t = blockIdx.x >= kD ? 1 : 0;
  const int col = blockIdx.x - t * kD;
  const int nblocks = t ? nblocks1 : nblocks0;
  float* __restrict__ dgain = t ? dgain1 : dgain0;
  partial += t ? (int64_t)nblocks0 * kD : 0;
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


template <typename T>
int32_t launch_fwd(const NormPair<T>& P, int nb, int64_t rows, float eps, hipStream_t s) {
  launch_k(probe_for(ALGX_PROBE_QKNORM_FWD), qknorm_fwd_kernel<T>, dim3(nb), dim3(kThreads), s,
           P, rows, eps);
  return check_launch("qknorm_fwd");
}

template <typename T>
int32_t launch_bwd(const NormPair<T>& P, int nb, float* partial, float* dgain0, float* dgain1,
                   int64_t rows, float eps, hipStream_t s) {
  launch_k(probe_for(ALGX_PROBE_QKNORM_BWD), qknorm_bwd_kernel<T>, dim3(nb), dim3(kThreads), s,
           P, partial, rows, eps);
  if (int32_t rc = check_launch("qknorm_bwd")) return rc;
  const bool pair = nb > P.nb0;
  qknorm_gain_finish<<<pair ? 2 * kD : kD, kThreads, 0, s>>>(partial, P.nb0, nb - P.nb0, dgain0,
                                                             dgain1);
  return check_launch("qknorm_gain_finish");
}

// Forward over one (x1 == nullptr) or two tensors of `rows` rows each.
int32_t norm_fwd(const void* x0, const void* x1, const float* g0, const float* g1, void* y0,
                 void* y1, int64_t rows, int32_t dtype, float eps, hipStream_t s) {
  const int nb0 = blocks_for(rows, dtype);
  const int nb = x1 != nullptr ? 2 * nb0 : nb0;
  if (dtype == ALGX_BF16) {
    const NormPair<bf16> P{{(const bf16*)x0, (const bf16*)x1}, {g0, g1}, {nullptr, nullptr},
                           {(bf16*)y0, (bf16*)y1}, nb0};
    return launch_fwd(P, nb, rows, eps, s);
  }
  const NormPair<float> P{{(const float*)x0, (const float*)x1}, {g0, g1}, {nullptr, nullptr},
                          {(float*)y0, (float*)y1}, nb0};
  return launch_fwd(P, nb, rows, eps, s);
}

int32_t norm_bwd(const void* x0, const void* x1, const float* g0, const float* g1,
                 const void* dy0, const void* dy1, void* dx0, void* dx1, float* dg0, float* dg1,
                 float* partial, int64_t rows, int32_t dtype, float eps, hipStream_t s) {
  const int nb0 = blocks_for(rows, dtype);
  const int nb = x1 != nullptr ? 2 * nb0 : nb0;
  if (dtype == ALGX_BF16) {
    const NormPair<bf16> P{{(const bf16*)x0, (const bf16*)x1}, {g0, g1},
                           {(const bf16*)dy0, (const bf16*)dy1}, {(bf16*)dx0, (bf16*)dx1}, nb0};
    return launch_bwd(P, nb, partial, dg0, dg1, rows, eps, s);
  }
  const NormPair<float> P{{(const float*)x0, (const float*)x1}, {g0, g1},
                          {(const float*)dy0, (const float*)dy1}, {(float*)dx0, (float*)dx1},
                          nb0};
  return launch_bwd(P, nb, partial, dg0, dg1, rows, eps, s);
}

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int32_t algx_qknorm_fwd(const void* x, const float* gain, void* y, int64_t rows,
                                   int32_t D, int32_t dtype, float eps, void* stream) {
  if (int32_t rc = check_args(x, gain, rows, D, dtype, eps)) return rc;
  if (rows == 0) return 0;
  if (y == nullptr) return fail("qknorm: null output");
  return norm_fwd(x, nullptr, gain, nullptr, y, nullptr, rows, dtype, eps, (hipStream_t)stream);
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
  if (rows == 0) return fill_f32(dgain, kD, 0.0f, s);
  if (dy == nullptr || dx == nullptr) return fail("qknorm: null dy/dx");
  return norm_bwd(x, nullptr, gain, nullptr, dy, nullptr, dx, nullptr, dgain, nullptr,
                  (float*)workspace, rows, dtype, eps, s);
}

extern "C" int32_t algx_qknorm_pair_fwd(const void* xq, const void* xk, const float* gain_q,
                                        const float* gain_k, void* yq, void* yk, int64_t rows,
                                        int32_t D, int32_t dtype, float eps, void* stream) {
  if (int32_t rc = check_args(xq, gain_q, rows, D, dtype, eps)) return rc;
  if (int32_t rc = check_args(xk, gain_k, rows, D, dtype, eps)) return rc;
  if (rows == 0) return 0;
  if (yq == nullptr || yk == nullptr) return fail("qknorm: null output");
  return norm_fwd(xq, xk, gain_q, gain_k, yq, yk, rows, dtype, eps, (hipStream_t)stream);
}

extern "C" int64_t algx_qknorm_pair_bwd_workspace_bytes(int64_t rows, int32_t D, int32_t dtype) {
  (void)D;
  return 2 * (int64_t)blocks_for(rows, dtype) * kD * sizeof(float);
}

extern "C" int32_t algx_qknorm_pair_bwd(const void* xq, const void* xk, const float* gain_q,
                                        const float* gain_k, const void* dyq, const void* dyk,
                                        void* dxq, void* dxk, float* dgain_q, float* dgain_k,
                                        void* workspace, int64_t rows, int32_t D, int32_t dtype,
                                        float eps, void* stream) {
  if (int32_t rc = check_args(xq, gain_q, rows, D, dtype, eps)) return rc;
  if (int32_t rc = check_args(xk, gain_k, rows, D, dtype, eps)) return rc;
  if (dgain_q == nullptr || dgain_k == nullptr || workspace == nullptr)
    return fail("qknorm: null dgain/workspace");
  hipStream_t s = (hipStream_t)stream;
  if (rows == 0) {
    if (int32_t rc = fill_f32(dgain_q, kD, 0.0f, s)) return rc;
    return fill_f32(dgain_k, kD, 0.0f, s);
  }
  if (dyq == nullptr || dyk == nullptr || dxq == nullptr || dxk == nullptr)
    return fail("qknorm: null dy/dx");
  return norm_bwd(xq, xk, gain_q, gain_k, dyq, dyk, dxq, dxk, dgain_q, dgain_k,
                  (float*)workspace, rows, dtype, eps, s);
}
