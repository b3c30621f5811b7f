// Attention prologue of the model block in one pass over HBM
// (model.py:166-174): from the q, k, v projections, laid out as rows of the
// (B, T, *) GEMM output, form
//   q_out = rotate(cast(rms_norm(q, q_gain))),  k_out likewise,  v_out = v
// in the (B, H, T, D) layout flash attention reads, where rotate is the
// rotate-half product with (T, D/2) cos/sin tables (algebraic.py:172-179).
// The norm is the QK RMS-norm (algebraic.py:76-83, qk_norm.py:29-59); the
// rotation rounds after every product and sum as the reference's bf16 ops do.
// The backward runs the same chain in reverse and writes dq, dk, dv straight
// into the rows of the projection gradient.
//
// D = 64. A row (b, t, h) is 128 bytes in bf16: 8 lanes of 16 bytes (16
// lanes in f32). The rotate-half partner of a lane's elements sits in lane
// ^ (lanes per row / 2), one xor-shuffle away. A workgroup owns 8 tokens of
// one sequence and every head slice of their q, k and v rows, so it reads
// whole projection rows and writes 1 KB runs of the (B, H, T, D) outputs.
// The gain gradients are reduced per workgroup and finished per column in a
// fixed order.
#include "common.h"

namespace algx {

namespace {

constexpr int kD = 64;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kBlockTokens = 8;

template <typename T> struct Vec;
template <> struct Vec<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct Vec<float> { typedef f32x4 type; static constexpr int n = 4; };

template <int LPR> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < LPR; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// A workgroup owns 8 consecutive tokens of one sequence and all 3 H head
// slices of their projection rows (q heads, then k, then v): it reads whole
// rows, and each (slice, 8 tokens) it writes is one contiguous 1 KB run of
// the (B, H, T, D) output. Wave w takes slices w, w + 4, ...
template <typename T, bool NORM, bool ROT>
__global__ __launch_bounds__(kThreads) void prologue_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, int64_t ld,
    const float* __restrict__ q_gain, const float* __restrict__ k_gain,
    const float* __restrict__ cosb, const float* __restrict__ sinb, T* __restrict__ q_out,
    T* __restrict__ k_out, T* __restrict__ v_out, int Tn, int H, int ntb, float eps) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  constexpr int LPR = kD / EPL;
  constexpr int RPW = 64 / LPR;
  constexpr int HALF = LPR / 2;
  const int b = blockIdx.x / ntb, t0 = (blockIdx.x % ntb) * kBlockTokens;
  const int lane = threadIdx.x & 63, sub = lane % LPR, rw = lane / LPR, w = threadIdx.x >> 6;
  float gq[EPL], gk[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    gq[e] = NORM ? q_gain[sub * EPL + e] : 1.0f;
    gk[e] = NORM ? k_gain[sub * EPL + e] : 1.0f;
  }
  const int j0 = (sub % HALF) * EPL;
  const bool first = sub < HALF;
  for (int sl = w; sl < 3 * H; sl += kWaves) {
    const int which = sl / H, h = sl % H;
    const T* src = (which == 0 ? q : (which == 1 ? k : v)) + (int64_t)b * Tn * ld + h * kD +
                   sub * EPL;
    T* dst = (which == 0 ? q_out : (which == 1 ? k_out : v_out)) +
             ((int64_t)b * H + h) * Tn * kD + sub * EPL;
#pragma unroll
    for (int i = 0; i < kBlockTokens; i += RPW) {
      const int t = t0 + i + rw;
      const bool ok = t < Tn;
      VT xin;
      if (ok) xin = *reinterpret_cast<const VT*>(src + (int64_t)t * ld);
      if (which == 2) {
        if (ok) *reinterpret_cast<VT*>(dst + (int64_t)t * kD) = xin;
        continue;
      }
      float y[EPL];
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        y[e] = ok ? to_f(xin[e]) : 0.0f;
        ss = __builtin_fmaf(y[e], y[e], ss);
      }
      if (NORM) {
        ss = group_sum<LPR>(ss);
        const float tau = rsq(ss * (1.0f / kD) + eps);
#pragma unroll
        for (int e = 0; e < EPL; ++e)
          y[e] = round_to<T>((y[e] * tau) * (which == 0 ? gq[e] : gk[e]));
      }
      VT out;
      if (ROT) {
        const int tc = ok ? t : 0;
        // the lane's EPL table entries as 16-byte loads (j0 is a multiple of EPL)
        float cv[EPL], sv[EPL];
#pragma unroll
        for (int q4 = 0; q4 < EPL; q4 += 4) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(cosb + (int64_t)tc * (kD / 2) + j0 + q4);
          const f32x4 bb = *reinterpret_cast<const f32x4*>(sinb + (int64_t)tc * (kD / 2) + j0 + q4);
#pragma unroll
          for (int z = 0; z < 4; ++z) { cv[q4 + z] = a[z]; sv[q4 + z] = bb[z]; }
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float p = __shfl_xor(y[e], HALF, 64);
          const float c = round_to<T>(cv[e]);
          const float s = round_to<T>(sv[e]);
          // first half: x1 c - x2 s; second half: x1 s + x2 c
          const float r = first ? round_to<T>(y[e] * c) - round_to<T>(p * s)
                                : round_to<T>(p * s) + round_to<T>(y[e] * c);
          out[e] = from_f<T>(r);
        }
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) out[e] = from_f<T>(y[e]);
      }
      if (ok) *reinterpret_cast<VT*>(dst + (int64_t)t * kD) = out;
    }
  }
}

// Reverse chain: rotation VJP (rounded as the autodiff of the bf16 products
// and sums), then the RMS-norm input VJP
//   dx = tau g dy - x tau^3 sum(dy g x) / D,   dgain += dy x tau,
// written into the projection-gradient rows; v's gradient is copied back.
// Same workgroup map as the forward; partial: [workgroup][q, k][D].
template <typename T, bool NORM, bool ROT>
__global__ __launch_bounds__(kThreads) void prologue_bwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, int64_t ld, const float* __restrict__ q_gain,
    const float* __restrict__ k_gain, const float* __restrict__ cosb,
    const float* __restrict__ sinb, const T* __restrict__ dq_out, const T* __restrict__ dk_out,
    const T* __restrict__ dv_out, T* __restrict__ dq, T* __restrict__ dk, T* __restrict__ dv,
    float* __restrict__ partial, int Tn, int H, int ntb, float eps) {
  typedef typename Vec<T>::type VT;
  constexpr int EPL = Vec<T>::n;
  constexpr int LPR = kD / EPL;
  constexpr int RPW = 64 / LPR;
  constexpr int HALF = LPR / 2;
  const int b = blockIdx.x / ntb, t0 = (blockIdx.x % ntb) * kBlockTokens;
  const int lane = threadIdx.x & 63, sub = lane % LPR, rw = lane / LPR, w = threadIdx.x >> 6;
  float gq[EPL], gk[EPL], dgq[EPL], dgk[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    gq[e] = NORM ? q_gain[sub * EPL + e] : 1.0f;
    gk[e] = NORM ? k_gain[sub * EPL + e] : 1.0f;
    dgq[e] = 0.0f;
    dgk[e] = 0.0f;
  }
  const int j0 = (sub % HALF) * EPL;
  const bool first = sub < HALF;
  for (int sl = w; sl < 3 * H; sl += kWaves) {
    const int which = sl / H, h = sl % H;
    const int64_t head_off = ((int64_t)b * H + h) * Tn * kD + sub * EPL;
    const int64_t row_off = (int64_t)b * Tn * ld + h * kD + sub * EPL;
    const T* dout = (which == 0 ? dq_out : (which == 1 ? dk_out : dv_out)) + head_off;
    T* dx = (which == 0 ? dq : (which == 1 ? dk : dv)) + row_off;
    const T* x = (which == 0 ? q : k) + row_off;
#pragma unroll
    for (int i = 0; i < kBlockTokens; i += RPW) {
      const int t = t0 + i + rw;
      const bool ok = t < Tn;
      VT din, xin;
      if (ok) {
        din = *reinterpret_cast<const VT*>(dout + (int64_t)t * kD);
        if (NORM && which != 2) xin = *reinterpret_cast<const VT*>(x + (int64_t)t * ld);
      }
      if (which == 2) {
        if (ok) *reinterpret_cast<VT*>(dx + (int64_t)t * ld) = din;
        continue;
      }
      float dy[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) dy[e] = ok ? to_f(din[e]) : 0.0f;
      if (ROT) {
        const int tc = ok ? t : 0;
        // the lane's EPL table entries as 16-byte loads (j0 is a multiple of EPL)
        float cv[EPL], sv[EPL];
#pragma unroll
        for (int q4 = 0; q4 < EPL; q4 += 4) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(cosb + (int64_t)tc * (kD / 2) + j0 + q4);
          const f32x4 bb = *reinterpret_cast<const f32x4*>(sinb + (int64_t)tc * (kD / 2) + j0 + q4);
#pragma unroll
          for (int z = 0; z < 4; ++z) { cv[q4 + z] = a[z]; sv[q4 + z] = bb[z]; }
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float p = __shfl_xor(dy[e], HALF, 64);
          const float c = round_to<T>(cv[e]);
          const float s = round_to<T>(sv[e]);
          // dx1 = d1 c + d2 s; dx2 = d2 c - d1 s
          dy[e] = first ? round_to<T>(round_to<T>(dy[e] * c) + round_to<T>(p * s))
                        : round_to<T>(round_to<T>(dy[e] * c) - round_to<T>(p * s));
        }
      }
      VT out;
      if (NORM) {
        float xs[EPL], g[EPL];
        float ss = 0.0f, dot = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          g[e] = which == 0 ? gq[e] : gk[e];
          xs[e] = ok ? to_f(xin[e]) : 0.0f;
          ss = __builtin_fmaf(xs[e], xs[e], ss);
          dot = __builtin_fmaf(dy[e] * g[e], xs[e], dot);
        }
        ss = group_sum<LPR>(ss);
        dot = group_sum<LPR>(dot);
        const float tau = rsq(ss * (1.0f / kD) + eps);
        const float cf = tau * tau * tau * dot * (1.0f / kD);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          out[e] = from_f<T>(tau * g[e] * dy[e] - cf * xs[e]);
          if (which == 0)
            dgq[e] = __builtin_fmaf(dy[e], xs[e] * tau, dgq[e]);
          else
            dgk[e] = __builtin_fmaf(dy[e], xs[e] * tau, dgk[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) out[e] = from_f<T>(dy[e]);
      }
      if (ok) *reinterpret_cast<VT*>(dx + (int64_t)t * ld) = out;
    }
  }
  if (!NORM) return;
  // Workgroup share of dgain: rows of the wave by xor-shuffles, then the
  // four waves in order through LDS.
  __shared__ float red[kWaves][2][kD];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    float a = dgq[e], c = dgk[e];
#pragma unroll
    for (int m = LPR; m < 64; m <<= 1) {
      a += __shfl_xor(a, m, 64);
      c += __shfl_xor(c, m, 64);
    }
    dgq[e] = a;
    dgk[e] = c;
  }
  if (rw == 0) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      red[w][0][sub * EPL + e] = dgq[e];
      red[w][1][sub * EPL + e] = dgk[e];
    }
  }
  __syncthreads();
  if (threadIdx.x < 2 * kD) {
    const int which = threadIdx.x / kD, col = threadIdx.x % kD;
    float s = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) s += red[ww][which][col];
    partial[((int64_t)blockIdx.x * 2 + which) * kD + col] = s;
  }
}

// dgain of q and k from the workgroup partials: one workgroup per (tensor,
// column), each thread summing a strided slice of the partial rows with
// independent loads in flight, then a fixed-order tree in LDS.
__global__ __launch_bounds__(256) void prologue_gain_finish(const float* __restrict__ partial,
                                                            int nparts, float* __restrict__ dq_gain,
                                                            float* __restrict__ dk_gain) {
  __shared__ float red[256];
  const int which = blockIdx.x / kD, col = blockIdx.x % kD;
  float s0 = 0.0f, s1 = 0.0f;
  int r = threadIdx.x;
  for (; r + 256 < nparts; r += 512) {
    s0 += partial[((int64_t)r * 2 + which) * kD + col];
    s1 += partial[((int64_t)(r + 256) * 2 + which) * kD + col];
  }
  if (r < nparts) s0 += partial[((int64_t)r * 2 + which) * kD + col];
  red[threadIdx.x] = s0 + s1;
  __syncthreads();
#pragma unroll
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) (which == 0 ? dq_gain : dk_gain)[col] = red[0];
}

int ntb_of(int T) { return (T + kBlockTokens - 1) / kBlockTokens; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int32_t check_prologue(const void* q, const void* k, const void* v, int64_t ld,
                       const float* q_gain, const float* k_gain, const float* cosb,
                       const float* sinb, int B, int T, int H, int D, int dtype, float eps) {
  if (D != kD) return fail("qk_prologue: D must be 64");
  if (dtype != ALGX_BF16 && dtype != ALGX_F32) return fail("qk_prologue: dtype must be bf16 or f32");
  if (B < 0 || T < 0 || H <= 0) return fail("qk_prologue: invalid sizes");
  if (ld < (int64_t)H * kD) return fail("qk_prologue: row stride below H * D");
  if ((q_gain == nullptr) != (k_gain == nullptr))
    return fail("qk_prologue: q_gain and k_gain go together");
  if ((cosb == nullptr) != (sinb == nullptr)) return fail("qk_prologue: cos and sin go together");
  if (q_gain != nullptr && !(eps > 0.0f)) return fail("qk_prologue: eps must be positive");
  const int esz = dtype == ALGX_BF16 ? 2 : 4;
  if ((ld * esz) % 16) return fail("qk_prologue: row stride must be a multiple of 16 bytes");
  if ((int64_t)B * T > 0) {
    if (q == nullptr || k == nullptr || v == nullptr) return fail("qk_prologue: null input");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v))
      return fail("qk_prologue: operands must be 16-byte aligned");
  }
  return 0;
}

template <typename T>
void launch_fwd(bool norm, bool rot, dim3 grid, hipStream_t s, const void* q, const void* k,
                const void* v, int64_t ld, const float* qg, const float* kg, const float* cb,
                const float* sb, void* qo, void* ko, void* vo, int Tn, int H, int ntb,
                float eps) {
#define ALGX_PRO_FWD(N, R)                                                                  \
  prologue_fwd_kernel<T, N, R><<<grid, kThreads, 0, s>>>(                                   \
      (const T*)q, (const T*)k, (const T*)v, ld, qg, kg, cb, sb, (T*)qo, (T*)ko, (T*)vo, Tn, H, \
      ntb, eps)
  if (norm && rot) ALGX_PRO_FWD(true, true);
  else if (norm) ALGX_PRO_FWD(true, false);
  else if (rot) ALGX_PRO_FWD(false, true);
  else ALGX_PRO_FWD(false, false);
#undef ALGX_PRO_FWD
}

template <typename T>
void launch_bwd(bool norm, bool rot, dim3 grid, hipStream_t s, const void* q, const void* k,
                int64_t ld, const float* qg, const float* kg, const float* cb, const float* sb,
                const void* dqo, const void* dko, const void* dvo, void* dq, void* dk, void* dv,
                float* partial, int Tn, int H, int ntb, float eps) {
#define ALGX_PRO_BWD(N, R)                                                                   \
  prologue_bwd_kernel<T, N, R><<<grid, kThreads, 0, s>>>(                                    \
      (const T*)q, (const T*)k, ld, qg, kg, cb, sb, (const T*)dqo, (const T*)dko,            \
      (const T*)dvo, (T*)dq, (T*)dk, (T*)dv, partial, Tn, H, ntb, eps)
  if (norm && rot) ALGX_PRO_BWD(true, true);
  else if (norm) ALGX_PRO_BWD(true, false);
  else if (rot) ALGX_PRO_BWD(false, true);
  else ALGX_PRO_BWD(false, false);
#undef ALGX_PRO_BWD
}

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int32_t algx_qk_prologue_fwd(const void* q, const void* k, const void* v, int64_t ld,
                                        const float* q_gain, const float* k_gain,
                                        const float* cos_t, const float* sin_t, void* q_out,
                                        void* k_out, void* v_out, int32_t B, int32_t T, int32_t H,
                                        int32_t D, int32_t dtype, float eps, void* stream) {
  if (int32_t rc = check_prologue(q, k, v, ld, q_gain, k_gain, cos_t, sin_t, B, T, H, D, dtype,
                                  eps))
    return rc;
  if ((int64_t)B * T == 0) return 0;
  if (q_out == nullptr || k_out == nullptr || v_out == nullptr)
    return fail("qk_prologue: null output");
  if (!aligned16(q_out) || !aligned16(k_out) || !aligned16(v_out))
    return fail("qk_prologue: operands must be 16-byte aligned");
  const int ntb = ntb_of(T);
  const dim3 grid((unsigned)((int64_t)B * ntb));
  hipStream_t s = (hipStream_t)stream;
  const bool norm = q_gain != nullptr, rot = cos_t != nullptr;
  if (dtype == ALGX_BF16)
    launch_fwd<bf16>(norm, rot, grid, s, q, k, v, ld, q_gain, k_gain, cos_t, sin_t, q_out, k_out,
                     v_out, T, H, ntb, eps);
  else
    launch_fwd<float>(norm, rot, grid, s, q, k, v, ld, q_gain, k_gain, cos_t, sin_t, q_out, k_out,
                      v_out, T, H, ntb, eps);
  return check_launch("qk_prologue_fwd");
}

extern "C" int64_t algx_qk_prologue_bwd_workspace_bytes(int32_t B, int32_t T, int32_t H,
                                                        int32_t D, int32_t dtype) {
  (void)D;
  (void)dtype;
  if (B <= 0 || T <= 0 || H <= 0) return 0;
  return 2 * (int64_t)B * ntb_of(T) * kD * (int64_t)sizeof(float);
}

extern "C" int32_t algx_qk_prologue_bwd(const void* q, const void* k, const float* q_gain,
                                        const float* k_gain, const float* cos_t,
                                        const float* sin_t, const void* dq_out,
                                        const void* dk_out, const void* dv_out, void* dq, void* dk,
                                        void* dv, int64_t ld, float* dq_gain, float* dk_gain,
                                        void* workspace, int32_t B, int32_t T, int32_t H,
                                        int32_t D, int32_t dtype, float eps, void* stream) {
  // q and k (the raw projections) are read only for the norm; v is not read.
  if (int32_t rc = check_prologue(q, k, q, ld, q_gain, k_gain, cos_t, sin_t, B, T, H, D, dtype,
                                  eps))
    return rc;
  const bool norm = q_gain != nullptr, rot = cos_t != nullptr;
  if (norm && (dq_gain == nullptr || dk_gain == nullptr))
    return fail("qk_prologue: gain gradients are required with gains");
  hipStream_t s = (hipStream_t)stream;
  if ((int64_t)B * T == 0) {
    if (!norm) return 0;
    if (int32_t rc = fill_f32(dq_gain, kD, 0.0f, s)) return rc;
    return fill_f32(dk_gain, kD, 0.0f, s);
  }
  if (dq_out == nullptr || dk_out == nullptr || dv_out == nullptr || dq == nullptr ||
      dk == nullptr || dv == nullptr)
    return fail("qk_prologue: null gradient");
  if (!aligned16(dq_out) || !aligned16(dk_out) || !aligned16(dv_out) || !aligned16(dq) ||
      !aligned16(dk) || !aligned16(dv))
    return fail("qk_prologue: operands must be 16-byte aligned");
  if (norm && workspace == nullptr) return fail("qk_prologue: null workspace");
  const int ntb = ntb_of(T);
  const dim3 grid((unsigned)((int64_t)B * ntb));
  float* partial = (float*)workspace;
  if (dtype == ALGX_BF16)
    launch_bwd<bf16>(norm, rot, grid, s, q, k, ld, q_gain, k_gain, cos_t, sin_t, dq_out, dk_out,
                     dv_out, dq, dk, dv, partial, T, H, ntb, eps);
  else
    launch_bwd<float>(norm, rot, grid, s, q, k, ld, q_gain, k_gain, cos_t, sin_t, dq_out, dk_out,
                      dv_out, dq, dk, dv, partial, T, H, ntb, eps);
  if (int32_t rc = check_launch("qk_prologue_bwd")) return rc;
  if (!norm) return 0;
  prologue_gain_finish<<<2 * kD, 256, 0, s>>>(partial, B * ntb, dq_gain, dk_gain);
  return check_launch("qk_prologue_gain_finish");
}
