// Attention side passes: range guard reduction, backward row pre-pass
// (di, dsink, dQ accumulator clear) and the dQ finishing cast.
#include "attn_aux.h"

namespace algx {

namespace {

template <typename T> struct V16;
template <> struct V16<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct V16<float> { typedef f32x4 type; static constexpr int n = 4; };

__device__ __forceinline__ float nan_to_inf(float x) { return x != x ? __builtin_inff() : x; }

template <int LPR> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < LPR; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}
template <int LPR> __device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = 1; m < LPR; m <<= 1) v = __builtin_fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// One pass over q, k, v: writes q_s = cast(q * scale) (flash.py:833) and the
// per-block maxima of |q_s|^2 (:841), |k|^2 (:842) and |v| (:849). NaN
// becomes +inf so that it fails the guard as jnp.max's NaN does.
template <typename T, int D>
__global__ __launch_bounds__(256) void prepare_guard_kernel(const T* __restrict__ q,
                                                            const T* __restrict__ k,
                                                            const T* __restrict__ v,
                                                            T* __restrict__ q_s, int64_t rows,
                                                            float q_scale,
                                                            float* __restrict__ partial) {
  typedef typename V16<T>::type VT;
  constexpr int EPL = V16<T>::n;
  constexpr int LPR = D / EPL;
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane % LPR, rw = lane / LPR;
  float mq = 0.0f, mk = 0.0f, mv = 0.0f;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * 4 * RPW;
  for (int64_t row = wave * RPW + rw; row < rows; row += stride) {
    const int64_t off = row * D + sub * EPL;
    VT a = *reinterpret_cast<const VT*>(q + off);
    VT b = *reinterpret_cast<const VT*>(k + off);
    VT c = *reinterpret_cast<const VT*>(v + off);
    float sq = 0.0f, sk = 0.0f, av = 0.0f;
    VT qo;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      qo[i] = from_f<T>(to_f(a[i]) * q_scale);
      const float qs = to_f(qo[i]);
      sq = __builtin_fmaf(qs, qs, sq);
      const float kk = to_f(b[i]);
      sk = __builtin_fmaf(kk, kk, sk);
      av = __builtin_fmaxf(av, nan_to_inf(__builtin_fabsf(to_f(c[i]))));
    }
    *reinterpret_cast<VT*>(q_s + off) = qo;
    sq = nan_to_inf(group_sum<LPR>(sq));
    sk = nan_to_inf(group_sum<LPR>(sk));
    mq = __builtin_fmaxf(mq, sq);
    mk = __builtin_fmaxf(mk, sk);
    mv = __builtin_fmaxf(mv, av);
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    mq = __builtin_fmaxf(mq, __shfl_xor(mq, m, 64));
    mk = __builtin_fmaxf(mk, __shfl_xor(mk, m, 64));
    mv = __builtin_fmaxf(mv, __shfl_xor(mv, m, 64));
  }
  __shared__ float red[3][4];
  if (lane == 0) {
    red[0][threadIdx.x >> 6] = mq;
    red[1][threadIdx.x >> 6] = mk;
    red[2][threadIdx.x >> 6] = mv;
  }
  __syncthreads();
  if (threadIdx.x < 3) {
    const float* r = red[threadIdx.x];
    partial[(int64_t)blockIdx.x * 3 + threadIdx.x] =
        __builtin_fmaxf(__builtin_fmaxf(r[0], r[1]), __builtin_fmaxf(r[2], r[3]));
  }
}

// q_s = cast(q * scale) alone (unguarded calls), flash.py:833.
template <typename T>
__global__ __launch_bounds__(256) void scale_kernel(const T* __restrict__ q, T* __restrict__ q_s,
                                                    int64_t n, float q_scale) {
  typedef typename V16<T>::type VT;
  constexpr int EPL = V16<T>::n;
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * EPL;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * EPL;
  for (; i < n; i += stride) {
    VT a = *reinterpret_cast<const VT*>(q + i);
#pragma unroll
    for (int e = 0; e < EPL; ++e) a[e] = from_f<T>(to_f(a[e]) * q_scale);
    *reinterpret_cast<VT*>(q_s + i) = a;
  }
}

// flash.py:843-849: in_range = q2*k2 <= (bound/1.01)^2 & |sink| <= bound/1.01 & |v| <= vmax.
__global__ __launch_bounds__(256) void guard_finish_kernel(const float* __restrict__ partial,
                                                           int nblocks, const float* sink, int H,
                                                           float bound_sq, float bound_s,
                                                           float vmax, int32_t* guard) {
  __shared__ float red[3][256];
  float mq = 0.0f, mk = 0.0f, mv = 0.0f;
  for (int b = threadIdx.x; b < nblocks; b += 256) {
    mq = __builtin_fmaxf(mq, partial[b * 3 + 0]);
    mk = __builtin_fmaxf(mk, partial[b * 3 + 1]);
    mv = __builtin_fmaxf(mv, partial[b * 3 + 2]);
  }
  red[0][threadIdx.x] = mq;
  red[1][threadIdx.x] = mk;
  red[2][threadIdx.x] = mv;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) {
#pragma unroll
      for (int j = 0; j < 3; ++j)
        red[j][threadIdx.x] = __builtin_fmaxf(red[j][threadIdx.x], red[j][threadIdx.x + w]);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float ms = 0.0f;
    if (sink != nullptr)
      for (int h = 0; h < H; ++h) ms = __builtin_fmaxf(ms, nan_to_inf(__builtin_fabsf(sink[h])));
    const float q2 = red[0][0], k2 = red[1][0], vm = red[2][0];
    bool ok = q2 * k2 <= bound_sq;
    if (sink != nullptr) ok = ok && ms <= bound_s;
    ok = ok && vm <= vmax;
    guard[0] = ok ? 1 : 0;
    float* f = reinterpret_cast<float*>(guard);
    f[1] = q2;
    f[2] = k2;
    f[3] = vm;
    f[4] = ms;
  }
}

// Backward pre-pass per row (flash.py:633, :721-723): di = sum(dO * o) with
// o the saved residual (float32 for precise-output variants); accumulates
// the sink gradient of the row's head; clears the dQ accumulator row.
// Grid: (row blocks, B*H); every block stays within one head.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_pre_kernel(
    const T* __restrict__ dout, const T* __restrict__ o, const float* __restrict__ o_precise,
    const float* __restrict__ stat, const float* __restrict__ sink, float* __restrict__ di,
    float* __restrict__ dq_acc, float* __restrict__ dsink, int H, int T_, KVariant low,
    KVariant high, const int32_t* __restrict__ guard) {
  typedef typename V16<T>::type VT;
  constexpr int EPL = V16<T>::n;
  constexpr int LPR = D / EPL;
  constexpr int RPW = 64 / LPR;
  const bool in_range = guard_in_range(guard);
  const KVariant& var = in_range ? low : high;
  const int lane = threadIdx.x & 63, sub = lane % LPR, rw = lane / LPR;
  const int bh = blockIdx.y, h = bh % H;
  const int64_t head = (int64_t)bh * T_;
  const bool has_sink = sink != nullptr;
  const float b = has_sink ? sink[h] : 0.0f;
  float ds_acc = 0.0f;
  const int rows_per_iter = 4 * RPW;
  for (int t = blockIdx.x * rows_per_iter + (threadIdx.x >> 6) * RPW + rw; t < T_;
       t += gridDim.x * rows_per_iter) {
    const int64_t row = head + t;
    const int64_t off = row * D + sub * EPL;
    VT g = *reinterpret_cast<const VT*>(dout + off);
    float acc = 0.0f;
    if (var.precise) {
#pragma unroll
      for (int i = 0; i < EPL; i += 4) {
        f32x4 ov = *reinterpret_cast<const f32x4*>(o_precise + off + i);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_fmaf(to_f(g[i + j]), ov[j], acc);
      }
    } else {
      VT ov = *reinterpret_cast<const VT*>(o + off);
#pragma unroll
      for (int i = 0; i < EPL; ++i) acc = __builtin_fmaf(to_f(g[i]), to_f(ov[i]), acc);
    }
    acc = group_sum<LPR>(acc);
    if (sub == 0) {
      di[row] = acc;
      if (has_sink) ds_acc += sink_grad_term(var, b, stat[row], acc);
    }
    if (dq_acc != nullptr) {
      f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < EPL; i += 4) *reinterpret_cast<f32x4*>(dq_acc + off + i) = z;
    }
  }
  if (has_sink && dsink != nullptr) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) ds_acc += __shfl_xor(ds_acc, m, 64);
    __shared__ float red[4];
    if (lane == 0) red[threadIdx.x >> 6] = ds_acc;
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(dsink + h, (red[0] + red[1]) + (red[2] + red[3]));
  }
}

// dq = cast(cast(acc * slope) * q_scale): the kernel's dQ output rounding
// (flash.py:592) followed by the VJP of the query pre-scale (flash.py:833).
template <typename T>
__global__ __launch_bounds__(256) void dq_finish_kernel(const float* __restrict__ acc,
                                                        T* __restrict__ dq, int64_t n,
                                                        KVariant low, KVariant high,
                                                        const int32_t* __restrict__ guard,
                                                        float q_scale) {
  const KVariant& var = guard_in_range(guard) ? low : high;
  const float slope = var.slope;
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
  for (; i < n; i += stride) {
    f32x4 a = *reinterpret_cast<const f32x4*>(acc + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) dq[i + j] = from_f<T>(round_to<T>(a[j] * slope) * q_scale);
  }
}

}  // namespace

constexpr int kGuardBlocks = 1024;

int32_t guard_words() { return 8 + 3 * kGuardBlocks; }

int32_t launch_prepare(const void* q, const void* k, const void* v, const float* sink, void* q_s,
                       int32_t* guard, int B, int H, int T, int D, int dtype, float q_scale,
                       float bound, float vmax, hipStream_t s) {
  const int64_t rows = (int64_t)B * H * T;
  if (guard == nullptr) {
    const int64_t n = rows * D;
    const int epl = dtype == ALGX_BF16 ? 8 : 4;
    int64_t nb = (n / epl + 255) / 256;
    if (nb > 8192) nb = 8192;
    if (nb < 1) nb = 1;
    if (dtype == ALGX_BF16)
      scale_kernel<bf16><<<(int)nb, 256, 0, s>>>((const bf16*)q, (bf16*)q_s, n, q_scale);
    else
      scale_kernel<float><<<(int)nb, 256, 0, s>>>((const float*)q, (float*)q_s, n, q_scale);
    return check_launch("attn_scale");
  }
  float* partial = reinterpret_cast<float*>(guard + 8);
  const int epl = dtype == ALGX_BF16 ? 8 : 4;
  const int rpw = 64 / (D / epl);
  int64_t nb = (rows + 4 * rpw * 4 - 1) / (4 * rpw * 4);
  if (nb < 1) nb = 1;
  if (nb > kGuardBlocks) nb = kGuardBlocks;
#define GUARD_CASE(TT, DD)                                                              \
  prepare_guard_kernel<TT, DD><<<(int)nb, 256, 0, s>>>((const TT*)q, (const TT*)k,      \
                                                       (const TT*)v, (TT*)q_s, rows, q_scale, partial)
  if (dtype == ALGX_BF16) {
    if (D == 64) GUARD_CASE(bf16, 64);
    else if (D == 32) GUARD_CASE(bf16, 32);
    else if (D == 16) GUARD_CASE(bf16, 16);
    else return fail("attn_guard: D must be 16, 32 or 64");
  } else {
    if (D == 64) GUARD_CASE(float, 64);
    else if (D == 32) GUARD_CASE(float, 32);
    else if (D == 16) GUARD_CASE(float, 16);
    else return fail("attn_guard: D must be 16, 32 or 64");
  }
#undef GUARD_CASE
  if (int32_t rc = check_launch("attn_guard_partial")) return rc;
  return launch_guard_finish(partial, (int)nb, sink, H, bound, vmax, guard, s);
}

int32_t launch_guard_finish(const float* partial, int nblocks, const float* sink, int H,
                            float bound, float vmax, int32_t* guard, hipStream_t s) {
  const double b101 = (double)bound / 1.01;
  guard_finish_kernel<<<1, 256, 0, s>>>(partial, nblocks, sink, H, (float)(b101 * b101),
                                        (float)b101, vmax, guard);
  return check_launch("attn_guard_finish");
}

int32_t launch_bwd_pre(const void* dout, const void* o, const float* o_precise,
                       const float* stat, const float* sink, float* di, float* dq_acc,
                       float* dsink, int B, int H, int T, int D, int dtype, const KVariant& low,
                       const KVariant& high, const int32_t* guard, hipStream_t s) {
  if (sink != nullptr && dsink != nullptr)
    if (int32_t rc = fill_f32(dsink, H, 0.0f, s)) return rc;
  const int epl = dtype == ALGX_BF16 ? 8 : 4;
  const int rpw = 64 / (D / epl);
  const int per_block = 4 * rpw * 4;
  dim3 grid((T + per_block - 1) / per_block, B * H);
#define PRE_CASE(TT, DD)                                                                   \
  bwd_pre_kernel<TT, DD><<<grid, 256, 0, s>>>((const TT*)dout, (const TT*)o, o_precise, stat, \
                                              sink, di, dq_acc, dsink, H, T, low, high, guard)
  if (dtype == ALGX_BF16) {
    if (D == 64) PRE_CASE(bf16, 64);
    else if (D == 32) PRE_CASE(bf16, 32);
    else if (D == 16) PRE_CASE(bf16, 16);
    else return fail("attn_bwd: D must be 16, 32 or 64");
  } else {
    if (D == 64) PRE_CASE(float, 64);
    else if (D == 32) PRE_CASE(float, 32);
    else if (D == 16) PRE_CASE(float, 16);
    else return fail("attn_bwd: D must be 16, 32 or 64");
  }
#undef PRE_CASE
  return check_launch("attn_bwd_pre");
}

int32_t launch_dq_finish(const float* acc, void* dq, int64_t n, int dtype, const KVariant& low,
                         const KVariant& high, const int32_t* guard, float q_scale,
                         hipStream_t s) {
  int64_t nb = (n / 4 + 255) / 256;
  if (nb > 8192) nb = 8192;
  if (nb < 1) nb = 1;
  if (dtype == ALGX_BF16)
    dq_finish_kernel<bf16><<<(int)nb, 256, 0, s>>>(acc, (bf16*)dq, n, low, high, guard, q_scale);
  else
    dq_finish_kernel<float><<<(int)nb, 256, 0, s>>>(acc, (float*)dq, n, low, high, guard, q_scale);
  return check_launch("attn_dq_finish");
}

}  // namespace algx
