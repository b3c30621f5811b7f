// Generic attention kernels: one thread per query (forward, dQ) or key
// (dK/dV) row, K/V or Q/dO tiles staged in LDS as float32, every numeric
// variant of flash.py, float32 or bf16 storage, D in {16, 32, 64}, any T.
//
// These carry the float32 parity path (float32 FMA throughout) and every
// shape the MFMA kernels do not take. Numerics follow flash.py:189-284
// (forward) and flash.py:333-361 (tile VJP), with the reference's rounding
// points: p -> storage dtype before PV and dV, ds -> storage dtype before dK
// and dQ, outputs cast at the end.
#include "attn_aux.h"

namespace algx {

namespace {

constexpr int kTile = 64;

template <typename T, int D>
__global__ __launch_bounds__(kTile) void fwd_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ sink, T* __restrict__ o, float* __restrict__ o_precise,
    float* __restrict__ stat, int H, int T_, KVariant var, const int32_t* __restrict__ guard,
    int want_low) {
  if (guard != nullptr && (int)guard_in_range(guard) != want_low) return;
  const int bh = blockIdx.y, h = bh % H, t = threadIdx.x;
  const int i = blockIdx.x * kTile + t;
  const bool valid = i < T_;
  const int64_t base = (int64_t)bh * T_ * D;
  __shared__ float Ks[kTile][D];
  __shared__ float Vs[kTile][D];
  float qr[D], acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qr[d] = valid ? to_f(q[base + (int64_t)i * D + d]) : 0.0f;
    acc[d] = 0.0f;
  }
  const bool has_sink = sink != nullptr;
  float m, l;
  sink_init(var, has_sink, has_sink ? sink[h] : 0.0f, m, l);
  const bool noshift = var.kind == ALGX_ASINH && !var.shift;
  const int last = min(T_ - 1, (int)blockIdx.x * kTile + kTile - 1);
  const int nkt = last / kTile + 1;
  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();
    const int j = kt * kTile + t;
#pragma unroll 8
    for (int d = 0; d < D; ++d) {
      Ks[t][d] = j < T_ ? to_f(k[base + (int64_t)j * D + d]) : 0.0f;
      Vs[t][d] = j < T_ ? to_f(v[base + (int64_t)j * D + d]) : 0.0f;
    }
    __syncthreads();
    if (!valid) continue;
    const int jmax = min(kTile - 1, i - kt * kTile);
    float s[kTile];
    float tmax = -__builtin_inff();
#pragma unroll
    for (int jj = 0; jj < kTile; ++jj) {
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) dot = __builtin_fmaf(qr[d], Ks[jj][d], dot);
      s[jj] = dot;
      if (jj <= jmax) tmax = __builtin_fmaxf(tmax, dot);
    }
    if (noshift) {
      for (int jj = 0; jj <= jmax; ++jj) {
        const float x = var.bounded ? s[jj] : __builtin_fminf(s[jj], var.clamp);
        float r;
        const float p = pow2n(rho_of(var, x, r), var.log2n);
        l += p;
        const float pb = round_to<T>(p);
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(pb, Vs[jj][d], acc[d]);
      }
      continue;
    }
    float m_new = __builtin_fmaxf(m, tmax), m_prev = m;
    if (!has_sink && kt == 0) {  // flash.py:239-245
      m_new = tmax;
      m_prev = m_new;
    }
    float alpha, shf = 0.0f;
    if (var.kind == ALGX_SOFTMAX) {
      alpha = __expf(m_prev - m_new);
    } else {
      float r;
      shf = rho_exact(-m_new, r);
      alpha = pow2n(rho_exact(m_prev, r) * shf, var.log2n);
    }
    l *= alpha;
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] *= alpha;
    for (int jj = 0; jj <= jmax; ++jj) {
      float p;
      if (var.kind == ALGX_SOFTMAX) {
        p = __expf(s[jj] - m_new);
      } else {
        float r;
        p = pow2n(rho_var(s[jj], var.fast, r) * shf, var.log2n);
      }
      l += p;
      const float pb = round_to<T>(p);
#pragma unroll
      for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(pb, Vs[jj][d], acc[d]);
    }
    m = m_new;
  }
  if (!valid) return;
  const float inv = 1.0f / l;
  const int64_t row = base + (int64_t)i * D;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const float val = acc[d] * inv;
    o[row + d] = from_f<T>(val);
    if (var.precise && o_precise != nullptr) o_precise[row + d] = val;
  }
  stat[(int64_t)bh * T_ + i] = final_stat(var, m, l);
}

// dK, dV: one thread per key row; query tiles from the key's tile onwards.
template <typename T, int D>
__global__ __launch_bounds__(kTile) void bwd_dkdv_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const T* __restrict__ dout,
    T* __restrict__ dk, T* __restrict__ dv, int T_, KVariant var,
    const int32_t* __restrict__ guard, int want_low) {
  if (guard != nullptr && (int)guard_in_range(guard) != want_low) return;
  const int bh = blockIdx.y, t = threadIdx.x;
  const int j = blockIdx.x * kTile + t;
  const bool valid = j < T_;
  const int64_t base = (int64_t)bh * T_ * D;
  __shared__ float Qs[kTile][D];
  __shared__ float Gs[kTile][D];
  __shared__ float Ss[kTile];
  __shared__ float Ds[kTile];
  float kr[D], vr[D], dka[D], dva[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    kr[d] = valid ? to_f(k[base + (int64_t)j * D + d]) : 0.0f;
    vr[d] = valid ? to_f(v[base + (int64_t)j * D + d]) : 0.0f;
    dka[d] = 0.0f;
    dva[d] = 0.0f;
  }
  const bool asinh = var.kind == ALGX_ASINH;
  const int nqt = (T_ + kTile - 1) / kTile;
  for (int qt = blockIdx.x; qt < nqt; ++qt) {
    __syncthreads();
    const int i = qt * kTile + t;
#pragma unroll 8
    for (int d = 0; d < D; ++d) {
      Qs[t][d] = i < T_ ? to_f(q[base + (int64_t)i * D + d]) : 0.0f;
      Gs[t][d] = i < T_ ? to_f(dout[base + (int64_t)i * D + d]) : 0.0f;
    }
    Ss[t] = i < T_ ? stat[(int64_t)bh * T_ + i] : 0.0f;
    Ds[t] = i < T_ ? di[(int64_t)bh * T_ + i] : 0.0f;
    __syncthreads();
    if (!valid) continue;
    for (int ii = 0; ii < kTile; ++ii) {
      const int iq = qt * kTile + ii;
      if (iq < j || iq >= T_) continue;
      float s = 0.0f, dp = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        s = __builtin_fmaf(Qs[ii][d], kr[d], s);
        dp = __builtin_fmaf(Gs[ii][d], vr[d], dp);
      }
      float rr;
      bool keep;
      const float p = bwd_weight(var, s, Ss[ii], rr, keep);
      float ds = p * (dp - Ds[ii]);
      if (asinh) ds = keep ? ds * rr : 0.0f;
      const float pb = round_to<T>(p), dsb = round_to<T>(ds);
#pragma unroll
      for (int d = 0; d < D; ++d) {
        dva[d] = __builtin_fmaf(pb, Gs[ii][d], dva[d]);
        dka[d] = __builtin_fmaf(dsb, Qs[ii][d], dka[d]);
      }
    }
  }
  if (!valid) return;
  const int64_t row = base + (int64_t)j * D;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    dk[row + d] = from_f<T>(dka[d] * var.slope);
    dv[row + d] = from_f<T>(dva[d]);
  }
}

// dQ: one thread per query row; key tiles up to the diagonal. Writes the
// final dq = cast(cast(dq_s * slope) * q_scale).
template <typename T, int D>
__global__ __launch_bounds__(kTile) void bwd_dq_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const T* __restrict__ dout,
    T* __restrict__ dq, int T_, float q_scale, KVariant var, const int32_t* __restrict__ guard,
    int want_low) {
  if (guard != nullptr && (int)guard_in_range(guard) != want_low) return;
  const int bh = blockIdx.y, t = threadIdx.x;
  const int i = blockIdx.x * kTile + t;
  const bool valid = i < T_;
  const int64_t base = (int64_t)bh * T_ * D;
  __shared__ float Ks[kTile][D];
  __shared__ float Vs[kTile][D];
  float qr[D], gr[D], dqa[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qr[d] = valid ? to_f(q[base + (int64_t)i * D + d]) : 0.0f;
    gr[d] = valid ? to_f(dout[base + (int64_t)i * D + d]) : 0.0f;
    dqa[d] = 0.0f;
  }
  const float st = valid ? stat[(int64_t)bh * T_ + i] : 0.0f;
  const float dd = valid ? di[(int64_t)bh * T_ + i] : 0.0f;
  const bool asinh = var.kind == ALGX_ASINH;
  const int last = min(T_ - 1, (int)blockIdx.x * kTile + kTile - 1);
  const int nkt = last / kTile + 1;
  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();
    const int j = kt * kTile + t;
#pragma unroll 8
    for (int d = 0; d < D; ++d) {
      Ks[t][d] = j < T_ ? to_f(k[base + (int64_t)j * D + d]) : 0.0f;
      Vs[t][d] = j < T_ ? to_f(v[base + (int64_t)j * D + d]) : 0.0f;
    }
    __syncthreads();
    if (!valid) continue;
    const int jmax = min(kTile - 1, i - kt * kTile);
    for (int jj = 0; jj <= jmax; ++jj) {
      float s = 0.0f, dp = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        s = __builtin_fmaf(qr[d], Ks[jj][d], s);
        dp = __builtin_fmaf(gr[d], Vs[jj][d], dp);
      }
      float rr;
      bool keep;
      const float p = bwd_weight(var, s, st, rr, keep);
      float ds = p * (dp - dd);
      if (asinh) ds = keep ? ds * rr : 0.0f;
      const float dsb = round_to<T>(ds);
#pragma unroll
      for (int d = 0; d < D; ++d) dqa[d] = __builtin_fmaf(dsb, Ks[jj][d], dqa[d]);
    }
  }
  if (!valid) return;
  const int64_t row = base + (int64_t)i * D;
#pragma unroll
  for (int d = 0; d < D; ++d) dq[row + d] = from_f<T>(round_to<T>(dqa[d] * var.slope) * q_scale);
}

}  // namespace

int32_t launch_fwd_generic(const void* q, const void* k, const void* v, const float* sink,
                           void* o, float* o_precise, float* stat, int B, int H, int T, int D,
                           int dtype, const KVariant& var, const int32_t* guard, int want_low,
                           hipStream_t s) {
  dim3 grid((T + kTile - 1) / kTile, B * H);
#define FWD_CASE(TT, DD)                                                                      \
  fwd_generic_kernel<TT, DD><<<grid, kTile, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, \
                                                    sink, (TT*)o, o_precise, stat, H, T, var, \
                                                    guard, want_low)
  if (dtype == ALGX_BF16) {
    if (D == 64) FWD_CASE(bf16, 64);
    else if (D == 32) FWD_CASE(bf16, 32);
    else if (D == 16) FWD_CASE(bf16, 16);
    else return fail("attn_fwd: D must be 16, 32 or 64");
  } else {
    if (D == 64) FWD_CASE(float, 64);
    else if (D == 32) FWD_CASE(float, 32);
    else if (D == 16) FWD_CASE(float, 16);
    else return fail("attn_fwd: D must be 16, 32 or 64");
  }
#undef FWD_CASE
  return check_launch("attn_fwd_generic");
}

int32_t launch_bwd_generic(const void* q, const void* k, const void* v, const float* stat,
                           const float* di, const void* dout, void* dq, void* dk, void* dv,
                           int B, int H, int T, int D, int dtype, float q_scale,
                           const KVariant& var, const int32_t* guard, int want_low,
                           hipStream_t s) {
  dim3 grid((T + kTile - 1) / kTile, B * H);
#define BWD_CASE(TT, DD)                                                                        \
  do {                                                                                          \
    bwd_dkdv_generic_kernel<TT, DD><<<grid, kTile, 0, s>>>(                                     \
        (const TT*)q, (const TT*)k, (const TT*)v, stat, di, (const TT*)dout, (TT*)dk, (TT*)dv, \
        T, var, guard, want_low);                                                               \
    bwd_dq_generic_kernel<TT, DD><<<grid, kTile, 0, s>>>((const TT*)q, (const TT*)k,            \
                                                         (const TT*)v, stat, di,                \
                                                         (const TT*)dout, (TT*)dq, T, q_scale,  \
                                                         var, guard, want_low);                 \
  } while (0)
  if (dtype == ALGX_BF16) {
    if (D == 64) BWD_CASE(bf16, 64);
    else if (D == 32) BWD_CASE(bf16, 32);
    else if (D == 16) BWD_CASE(bf16, 16);
    else return fail("attn_bwd: D must be 16, 32 or 64");
  } else {
    if (D == 64) BWD_CASE(float, 64);
    else if (D == 32) BWD_CASE(float, 32);
    else if (D == 16) BWD_CASE(float, 16);
    else return fail("attn_bwd: D must be 16, 32 or 64");
  }
#undef BWD_CASE
  return check_launch("attn_bwd_generic");
}

}  // namespace algx
