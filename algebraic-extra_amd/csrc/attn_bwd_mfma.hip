// gfx950 MFMA attention backward (flash.py:333-361 tile VJP, :630-638;
// head_resident.py:95-132).
//
// One workgroup owns 128 keys of one (b, h) (32 per wave; the wave's K and V
// rows stay in registers as MFMA B operands) and walks 64-query tiles from
// the diagonal to T. Each tile is handled as two 32-query halves: S and dP
// are formed with queries on the M axis, so each lane holds one key column
// and 16 queries; p and ds are formed in registers and feed
// dV^T += dO^T P and dK^T += Q_s^T dS directly (dO^T and Q_s^T are staged
// transposed in LDS with the k-slot order the accumulator layout implies).
// The next half's S/dP MFMAs are issued before the current half's dV/dK
// MFMAs so the MFMA pipe runs under the VALU weight/gradient math.
//
// dS goes through LDS once, so that the four waves together form the
// workgroup's dQ tile (64 queries x 64 d over 128 keys), which is added into
// a float32 dQ accumulator with no-return atomics; workgroups of one head sit
// on one XCD, so those atomics resolve in that XCD's L2.
#include <type_traits>

#include "attn_mfma.h"

namespace algx {
namespace mfma {
namespace {

// p and ds of one score (flash.py:339-361); ds already multiplied by r.
template <int MODE, bool FAST, bool BOUNDED, int L2N>
__device__ __forceinline__ void tile_grad(float s, float dp, float st, float dd, float clamp,
                                          int log2n, bool inv_stat, float& p, float& ds) {
  if (MODE == MODE_SOFTMAX) {
    p = __builtin_amdgcn_exp2f((s - st) * kLog2e);
    ds = p * (dp - dd);
    return;
  }
  const float x = (MODE == MODE_NOSHIFT && !BOUNDED) ? __builtin_fminf(s, clamp) : s;
  float r;
  const float rh = FAST ? rho_fast(x, r) : rho_exact(x, r);
  p = (MODE == MODE_NOSHIFT && inv_stat) ? powN<L2N>(rh, log2n) * st : powN<L2N>(rh * st, log2n);
  ds = p * (dp - dd) * r;
  if (MODE == MODE_NOSHIFT && !BOUNDED && !(s < clamp)) ds = 0.0f;
}

struct BwdLds {
  bf16* Qs;
  bf16* Gs;
  bf16* Qt;
  bf16* Gt;
  float* St;
  float* Dt;
  bf16* dSs;
  bf16* Kt;
};

template <int MODE, bool FAST, bool BOUNDED, int L2N>
__device__ __forceinline__ void bwd_body(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const bf16* __restrict__ dout,
    float* __restrict__ dq_acc, bf16* __restrict__ dk, bf16* __restrict__ dv, int T_,
    const KVariant& var, const BwdLds& L) {
  const int nkb = T_ / BBN;
  const int nheads = gridDim.x / nkb;
  int bh, kb;
  map_block(blockIdx.x, nheads, nkb, false, bh, kb);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int64_t base = (int64_t)bh * T_ * HD;
  const int64_t rbase = (int64_t)bh * T_;
  const int key0 = kb * BBN, kw = key0 + 32 * w, kcol = kw + c32;
  const int log2n = var.log2n;
  const bool inv_stat = var.inv_stat;
  const float clamp = var.clamp;

  // B operands: lane holds K[kcol][16ks + 8g ..] and V[kcol][16ks + 8g ..].
  bf16x8 kreg[4], vreg[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    kreg[ks] = *reinterpret_cast<const bf16x8*>(k + base + (int64_t)kcol * HD + 16 * ks + 8 * g);
    vreg[ks] = *reinterpret_cast<const bf16x8*>(v + base + (int64_t)kcol * HD + 16 * ks + 8 * g);
  }
  // K^T of the workgroup's 128 keys (natural key order) for the dQ product.
  {
    const int kg = tid >> 3, dc = tid & 7;
    bf16x8 rows[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      rows[i] = *reinterpret_cast<const bf16x8*>(k + base + (int64_t)(key0 + 4 * kg + i) * HD +
                                                 8 * dc);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      bf16x4 col = {rows[0][d], rows[1][d], rows[2][d], rows[3][d]};
      *reinterpret_cast<bf16x4*>(&L.Kt[(8 * dc + d) * KTSTR + 4 * kg]) = col;
    }
  }

  f32x16 dka[2], dva[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    zero16(dka[dt]);
    zero16(dva[dt]);
  }

  // Loaders: threads 0..127 move Q_s rows, 128..255 move dO rows, 4
  // consecutive queries x 8 d each; threads 0..63 also move stat and di.
  const bool qloader = tid < 128;
  const int u = tid & 127, qg = u >> 3, dc = u & 7;
  bf16x8 pre[4];
  float pst = 0.0f, pdi = 0.0f;
  auto gload = [&](int qt) {
    const int64_t row0 = (int64_t)(qt * BBM + 4 * qg);
    const bf16* src = (qloader ? q : dout) + base + row0 * HD + 8 * dc;
#pragma unroll
    for (int i = 0; i < 4; ++i) pre[i] = *reinterpret_cast<const bf16x8*>(src + i * HD);
    if (tid < BBM) {
      pst = stat[rbase + qt * BBM + tid];
      pdi = di[rbase + qt * BBM + tid];
    }
  };
  auto lstore = [&]() {
    bf16* rowbuf = qloader ? L.Qs : L.Gs;
    bf16* tbuf = qloader ? L.Qt : L.Gt;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<bf16x8*>(&rowbuf[(4 * qg + i) * QSTR + 8 * dc]) = pre[i];
    const int pos = 16 * (qg >> 2) + slot_pos(4 * (qg & 3));
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      bf16x4 col = {pre[0][d], pre[1][d], pre[2][d], pre[3][d]};
      *reinterpret_cast<bf16x4*>(&tbuf[(8 * dc + d) * QTSTR + pos]) = col;
    }
    if (tid < BBM) {
      L.St[tid] = pst;
      L.Dt[tid] = pdi;
    }
  };

  // S and dP of query half mq: acc[r] <-> query 32mq + 8(r/4) + 4g + r%4, key kcol.
  auto half_scores = [&](int mq, f32x16& s, f32x16& dp) {
    zero16(s);
    zero16(dp);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 aq = *reinterpret_cast<const bf16x8*>(&L.Qs[(32 * mq + c32) * QSTR + 16 * ks + 8 * g]);
      const bf16x8 ag = *reinterpret_cast<const bf16x8*>(&L.Gs[(32 * mq + c32) * QSTR + 16 * ks + 8 * g]);
      s = mfma32(aq, kreg[ks], s);
      dp = mfma32(ag, vreg[ks], dp);
    }
  };
  // p, ds of half mq -> bf16 k-slot packs (two 16-query chunks each). Only
  // tiles that cross the diagonal (diag_tag = true_type) evaluate the mask.
  auto half_grads = [&](auto diag_tag, int q0, int mq, const f32x16& s, const f32x16& dp,
                        bf16x8 (&pb)[2], bf16x8 (&db)[2]) {
    constexpr bool DIAG = decltype(diag_tag)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int qo = 32 * mq + 8 * j + 4 * g;
      const f32x4 st4 = *reinterpret_cast<const f32x4*>(&L.St[qo]);
      const f32x4 di4 = *reinterpret_cast<const f32x4*>(&L.Dt[qo]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * j + i;
        float p, ds;
        tile_grad<MODE, FAST, BOUNDED, L2N>(s[r], dp[r], st4[i], di4[i], clamp, log2n, inv_stat,
                                            p, ds);
        if (DIAG && q0 + qo + i < kcol) {
          p = 0.0f;
          ds = 0.0f;
        }
        pb[r >> 3][r & 7] = (bf16)p;
        db[r >> 3][r & 7] = (bf16)ds;
      }
    }
  };
  // dV^T += dO^T P and dK^T += Q_s^T dS over the half's two 16-query chunks;
  // dS of the half -> LDS as [query][key].
  auto half_update = [&](int mq, const bf16x8 (&pb)[2], const bf16x8 (&db)[2]) {
#pragma unroll
    for (int kcl = 0; kcl < 2; ++kcl) {
      const int kc = 2 * mq + kcl;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const bf16x8 ag = *reinterpret_cast<const bf16x8*>(&L.Gt[(32 * dt + c32) * QTSTR + 16 * kc + 8 * g]);
        const bf16x8 aq = *reinterpret_cast<const bf16x8*>(&L.Qt[(32 * dt + c32) * QTSTR + 16 * kc + 8 * g]);
        dva[dt] = mfma32(ag, pb[kcl], dva[dt]);
        dka[dt] = mfma32(aq, db[kcl], dka[dt]);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qo = 32 * mq + 8 * (r >> 2) + 4 * g + (r & 3);
      L.dSs[qo * DSSTR + 32 * w + c32] = db[r >> 3][r & 7];
    }
  };

  const int qt0 = key0 / BBM, nqt = T_ / BBM;
  gload(qt0);
  for (int qt = qt0; qt < nqt; ++qt) {
    __syncthreads();  // previous tile's LDS reads are done
    lstore();
    __syncthreads();
    if (qt + 1 < nqt) gload(qt + 1);
    const int q0 = qt * BBM;
    if (q0 + BBM - 1 >= kw) {
      const bool diag = q0 < kw + 31;
      f32x16 s0, dp0, s1, dp1;
      bf16x8 pb0[2], db0[2], pb1[2], db1[2];
      half_scores(0, s0, dp0);
      if (diag)
        half_grads(std::true_type{}, q0, 0, s0, dp0, pb0, db0);
      else
        half_grads(std::false_type{}, q0, 0, s0, dp0, pb0, db0);
      half_scores(1, s1, dp1);
      half_update(0, pb0, db0);
      if (diag)
        half_grads(std::true_type{}, q0, 1, s1, dp1, pb1, db1);
      else
        half_grads(std::false_type{}, q0, 1, s1, dp1, pb1, db1);
      half_update(1, pb1, db1);
    } else {
#pragma unroll
      for (int mq = 0; mq < 2; ++mq)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qo = 32 * mq + 8 * (r >> 2) + 4 * g + (r & 3);
          L.dSs[qo * DSSTR + 32 * w + c32] = (bf16)0.0f;
        }
    }
    __syncthreads();
    // dQ tile: wave w forms queries 32*(w/2).., d 32*(w%2).. over 128 keys.
    {
      const int mq = w >> 1, dt = w & 1;
      f32x16 acc;
      zero16(acc);
#pragma unroll
      for (int kk = 0; kk < BBN / 16; ++kk) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&L.dSs[(32 * mq + c32) * DSSTR + 16 * kk + 8 * g]);
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(&L.Kt[(32 * dt + c32) * KTSTR + 16 * kk + 8 * g]);
        acc = mfma32(a, b, acc);
      }
      // acc[r]: dQ[q0 + 32mq + 8(r/4) + 4g + r%4][32dt + c32]
      float* dst = dq_acc + base + (int64_t)(q0 + 32 * mq + 4 * g) * HD + 32 * dt + c32;
#pragma unroll
      for (int r = 0; r < 16; ++r) atomicAdd(dst + (int64_t)(8 * (r >> 2) + (r & 3)) * HD, acc[r]);
    }
  }

  // dka[dt][r]: dK[kcol][32dt + 8(r/4) + 4g + r%4] (before the slope n).
  const int64_t krow = base + (int64_t)kcol * HD;
  const float slope = var.slope;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * dt + 8 * j + 4 * g;
      bf16x4 kb4 = {(bf16)(dka[dt][4 * j] * slope), (bf16)(dka[dt][4 * j + 1] * slope),
                    (bf16)(dka[dt][4 * j + 2] * slope), (bf16)(dka[dt][4 * j + 3] * slope)};
      bf16x4 vb4 = {(bf16)dva[dt][4 * j], (bf16)dva[dt][4 * j + 1], (bf16)dva[dt][4 * j + 2],
                    (bf16)dva[dt][4 * j + 3]};
      *reinterpret_cast<bf16x4*>(dk + krow + d) = kb4;
      *reinterpret_cast<bf16x4*>(dv + krow + d) = vb4;
    }
}

template <int LO, int HI>
__global__ __launch_bounds__(256, 2) void bwd_mfma_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const bf16* __restrict__ dout,
    float* __restrict__ dq_acc, bf16* __restrict__ dk, bf16* __restrict__ dv, int T_,
    KVariant lo, KVariant hi, const int32_t* __restrict__ guard) {
  __shared__ __attribute__((aligned(16))) bf16 Qs[BBM * QSTR];
  __shared__ __attribute__((aligned(16))) bf16 Gs[BBM * QSTR];
  __shared__ __attribute__((aligned(16))) bf16 Qt[HD * QTSTR];
  __shared__ __attribute__((aligned(16))) bf16 Gt[HD * QTSTR];
  __shared__ __attribute__((aligned(16))) float St[BBM];
  __shared__ __attribute__((aligned(16))) float Dt[BBM];
  __shared__ __attribute__((aligned(16))) bf16 dSs[BBM * DSSTR];
  __shared__ __attribute__((aligned(16))) bf16 Kt[HD * KTSTR];
  const BwdLds lds{Qs, Gs, Qt, Gt, St, Dt, dSs, Kt};
  if (LO == HI || guard_in_range(guard))
    bwd_body<LO & 3, (LO & 4) != 0, (LO & 8) != 0, (LO >> 4)>(q, k, v, stat, di, dout, dq_acc, dk,
                                                              dv, T_, lo, lds);
  else
    bwd_body<HI & 3, (HI & 4) != 0, (HI & 8) != 0, (HI >> 4)>(q, k, v, stat, di, dout, dq_acc, dk,
                                                              dv, T_, hi, lds);
}

typedef void (*BwdFn)(const bf16*, const bf16*, const bf16*, const float*, const float*,
                      const bf16*, float*, bf16*, bf16*, int, KVariant, KVariant,
                      const int32_t*);

BwdFn pick_bwd(int cl, int ch) { ALGX_PICK_ALL(bwd_mfma_kernel) }

}  // namespace
}  // namespace mfma

int32_t launch_bwd_mfma(const void* q, const void* k, const void* v, const float* stat,
                        const float* di, const void* dout, float* dq_acc, void* dk, void* dv,
                        int B, int H, int T, const KVariant& lo, const KVariant& hi,
                        const int32_t* guard, hipStream_t s) {
  using namespace mfma;
  const int grid = B * H * (T / BBN);
  BwdFn fn = pick_bwd(cfg_for(lo), guard != nullptr ? cfg_for(hi) : cfg_for(lo));
  if (fn == nullptr) return fail("attn_bwd: no MFMA kernel for this variant pair");
  ProbeScope probe(ALGX_PROBE_ATTN_BWD, s);
  fn<<<grid, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v, stat, di,
                          (const bf16*)dout, dq_acc, (bf16*)dk, (bf16*)dv, T, lo, hi, guard);
  return check_launch("attn_bwd_mfma");
}

}  // namespace algx
