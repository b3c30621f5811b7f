// gfx950 MFMA attention kernels: bf16 operands, float32 accumulation, D = 64.
//
// Forward (flash.py:189-284, head_resident.py:24-93): one workgroup of 4
// waves owns 128 queries of one (b, h); each wave owns 32 of them and walks
// 64-key tiles up to the diagonal. The score tile is formed transposed,
// S^T = K Q^T, with v_mfma_f32_32x32x16_bf16 (K from LDS as the A operand,
// the wave's scaled Q rows held in registers as the B operand), so that each
// lane ends up holding 16 keys of ONE query row. The asinh/softmax weight, the
// causal mask and the row sum run on those registers; the bf16 weights are
// then fed straight back as the B operand of O^T += V^T P^T, whose A operand
// is a transposed V tile in LDS. The k-slot order that the accumulator
// layout implies (16-key chunks with bits 2 and 3 of the key offset swapped)
// is applied when V is transposed into LDS, so no register shuffle is needed.
//
// Backward (flash.py:333-361 tile VJP; head_resident.py:95-132): one
// workgroup owns 128 keys (32 per wave, K and V in registers) and walks
// 64-query tiles from the diagonal to T. S and dP are formed with queries on
// the M axis so each lane holds one key column; p and ds are formed in
// registers and feed dV^T += dO^T P and dK^T += Q_s^T dS directly (dO^T and
// Q_s^T are staged transposed in LDS with the same k-slot order). dS goes
// through LDS once so the four waves together form the workgroup's dQ tile
// (64 queries x 64 d over 128 keys), which is added into a float32 dQ
// accumulator with no-return atomics.
//
// Workgroups of one head are placed on one XCD (blockIdx % 8 selects the
// XCD) so that the head's K/V (forward) and dQ accumulator rows (backward)
// stay in that XCD's L2; the heaviest causal tiles launch first.
#include "attn_aux.h"

namespace algx {

namespace {

constexpr int HD = 64;
// forward tiles
constexpr int FBM = 128, FBN = 64;
constexpr int KSTR = 72;  // K tile row stride (bf16): 144 B rows
constexpr int VSTR = 72;  // V^T tile row stride
// backward tiles
constexpr int BBN = 128, BBM = 64;
constexpr int QSTR = 72;   // Q_s / dO row stride (64 d)
constexpr int QTSTR = 72;  // Q_s^T / dO^T row stride (64 q)
constexpr int DSSTR = 136; // dS row stride (128 keys)
constexpr int KTSTR = 136; // K^T row stride (128 keys)

enum { MODE_SOFTMAX = 0, MODE_NOSHIFT = 1, MODE_SHIFT = 2 };

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Position of key offset `off` (0..15) inside a 16-key chunk of a transposed
// operand tile: bits 2 and 3 swapped, i.e. k-slot (g, s) of lane group g holds
// key offset 8*(s/4) + 4*g + s%4, matching the 32x32 accumulator layout.
__device__ __forceinline__ int slot_pos(int off) {
  return (off & 3) | ((off >> 3) & 1) << 2 | ((off >> 2) & 1) << 3;
}

// blockIdx -> (head, tile); heads are dealt to XCDs so every tile of a head
// runs on the same XCD; `heavy_last` orders tiles by decreasing work.
__device__ __forceinline__ void map_block(int bid, int nheads, int ntiles, bool descending,
                                          int& bh, int& tile) {
  int r;
  if ((nheads & 7) == 0) {
    const int nh8 = nheads >> 3;
    r = bid >> 3;
    bh = (bid & 7) + 8 * (r % nh8);
    r = r / nh8;
  } else {
    bh = bid % nheads;
    r = bid / nheads;
  }
  tile = descending ? ntiles - 1 - r : r;
}

__device__ __forceinline__ bf16x8 scale_bf16x8(bf16x8 x, float s) {
  bf16x8 y;
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = (bf16)((float)x[e] * s);
  return y;
}

// x^(2^log2n) with a compile-time exponent when L2N > 0.
template <int L2N> __device__ __forceinline__ float powN(float x, int log2n) {
  if (L2N > 0) {
#pragma unroll
    for (int i = 0; i < L2N; ++i) x = x * x;
    return x;
  }
  return pow2n(x, log2n);
}

template <int MODE, bool FAST, bool BOUNDED, int L2N>
__global__ __launch_bounds__(256) void fwd_mfma_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ sink, bf16* __restrict__ o, float* __restrict__ o_precise,
    float* __restrict__ stat, int H, int T_, float q_scale, KVariant var,
    const int32_t* __restrict__ guard, int want_low) {
  if (guard != nullptr && (int)guard_in_range(guard) != want_low) return;
  const int nheads = gridDim.x / (T_ / FBM);
  int bh, qb;
  map_block(blockIdx.x, nheads, T_ / FBM, true, bh, qb);
  const int h = bh % H;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int64_t base = (int64_t)bh * T_ * HD;
  const int q0 = qb * FBM, qw = q0 + 32 * w, qrow = qw + c32;

  __shared__ __attribute__((aligned(16))) bf16 Ks[2][FBN * KSTR];
  __shared__ __attribute__((aligned(16))) bf16 Vt[2][HD * VSTR];

  // B operand of S^T = K Q_s^T: lane holds Q_s[qrow][16*ks + 8*g .. +7].
  bf16x8 qreg[4];
  {
    const bf16* qp = q + base + (int64_t)qrow * HD + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qreg[ks] = scale_bf16x8(*reinterpret_cast<const bf16x8*>(qp + 16 * ks), q_scale);
  }

  const bool has_sink = sink != nullptr;
  float m_row, l_row;
  sink_init(var, has_sink, has_sink ? sink[h] : 0.0f, m_row, l_row);
  if (g == 1) l_row = 0.0f;  // the two lane halves carry partial row sums
  f32x16 oacc[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.0f;

  // Tile loaders: threads 0..127 move K rows, 128..255 move V rows of 4 keys.
  bf16x8 pre[4];
  const bool kloader = tid < 128;
  const int u = tid & 127;
  auto gload = [&](int kb) {
    const bf16* src = (kloader ? k : v) + base + (int64_t)kb * FBN * HD;
    if (kloader) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int id = u + 128 * c;
        pre[c] = *reinterpret_cast<const bf16x8*>(src + (id >> 3) * HD + (id & 7) * 8);
      }
    } else {
      const int kg = u >> 3, dc = u & 7;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pre[i] = *reinterpret_cast<const bf16x8*>(src + (4 * kg + i) * HD + 8 * dc);
    }
  };
  auto lstore = [&](int buf) {
    if (kloader) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int id = u + 128 * c;
        *reinterpret_cast<bf16x8*>(&Ks[buf][(id >> 3) * KSTR + (id & 7) * 8]) = pre[c];
      }
    } else {
      const int kg = u >> 3, dc = u & 7;
      const int pos = 16 * (kg >> 2) + slot_pos(4 * (kg & 3));
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        bf16x4 col = {pre[0][d], pre[1][d], pre[2][d], pre[3][d]};
        *reinterpret_cast<bf16x4*>(&Vt[buf][(8 * dc + d) * VSTR + pos]) = col;
      }
    }
  };

  const int nkb = (q0 + FBM) / FBN;
  gload(0);
  lstore(0);
  __syncthreads();
  const int log2n = var.log2n;
  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) gload(kb + 1);
    const int k0 = kb * FBN;
    if (k0 <= qw + 31) {
      const bool diag = k0 + FBN - 1 > qw;
      f32x16 sacc[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[mt][r] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 a =
              *reinterpret_cast<const bf16x8*>(&Ks[buf][(32 * mt + c32) * KSTR + 16 * ks + 8 * g]);
          sacc[mt] = mfma32(a, qreg[ks], sacc[mt]);
        }
      }
      // sacc[mt][r]: score of query qrow with key k0 + 32mt + 8(r/4) + 4g + r%4.
      float lsum = 0.0f;
      if (MODE == MODE_NOSHIFT) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float s = sacc[mt][r];
            const float x = BOUNDED ? s : __builtin_fminf(s, var.clamp);
            float rr;
            float p = powN<L2N>(FAST ? rho_fast(x, rr) : rho_exact(x, rr), log2n);
            if (diag) {
              const int key = k0 + 32 * mt + 8 * (r >> 2) + 4 * g + (r & 3);
              if (key > qrow) p = 0.0f;
            }
            sacc[mt][r] = p;
            lsum += p;
          }
        l_row += lsum;
      } else {
        float tmax = -__builtin_inff();
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float s = sacc[mt][r];
            if (diag) {
              const int key = k0 + 32 * mt + 8 * (r >> 2) + 4 * g + (r & 3);
              if (key > qrow) s = -__builtin_inff();
            }
            sacc[mt][r] = s;
            tmax = __builtin_fmaxf(tmax, s);
          }
        tmax = __builtin_fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        float m_new = __builtin_fmaxf(m_row, tmax), m_prev = m_row;
        if (!has_sink && kb == 0) {  // flash.py:239-245
          m_new = tmax;
          m_prev = m_new;
        }
        float alpha;
        if (MODE == MODE_SOFTMAX) {
          alpha = __builtin_amdgcn_exp2f((m_prev - m_new) * kLog2e);
          const float mb = m_new * kLog2e;
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[mt][r], kLog2e, -mb));
              sacc[mt][r] = p;
              lsum += p;
            }
        } else {
          float rr;
          const float shf = rho_exact(-m_new, rr);
          alpha = powN<L2N>(rho_exact(m_prev, rr) * shf, log2n);
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float s = sacc[mt][r];
              float p = powN<L2N>((FAST ? rho_fast(s, rr) : rho_exact(s, rr)) * shf, log2n);
              if (s == -__builtin_inff()) p = 0.0f;
              sacc[mt][r] = p;
              lsum += p;
            }
        }
        l_row = __builtin_fmaf(l_row, alpha, lsum);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        m_row = m_new;
      }
      // O^T += V^T P^T over four 16-key chunks.
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const int mt = kc >> 1, rr = 8 * (kc & 1);
        bf16x8 pb;
#pragma unroll
        for (int s = 0; s < 8; ++s) pb[s] = (bf16)sacc[mt][rr + s];
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const bf16x8 a =
              *reinterpret_cast<const bf16x8*>(&Vt[buf][(32 * dt + c32) * VSTR + 16 * kc + 8 * g]);
          oacc[dt] = mfma32(a, pb, oacc[dt]);
        }
      }
    }
    if (kb + 1 < nkb) lstore(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = l_row + __shfl_xor(l_row, 32, 64);
  const float inv = 1.0f / l_tot;
  const int64_t orow = base + (int64_t)qrow * HD;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * dt + 8 * j + 4 * g;
      f32x4 val;
#pragma unroll
      for (int i = 0; i < 4; ++i) val[i] = oacc[dt][4 * j + i] * inv;
      bf16x4 ob = {(bf16)val[0], (bf16)val[1], (bf16)val[2], (bf16)val[3]};
      *reinterpret_cast<bf16x4*>(o + orow + d) = ob;
      if (MODE == MODE_SHIFT && var.precise && o_precise != nullptr)
        *reinterpret_cast<f32x4*>(o_precise + orow + d) = val;
    }
  if (g == 0) stat[(int64_t)bh * T_ + qrow] = final_stat(var, m_row, l_tot);
}

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

template <int MODE, bool FAST, bool BOUNDED, int L2N>
__global__ __launch_bounds__(256, 2) void bwd_mfma_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const bf16* __restrict__ dout,
    float* __restrict__ dq_acc, bf16* __restrict__ dk, bf16* __restrict__ dv, int T_,
    float q_scale, KVariant var, const int32_t* __restrict__ guard, int want_low) {
  if (guard != nullptr && (int)guard_in_range(guard) != want_low) return;
  const int nkb = T_ / BBN;
  const int nheads = gridDim.x / nkb;
  int bh, kb;
  map_block(blockIdx.x, nheads, nkb, false, bh, kb);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int64_t base = (int64_t)bh * T_ * HD;
  const int64_t rbase = (int64_t)bh * T_;
  const int key0 = kb * BBN, kw = key0 + 32 * w, kcol = kw + c32;

  __shared__ __attribute__((aligned(16))) bf16 Qs[BBM * QSTR];
  __shared__ __attribute__((aligned(16))) bf16 Gs[BBM * QSTR];
  __shared__ __attribute__((aligned(16))) bf16 Qt[HD * QTSTR];
  __shared__ __attribute__((aligned(16))) bf16 Gt[HD * QTSTR];
  __shared__ __attribute__((aligned(16))) float St[BBM];
  __shared__ __attribute__((aligned(16))) float Dt[BBM];
  __shared__ __attribute__((aligned(16))) bf16 dSs[BBM * DSSTR];
  __shared__ __attribute__((aligned(16))) bf16 Kt[HD * KTSTR];

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
      *reinterpret_cast<bf16x4*>(&Kt[(8 * dc + d) * KTSTR + 4 * kg]) = col;
    }
  }

  f32x16 dka[2], dva[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dka[dt][r] = 0.0f;
      dva[dt][r] = 0.0f;
    }

  // Loaders: threads 0..127 move Q rows (scaled), 128..255 move dO rows,
  // 4 consecutive queries x 8 d each; threads 0..63 also move stat and di.
  const bool qloader = tid < 128;
  const int u = tid & 127, qg = u >> 3, dc = u & 7;
  bf16x8 pre[4];
  float pst = 0.0f, pdi = 0.0f;
  auto gload = [&](int qt) {
    const int64_t row0 = (int64_t)(qt * BBM + 4 * qg);
    const bf16* src = (qloader ? q : dout) + base + row0 * HD + 8 * dc;
#pragma unroll
    for (int i = 0; i < 4; ++i) pre[i] = *reinterpret_cast<const bf16x8*>(src + i * HD);
    if (qloader) {
#pragma unroll
      for (int i = 0; i < 4; ++i) pre[i] = scale_bf16x8(pre[i], q_scale);
    }
    if (tid < BBM) {
      pst = stat[rbase + qt * BBM + tid];
      pdi = di[rbase + qt * BBM + tid];
    }
  };
  auto lstore = [&]() {
    bf16* rowbuf = qloader ? Qs : Gs;
    bf16* tbuf = qloader ? Qt : Gt;
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
      St[tid] = pst;
      Dt[tid] = pdi;
    }
  };

  const int qt0 = key0 / BBM, nqt = T_ / BBM;
  const int log2n = var.log2n;
  const bool inv_stat = var.inv_stat;
  const float clamp = var.clamp;
  gload(qt0);
  for (int qt = qt0; qt < nqt; ++qt) {
    __syncthreads();  // previous tile's LDS reads are done
    lstore();
    __syncthreads();
    if (qt + 1 < nqt) gload(qt + 1);
    const int q0 = qt * BBM;
    if (q0 + BBM - 1 >= kw) {
      const bool diag = q0 < kw + 31;
      f32x16 sacc[2], pacc[2];
#pragma unroll
      for (int mq = 0; mq < 2; ++mq) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sacc[mq][r] = 0.0f;
          pacc[mq][r] = 0.0f;
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 aq =
              *reinterpret_cast<const bf16x8*>(&Qs[(32 * mq + c32) * QSTR + 16 * ks + 8 * g]);
          const bf16x8 ag =
              *reinterpret_cast<const bf16x8*>(&Gs[(32 * mq + c32) * QSTR + 16 * ks + 8 * g]);
          sacc[mq] = mfma32(aq, kreg[ks], sacc[mq]);
          pacc[mq] = mfma32(ag, vreg[ks], pacc[mq]);
        }
      }
      // sacc[mq][r]: score of query q0 + 32mq + 8(r/4) + 4g + r%4 with key kcol.
#pragma unroll
      for (int mq = 0; mq < 2; ++mq)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int qo = 32 * mq + 8 * j + 4 * g;
          const f32x4 st4 = *reinterpret_cast<const f32x4*>(&St[qo]);
          const f32x4 di4 = *reinterpret_cast<const f32x4*>(&Dt[qo]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float p, ds;
            tile_grad<MODE, FAST, BOUNDED, L2N>(sacc[mq][4 * j + i], pacc[mq][4 * j + i], st4[i],
                                           di4[i], clamp, log2n, inv_stat, p, ds);
            if (diag && q0 + qo + i < kcol) {
              p = 0.0f;
              ds = 0.0f;
            }
            sacc[mq][4 * j + i] = p;
            pacc[mq][4 * j + i] = ds;
          }
        }
      // dV^T += dO^T P and dK^T += Q_s^T dS over four 16-query chunks.
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const int mq = kc >> 1, rr = 8 * (kc & 1);
        bf16x8 pb, db;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          pb[s] = (bf16)sacc[mq][rr + s];
          db[s] = (bf16)pacc[mq][rr + s];
        }
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const bf16x8 ag =
              *reinterpret_cast<const bf16x8*>(&Gt[(32 * dt + c32) * QTSTR + 16 * kc + 8 * g]);
          const bf16x8 aq =
              *reinterpret_cast<const bf16x8*>(&Qt[(32 * dt + c32) * QTSTR + 16 * kc + 8 * g]);
          dva[dt] = mfma32(ag, pb, dva[dt]);
          dka[dt] = mfma32(aq, db, dka[dt]);
        }
      }
      // dS (bf16) -> LDS as [query][key] for the workgroup dQ product.
#pragma unroll
      for (int mq = 0; mq < 2; ++mq)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qo = 32 * mq + 8 * (r >> 2) + 4 * g + (r & 3);
          dSs[qo * DSSTR + 32 * w + c32] = (bf16)pacc[mq][r];
        }
    } else {
#pragma unroll
      for (int mq = 0; mq < 2; ++mq)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qo = 32 * mq + 8 * (r >> 2) + 4 * g + (r & 3);
          dSs[qo * DSSTR + 32 * w + c32] = (bf16)0.0f;
        }
    }
    __syncthreads();
    // dQ tile: wave w forms queries 32*(w/2).., d 32*(w%2).. over 128 keys.
    {
      const int mq = w >> 1, dt = w & 1;
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
      for (int kk = 0; kk < BBN / 16; ++kk) {
        const bf16x8 a =
            *reinterpret_cast<const bf16x8*>(&dSs[(32 * mq + c32) * DSSTR + 16 * kk + 8 * g]);
        const bf16x8 b =
            *reinterpret_cast<const bf16x8*>(&Kt[(32 * dt + c32) * KTSTR + 16 * kk + 8 * g]);
        acc = mfma32(a, b, acc);
      }
      // acc[r]: dQ[q0 + 32mq + 8(r/4) + 4g + r%4][32dt + c32]
      float* dst = dq_acc + base + (int64_t)(q0 + 32 * mq + 4 * g) * HD + 32 * dt + c32;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        atomicAdd(dst + (int64_t)(8 * (r >> 2) + (r & 3)) * HD, acc[r]);
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

typedef void (*FwdFn)(const bf16*, const bf16*, const bf16*, const float*, bf16*, float*, float*,
                      int, int, float, KVariant, const int32_t*, int);
typedef void (*BwdFn)(const bf16*, const bf16*, const bf16*, const float*, const float*,
                      const bf16*, float*, bf16*, bf16*, int, float, KVariant, const int32_t*,
                      int);

template <int MODE, bool FAST, bool BOUNDED>
FwdFn fwd_by_power(int log2n) {
  switch (log2n) {
    case 3: return fwd_mfma_kernel<MODE, FAST, BOUNDED, 3>;
    case 4: return fwd_mfma_kernel<MODE, FAST, BOUNDED, 4>;
    case 5: return fwd_mfma_kernel<MODE, FAST, BOUNDED, 5>;
    default: return fwd_mfma_kernel<MODE, FAST, BOUNDED, 0>;
  }
}

template <int MODE, bool FAST, bool BOUNDED>
BwdFn bwd_by_power(int log2n) {
  switch (log2n) {
    case 3: return bwd_mfma_kernel<MODE, FAST, BOUNDED, 3>;
    case 4: return bwd_mfma_kernel<MODE, FAST, BOUNDED, 4>;
    case 5: return bwd_mfma_kernel<MODE, FAST, BOUNDED, 5>;
    default: return bwd_mfma_kernel<MODE, FAST, BOUNDED, 0>;
  }
}

FwdFn pick_fwd(const KVariant& v) {
  if (v.kind == ALGX_SOFTMAX) return fwd_mfma_kernel<MODE_SOFTMAX, false, false, 1>;
  if (v.shift)
    return v.fast ? fwd_by_power<MODE_SHIFT, true, false>(v.log2n)
                  : fwd_by_power<MODE_SHIFT, false, false>(v.log2n);
  if (v.bounded)
    return v.fast ? fwd_by_power<MODE_NOSHIFT, true, true>(v.log2n)
                  : fwd_by_power<MODE_NOSHIFT, false, true>(v.log2n);
  return v.fast ? fwd_by_power<MODE_NOSHIFT, true, false>(v.log2n)
                : fwd_by_power<MODE_NOSHIFT, false, false>(v.log2n);
}

BwdFn pick_bwd(const KVariant& v) {
  if (v.kind == ALGX_SOFTMAX) return bwd_mfma_kernel<MODE_SOFTMAX, false, false, 1>;
  if (v.shift)
    return v.fast ? bwd_by_power<MODE_SHIFT, true, false>(v.log2n)
                  : bwd_by_power<MODE_SHIFT, false, false>(v.log2n);
  if (v.bounded)
    return v.fast ? bwd_by_power<MODE_NOSHIFT, true, true>(v.log2n)
                  : bwd_by_power<MODE_NOSHIFT, false, true>(v.log2n);
  return v.fast ? bwd_by_power<MODE_NOSHIFT, true, false>(v.log2n)
                : bwd_by_power<MODE_NOSHIFT, false, false>(v.log2n);
}

}  // namespace

bool mfma_supported(int T, int D, int dtype) {
  return dtype == ALGX_BF16 && D == HD && T >= FBM && T % FBM == 0 && T % BBN == 0;
}

int32_t launch_fwd_mfma(const void* q, const void* k, const void* v, const float* sink, void* o,
                        float* o_precise, float* stat, int B, int H, int T, float q_scale,
                        const KVariant& var, const int32_t* guard, int want_low, hipStream_t s) {
  const int grid = B * H * (T / FBM);
  pick_fwd(var)<<<grid, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v, sink,
                                     (bf16*)o, o_precise, stat, H, T, q_scale, var, guard,
                                     want_low);
  return check_launch("attn_fwd_mfma");
}

int32_t launch_bwd_mfma(const void* q, const void* k, const void* v, const float* stat,
                        const float* di, const void* dout, float* dq_acc, void* dk, void* dv,
                        int B, int H, int T, float q_scale, const KVariant& var,
                        const int32_t* guard, int want_low, hipStream_t s) {
  const int grid = B * H * (T / BBN);
  pick_bwd(var)<<<grid, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v, stat, di,
                                     (const bf16*)dout, dq_acc, (bf16*)dk, (bf16*)dv, T, q_scale,
                                     var, guard, want_low);
  return check_launch("attn_bwd_mfma");
}

}  // namespace algx
