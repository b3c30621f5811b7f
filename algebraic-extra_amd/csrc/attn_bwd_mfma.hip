// gfx950 MFMA attention backward (flash.py:333-361 tile VJP, :630-638;
// head_resident.py:95-132).
//
// One workgroup of 8 waves owns 256 keys of one (b, h) (32 per wave; the
// wave's K and V rows stay in registers as MFMA B operands) and walks 64-query
// tiles from the diagonal to T. Per 32-query half of a tile, S and dP are
// formed with queries on the M axis, so each lane holds one key and 16
// queries. dP already carries -di: one extra MFMA k-block multiplies
// [-di_hi, -di_lo] (di split into two bf16 parts) by a ones column of V.
// p and ds are formed in registers and feed dV^T += dO^T P and
// dK^T += Q_s^T dS directly; dO^T and Q_s^T come from the row-major LDS tiles
// through transposing LDS reads (ds_read_b64_tr_b16) in the k-slot order the
// accumulator layout implies, so no transposed copy is ever stored.
//
// dS^T goes to LDS once ([key][query], 8-byte stores), and each wave then
// forms a 16-query x 32-d block of the tile's dQ over all 256 keys with
// v_mfma_f32_16x16x32_bf16 (dS through transposing reads, K from a K^T copy
// in LDS with 16-byte reads) and adds it to a float32 accumulator with
// no-return atomics: one add per element per 256 keys.
//
// Pipelining: Q_s/dO/stat/di tiles and dS^T are double-buffered in LDS, so a
// tile needs one barrier. The dQ of tile t-1 is formed while tile t's
// weights are computed, and tile t+2 is fetched from HBM while tile t runs.
#include <type_traits>

#include "attn_mfma.h"

namespace algx {
namespace mfma {
namespace {

constexpr int BKN = 256;   // keys per workgroup
constexpr int BQ = 64;     // queries per tile
constexpr int NWAVE = 8;
constexpr int NTHR = 64 * NWAVE;
constexpr int RSTR = 72;   // LDS row stride (bf16) of the Q_s and dO tiles: 144 B
constexpr int DSTR = 68;   // LDS row stride (bf16) of the dS^T tiles: 136 B
constexpr int KTR = BKN + 8;  // LDS row stride of K^T [d][key]

// Physical LDS rows. Query row r of a Q_s/dO tile sits at qrow_of(r): the two
// 2-bit fields of r inside its 16-row block swapped, so the four consecutive
// rows a transposing read gathers land 16 banks apart (144-byte pitch) while
// any 16 consecutive rows still cover the banks for 16-byte row reads. Key
// row r of a dS^T tile sits at krow_of(r), a bit permutation inside its
// 32-row block that puts the eight rows of one transposing read pass 8 banks
// apart (136-byte pitch); 32 consecutive rows stay distinct for the 8-byte
// row stores. Both are fixed permutations, so every access is a per-lane base
// plus compile-time offsets.
__host__ __device__ constexpr int qrow_of(int r) {
  return (r & ~15) | ((r & 3) << 2) | ((r >> 2) & 3);
}
__host__ __device__ constexpr int krow_of(int r) {
  return (r & ~31) | ((r >> 3) & 1) << 4 | (r & 3) << 2 | ((r >> 2) & 1) << 1 | ((r >> 4) & 1);
}
// The identities the kernel's addressing uses: both maps are permutations of
// their blocks (qrow_of an involution, used by the tile loader as its own
// inverse), and the rows a transposing read gathers, logical 4a + j (+ 8) and
// 8G + j (+ 4), sit at a per-lane base plus 2.
constexpr bool row_maps_ok() {
  bool seen_q[64] = {}, seen_k[256] = {};
  for (int r = 0; r < 64; ++r) {
    if (qrow_of(qrow_of(r)) != r || qrow_of(r) >> 4 != r >> 4) return false;
    seen_q[qrow_of(r)] = true;
  }
  for (int r = 0; r < 256; ++r) {
    if (krow_of(r) >> 5 != r >> 5) return false;
    seen_k[krow_of(r)] = true;
  }
  for (int r = 0; r < 64; ++r)
    if (!seen_q[r]) return false;
  for (int r = 0; r < 256; ++r)
    if (!seen_k[r]) return false;
  for (int k = 0; k < 4; ++k)
    for (int a = 0; a < 2; ++a)
      for (int j = 0; j < 4; ++j)
        for (int o = 0; o < 2; ++o)
          if (qrow_of(16 * k + 4 * a + j + 8 * o) != 16 * k + 4 * j + a + 2 * o) return false;
  for (int kk = 0; kk < 8; ++kk)
    for (int G = 0; G < 4; ++G)
      for (int j = 0; j < 4; ++j)
        for (int o = 0; o < 2; ++o)
          if (krow_of(32 * kk + 8 * G + j + 4 * o) !=
              32 * kk + 16 * (G & 1) + 4 * j + (G >> 1) + 2 * o)
            return false;
  return true;
}
static_assert(row_maps_ok(), "LDS row permutations");

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// p and ds of one score (flash.py:339-361); dpp = dP - di, ds already
// multiplied by r. For the unshifted kernels `st` is the row factor with
// p = rho^n * st: the statistic itself when it is 1/Z (inv_stat), its n-th
// power otherwise ((rho * Z^(-1/n))^n = rho^n / Z, rho being clamped so rho^n
// is finite).
template <int MODE, bool FAST, bool BOUNDED, int L2N, bool POLY>
__device__ __forceinline__ void tile_grad(float s, float dpp, float st, float clamp, int log2n,
                                          float& p, float& ds) {
  if (MODE == MODE_SOFTMAX) {
    p = __builtin_amdgcn_exp2f((s - st) * kLog2e);
    ds = p * dpp;
    return;
  }
  const float x = (MODE == MODE_NOSHIFT && !BOUNDED) ? __builtin_fminf(s, clamp) : s;
  float r;
  const float rh = POLY ? rho_poly(x, r) : FAST ? rho_fast(x, r) : rho_exact(x, r);
  p = MODE == MODE_NOSHIFT ? powN<L2N>(rh, log2n) * st : powN<L2N>(rh * st, log2n);
  ds = (p * r) * dpp;
  if (MODE == MODE_NOSHIFT && !BOUNDED && !(s < clamp)) ds = 0.0f;
}

struct BwdLds {
  bf16 q[2][BQ * RSTR];     // Q_s tile, row-major [query][d]
  bf16 g[2][BQ * RSTR];     // dO tile
  float st[2][BQ];          // statistic (or its row factor)
  float dd[2][BQ];          // di
  bf16 dst[2][BKN * DSTR];  // dS^T [key][query]
  bf16 kt[HD * KTR];        // K^T of the workgroup [d][key]
};

template <int MODE, bool FAST, bool BOUNDED, int L2N, bool POLY>
__device__ __forceinline__ void bwd_body(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const bf16* __restrict__ dout,
    float* __restrict__ dq_acc, bf16* __restrict__ dk, bf16* __restrict__ dv, int T_,
    const KVariant& var, BwdLds& L) {
  const int nkb = (T_ + BKN - 1) / BKN;
  const int nheads = gridDim.x / nkb;
  int bh, kb;
  map_block(blockIdx.x, nheads, nkb, false, bh, kb);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int G = lane >> 4, i16 = lane & 15, j4 = i16 >> 2, m4 = i16 & 3;
  const int64_t base = (int64_t)bh * T_ * HD;
  const int64_t rbase = (int64_t)bh * T_;
  const int key0 = kb * BKN, kw = key0 + 32 * w, kcol = kw + c32;
  const bool wave_keys = kw < T_;  // T % 64 == 0: a wave's 32 keys are all valid or none
  const int log2n = var.log2n;
  const bool stat_pow = MODE == MODE_NOSHIFT && !var.inv_stat;
  const float clamp = var.clamp;

  // B operands: lane holds K[kcol][16ks + 8g ..] and V[kcol][16ks + 8g ..].
  bf16x8 kreg[4], vreg[4];
  // A wave whose keys lie past T (only in a last, partial key block, which
  // the diagonal loop handles) never forms scores, so it reads the last row.
  {
    const int kc = wave_keys ? kcol : T_ - 1;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kreg[ks] = *reinterpret_cast<const bf16x8*>(k + base + (int64_t)kc * HD + 16 * ks + 8 * g);
      vreg[ks] = *reinterpret_cast<const bf16x8*>(v + base + (int64_t)kc * HD + 16 * ks + 8 * g);
    }
  }
  // Ones in the k rows 64, 65 of the extended V^T (dP's -di block).
  const bf16 one = (bf16)1.0f, zero = (bf16)0.0f;
  const bf16x8 ones = g == 0 ? bf16x8{one, one, zero, zero, zero, zero, zero, zero} : bf16x8{};
  const float neg_g0 = g == 0 ? -1.0f : 0.0f;
  // K^T of the workgroup's keys for the dQ product (8 lanes share a key row,
  // so the global reads coalesce), loaded here and moved to LDS in the
  // prologue below.
  constexpr int KT_CHUNKS = BKN * HD / 8 / NTHR;
  bf16x8 ktv[KT_CHUNKS];
#pragma unroll
  for (int i = 0; i < KT_CHUNKS; ++i) {
    const int c = tid + NTHR * i, row = c >> 3, col = 8 * (c & 7);
    // rows past T read the last row (zeroed when stored): no branch around
    // the load
    const int kr = key0 + row < T_ ? key0 + row : T_ - 1;
    ktv[i] = *reinterpret_cast<const bf16x8*>(k + base + (int64_t)kr * HD + col);
  }

  f32x16 dka[2], dva[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    zero16(dka[dt]);
    zero16(dva[dt]);
  }

  // Tile loader: thread t moves d 8(t%8) .. +7 of the Q_s and dO row stored
  // at physical row prow; the 16 threads of one LDS store pass cover rows 8
  // apart (32 banks apart).
  const int prow = 16 * (tid >> 7) + ((tid >> 4) & 7) + 8 * ((tid >> 3) & 1);
  const int lrow = qrow_of(prow), lcol = 8 * (tid & 7);
  bf16x8 preq, preg;
  float pst = 0.0f, pdi = 0.0f;
  const int qt0 = key0 / BQ, nqt = T_ / BQ;
  // Every wave moves stat and di of query `lane` (the same values), which
  // keeps the loop free of branches.
  auto gload = [&](int qt) {
    const int64_t off = base + (int64_t)(qt * BQ + lrow) * HD + lcol;
    preq = *reinterpret_cast<const bf16x8*>(q + off);
    preg = *reinterpret_cast<const bf16x8*>(dout + off);
    pst = stat[rbase + qt * BQ + lane];
    pdi = di[rbase + qt * BQ + lane];
  };
  auto lstore = [&](int buf) {
    *reinterpret_cast<bf16x8*>(&L.q[buf][prow * RSTR + lcol]) = preq;
    *reinterpret_cast<bf16x8*>(&L.g[buf][prow * RSTR + lcol]) = preg;
    L.st[buf][lane] = stat_pow ? powN<L2N>(pst, log2n) : pst;
    L.dd[buf][lane] = pdi;
  };

  // S and dP - di of query half mq: acc[r] <-> query 32mq + 8(r/4) + 4g + r%4, key kcol.
  auto half_scores = [&](int buf, int mq, f32x16& s, f32x16& dp) {
    zero16(s);
    zero16(dp);
    const bf16* qrow = &L.q[buf][(32 * mq + qrow_of(c32)) * RSTR + 8 * g];
    const bf16* grow = &L.g[buf][(32 * mq + qrow_of(c32)) * RSTR + 8 * g];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      s = mfma32(*reinterpret_cast<const bf16x8*>(qrow + 16 * ks), kreg[ks], s);
      dp = mfma32(*reinterpret_cast<const bf16x8*>(grow + 16 * ks), vreg[ks], dp);
    }
    // Lanes g = 1 feed zeros; a multiply by a lane mask (not a branch around
    // the load) keeps the tile in one basic block.
    const float dd = L.dd[buf][32 * mq + c32] * neg_g0;
    const bf16 hi = (bf16)dd;
    const bf16 lo = (bf16)(dd - (float)hi);
    dp = mfma32(bf16x8{hi, lo, zero, zero, zero, zero, zero, zero}, ones, dp);
  };
  // p, ds of half mq -> bf16 k-slot packs (two 16-query chunks each). Only
  // tiles that cross the diagonal (diag_tag = true_type) evaluate the mask.
  auto half_grads = [&](auto diag_tag, int buf, int q0, int mq, const f32x16& s,
                        const f32x16& dp, bf16x8 (&pb)[2], bf16x8 (&db)[2]) {
    constexpr bool DIAG = decltype(diag_tag)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int qo = 32 * mq + 8 * j + 4 * g;
      const f32x4 st4 = *reinterpret_cast<const f32x4*>(&L.st[buf][qo]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * j + i;
        float p, ds;
        tile_grad<MODE, FAST, BOUNDED, L2N, POLY>(s[r], dp[r], st4[i], clamp, log2n, p, ds);
        if (DIAG && q0 + qo + i < kcol) {
          p = 0.0f;
          ds = 0.0f;
        }
        pb[r >> 3][r & 7] = (bf16)p;
        db[r >> 3][r & 7] = (bf16)ds;
      }
    }
  };
  // dV^T += dO^T P and dK^T += Q_s^T dS over the half's two 16-query chunks
  // (A operands through transposing reads); dS^T of the half -> LDS.
  auto half_update = [&](int buf, int mq, const bf16x8 (&pb)[2], const bf16x8 (&db)[2]) {
#pragma unroll
    for (int kcl = 0; kcl < 2; ++kcl) {
      // Physical rows of queries 16(2mq + kcl) + 4(G >> 1) + j4 (+ 8).
      const int qbase = 16 * (2 * mq + kcl) + 4 * j4 + (G >> 1);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const int col = 32 * dt + 16 * (G & 1) + 4 * m4;
        const bf16x8 ag = join(read_tr(&L.g[buf][qbase * RSTR + col]),
                               read_tr(&L.g[buf][(qbase + 2) * RSTR + col]));
        const bf16x8 aq = join(read_tr(&L.q[buf][qbase * RSTR + col]),
                               read_tr(&L.q[buf][(qbase + 2) * RSTR + col]));
        dva[dt] = mfma32(ag, pb[kcl], dva[dt]);
        dka[dt] = mfma32(aq, db[kcl], dka[dt]);
      }
    }
    bf16* drow = &L.dst[buf][(32 * w + krow_of(c32)) * DSTR + 32 * mq + 4 * g];
#pragma unroll
    for (int kcl = 0; kcl < 2; ++kcl) {
      *reinterpret_cast<bf16x4*>(drow + 16 * kcl) =
          bf16x4{db[kcl][0], db[kcl][1], db[kcl][2], db[kcl][3]};
      *reinterpret_cast<bf16x4*>(drow + 16 * kcl + 8) =
          bf16x4{db[kcl][4], db[kcl][5], db[kcl][6], db[kcl][7]};
    }
  };
  auto zero_dst = [&](int buf) {
    bf16* drow = &L.dst[buf][(32 * w + krow_of(c32)) * DSTR + 4 * g];
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<bf16x4*>(drow + 8 * j) = bf16x4{};
  };
  // dQ of tile qt from dS^T[buf]: wave w forms queries 16(w%4).., d 32(w/4)..
  // over the 256 keys (16x16x32 MFMAs), then adds it to the accumulator.
  auto dq_tile = [&](int qt, int buf) {
    const int qr = 16 * (w & 3), dc = 32 * (w >> 2);
    f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
#pragma unroll
    for (int kk = 0; kk < BKN / 32; ++kk) {
      // Physical rows of keys 32kk + 8G + j4 (+ 4).
      const int krow = 32 * kk + 16 * (G & 1) + 4 * j4 + (G >> 1);
      const bf16x8 a = join(read_tr(&L.dst[buf][krow * DSTR + qr + 4 * m4]),
                            read_tr(&L.dst[buf][(krow + 2) * DSTR + qr + 4 * m4]));
      const bf16* kcol = &L.kt[(dc + i16) * KTR + 32 * kk + 8 * G];
      const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(kcol);
      const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(kcol + 16 * KTR);
      acc0 = mfma16(a, b0, acc0);
      acc1 = mfma16(a, b1, acc1);
    }
    // acc[i]: dQ[qt*64 + qr + 4G + i][dc + 16nb + i16]
    float* dst = dq_acc + base + (int64_t)(qt * BQ + qr + 4 * G) * HD + dc + i16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      atomicAdd(dst + (int64_t)i * HD, acc0[i]);
      atomicAdd(dst + (int64_t)i * HD + 16, acc1[i]);
    }
  };

  // Prologue: every setup load (the wave's K and V rows, the K^T block and
  // tiles qt0 and qt0+1) is in flight at once, so the setup costs one memory
  // round trip rather than one per step. K^T and tile qt0 go to LDS; tile
  // qt0+1 stays in registers until the first iteration stores it.
  gload(qt0);
#pragma unroll
  for (int i = 0; i < KT_CHUNKS; ++i) {
    const int c = tid + NTHR * i, row = c >> 3, col = 8 * (c & 7);
    const bf16x8 val = key0 + row < T_ ? ktv[i] : bf16x8{};
#pragma unroll
    for (int e = 0; e < 8; ++e) L.kt[(col + e) * KTR + row] = val[e];
  }
  lstore(0);
  gload(qt0 + 1 < nqt ? qt0 + 1 : qt0);
  __syncthreads();

  // Each iteration ends with the LDS store of the next tile (whose wait
  // covers the fetch issued one iteration earlier, nothing later), the dQ
  // step of the previous tile (none before the first) and the fetch of the
  // tile after next. Tile indices past the end are clamped: that extra work
  // lands in buffers no later step reads, or adds zeros.
  const int qdiag = qt0 + BKN / BQ < nqt ? qt0 + BKN / BQ : nqt;
  int qt = qt0;
  for (; qt < qdiag; ++qt) {
    const int buf = (qt - qt0) & 1;
    const int q0 = qt * BQ;
    if (wave_keys && q0 + BQ - 1 >= kw) {
      const bool diag = q0 < kw + 31;
#pragma unroll
      for (int mq = 0; mq < 2; ++mq) {
        f32x16 s, dp;
        bf16x8 pb[2], db[2];
        half_scores(buf, mq, s, dp);
        if (diag)
          half_grads(std::true_type{}, buf, q0, mq, s, dp, pb, db);
        else
          half_grads(std::false_type{}, buf, q0, mq, s, dp, pb, db);
        half_update(buf, mq, pb, db);
      }
    } else {
      zero_dst(buf);
    }
    lstore(buf ^ 1);
    if (qt > qt0) dq_tile(qt - 1, buf ^ 1);
    gload(qt + 2 < nqt ? qt + 2 : nqt - 1);
    __syncthreads();
  }
  // Tiles below the diagonal: no masks and no per-wave branches, so the
  // MFMAs of one half interleave with the weight math of the other in a
  // single basic block.
  for (; qt < nqt; ++qt) {
    const int buf = (qt - qt0) & 1;
    const int q0 = qt * BQ;
    f32x16 s0, dp0, s1, dp1;
    bf16x8 pb0[2], db0[2], pb1[2], db1[2];
    // Waves w and w + 4 share a SIMD and the tile's barrier; the upper four
    // form the previous tile's dQ first, so the pair's MFMA and VALU phases
    // are offset rather than coincident.
    const bool dq_first = w >= 4;
    if (dq_first) dq_tile(qt - 1, buf ^ 1);
    half_scores(buf, 0, s0, dp0);
    half_grads(std::false_type{}, buf, q0, 0, s0, dp0, pb0, db0);
    half_scores(buf, 1, s1, dp1);
    half_update(buf, 0, pb0, db0);
    half_grads(std::false_type{}, buf, q0, 1, s1, dp1, pb1, db1);
    half_update(buf, 1, pb1, db1);
    if (!dq_first) dq_tile(qt - 1, buf ^ 1);
    lstore(buf ^ 1);
    gload(qt + 2 < nqt ? qt + 2 : nqt - 1);
    __syncthreads();
  }
  dq_tile(nqt - 1, (nqt - 1 - qt0) & 1);

  if (!wave_keys) return;
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
__global__ __launch_bounds__(NTHR, 1) void bwd_mfma_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const bf16* __restrict__ dout,
    float* __restrict__ dq_acc, bf16* __restrict__ dk, bf16* __restrict__ dv, int T_,
    KVariant lo, KVariant hi, const int32_t* __restrict__ guard) {
  __shared__ __attribute__((aligned(16))) BwdLds lds;
  if (LO == HI || guard_in_range(guard))
    bwd_body<cfg_mode(LO), cfg_fast(LO), cfg_bounded(LO), cfg_l2n(LO), cfg_poly(LO)>(
        q, k, v, stat, di, dout, dq_acc, dk, dv, T_, lo, lds);
  else
    bwd_body<cfg_mode(HI), cfg_fast(HI), cfg_bounded(HI), cfg_l2n(HI), cfg_poly(HI)>(
        q, k, v, stat, di, dout, dq_acc, dk, dv, T_, hi, lds);
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
  if (T % BQ != 0 || T < BQ) return fail("attn_bwd: MFMA kernel needs T % 64 == 0");
  const int grid = B * H * ((T + BKN - 1) / BKN);
  BwdFn fn = pick_bwd(cfg_for(lo), guard != nullptr ? cfg_for(hi) : cfg_for(lo));
  if (fn == nullptr) return fail("attn_bwd: no MFMA kernel for this variant pair");
  launch_k(probe_for(ALGX_PROBE_ATTN_BWD), fn, dim3(grid), dim3(NTHR), s, (const bf16*)q,
           (const bf16*)k, (const bf16*)v, stat, di, (const bf16*)dout, dq_acc, (bf16*)dk,
           (bf16*)dv, T, lo, hi, guard);
  return check_launch("attn_bwd_mfma");
}

}  // namespace algx
