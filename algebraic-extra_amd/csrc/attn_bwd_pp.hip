// gfx950 MFMA attention backward, ping-pong schedule (flash.py:333-361 tile
// VJP, :630-638; head_resident.py:95-132).
//
// Work split as in the one-phase kernel: a workgroup of 8 waves owns 256 keys
// of one (b, h), 32 per wave (K and V rows of the wave in registers as MFMA B
// operands, dK and dV accumulated in registers), and walks 64-query tiles from
// the diagonal to T. Per tile a wave runs
//   SDP  S and dP - di of both 32-query halves (18 MFMAs; queries on the M
//        axis, so each lane holds one key and 16 queries per half),
//   GRAD p = rho(s)^n * st and ds = p * r * (dP - di) in registers (VALU),
//   UPD  dV^T += dO^T P, dK^T += Q_s^T dS (16 MFMAs, dO^T and Q_s^T through
//        transposing LDS reads) and dS^T -> LDS,
//   DQ   a 16-query x 32-d block of the tile's dQ over all 256 keys (16
//        16x16x32 MFMAs from dS^T and a K^T copy in LDS), added to a float32
//        accumulator with no-return atomics.
//
// Schedule. The work runs in 32-query units u (halves of tiles): SDP, GRAD and
// UPD of one half, and half of the keys of DQ. The two waves that share a SIMD
// (w and w + 4) belong to different groups, and the groups run half a unit
// apart: per unit a wave has a VALU phase (GRAD(u)) and an MFMA phase (UPD(u),
// half of DQ of tile u/2 - 1, SDP(u+1)), separated by workgroup barriers, and
// while group 0 is in its VALU phase group 1 is in its MFMA phase and the
// other way round, so each SIMD keeps both its VALU and its matrix core fed
// from two instruction streams.
//
//   unit u   group 0: GRAD(u)                  | UPD(u) DQ SDP(u+1)  |
//            group 1: UPD(u-1) DQ SDP(u)       | GRAD(u)             |
//
// Buffers. A tile's Q_s, dO and row statistics are read from group 0's SDP of
// its first unit to group 1's UPD of its second, six half-units, and dS^T of
// tile t is complete after group 1's UPD of its second unit and read by DQ
// in the next two units; both are double-buffered. Group 0 moves the Q_s
// tiles, group 1 the dO tiles with di and the row statistic, each storing a
// tile in the VALU phase of the one unit where its buffer is free and the
// other group does not read it, and fetching the next one right after.
//
// LDS layout: row-major tiles with padded rows (144 B for Q_s and dO, 136 B for
// dS^T) so that the operand addresses stay affine in the lane index (one base
// register plus immediate offsets) and the three Q_s/dO buffers, two dS^T
// buffers and the K^T copy fit in the 160 KiB of a CU.
#include <type_traits>

#include "attn_mfma.h"

namespace algx {
namespace mfma {
namespace {

constexpr int BKN = 256;   // keys per workgroup
constexpr int BQ = 64;     // queries per tile
constexpr int NWAVE = 8;
constexpr int NTHR = 64 * NWAVE;
constexpr int RSTR = 72;   // LDS row stride (bf16) of the Q_s and dO tiles
constexpr int DSTR = 68;   // LDS row stride (bf16) of dS^T (8-byte stores conflict-free)
constexpr int KTR = BKN + 8;  // LDS row stride of K^T [d][key]
constexpr int NBUF = 2;    // Q_s / dO / statistic buffers

// Value of `x` in lane 16 * (lane / 16) + r (DPP row_newbcast; it folds into
// the VALU operation that consumes it).
__device__ __forceinline__ float row_bcast(float x, int r) {
#define ALGX_BC(R) \
  case R:          \
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + R, 0xF, 0xF, true));
  switch (r) {
    ALGX_BC(0) ALGX_BC(1) ALGX_BC(2) ALGX_BC(3) ALGX_BC(4) ALGX_BC(5) ALGX_BC(6) ALGX_BC(7)
    ALGX_BC(8) ALGX_BC(9) ALGX_BC(10) ALGX_BC(11) ALGX_BC(12) ALGX_BC(13) ALGX_BC(14)
    default: ALGX_BC(15)
  }
#undef ALGX_BC
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// p and ds of one score (flash.py:339-361); dpp = dP - di, ds already
// multiplied by r. For the unshifted kernels `st` is the row factor with
// p = rho^n * st: the statistic itself when it is 1/Z (inv_stat), its n-th
// power otherwise ((rho * Z^(-1/n))^n = rho^n / Z, rho being clamped so rho^n
// is finite).
template <int MODE, bool FAST, bool BOUNDED, int L2N>
__device__ __forceinline__ void tile_grad(float s, float dpp, float st, float clamp, int log2n,
                                          float& p, float& ds) {
  if (MODE == MODE_SOFTMAX) {
    p = __builtin_amdgcn_exp2f((s - st) * kLog2e);
    ds = p * dpp;
    return;
  }
  const float x = (MODE == MODE_NOSHIFT && !BOUNDED) ? __builtin_fminf(s, clamp) : s;
  float r;
  const float rh = FAST ? rho_fast(x, r) : rho_exact(x, r);
  p = MODE == MODE_NOSHIFT ? powN<L2N>(rh, log2n) * st : powN<L2N>(rh * st, log2n);
  ds = (p * r) * dpp;
  if (MODE == MODE_NOSHIFT && !BOUNDED && !(s < clamp)) ds = 0.0f;
}

// Scheduling fence inside the MFMA phase: keeps the compiler from reading
// every operand of the phase ahead of its first MFMA (register pressure).
#ifndef ALGX_PP_FENCES
#define ALGX_PP_FENCES 1
#endif
#if ALGX_PP_FENCES
#define ALGX_PP_FENCE() __builtin_amdgcn_sched_barrier(0)
#else
#define ALGX_PP_FENCE() ((void)0)
#endif

struct PpLds {
  bf16 q[NBUF][BQ * RSTR];   // Q_s tiles, [query][d]
  bf16 g[NBUF][BQ * RSTR];   // dO tiles
  float st[NBUF][BQ];        // row factor of the statistic
  float dd[NBUF][BQ];        // di
  bf16 dst[2][BKN * DSTR];   // dS^T [key][query]
  bf16 kt[HD * KTR];         // K^T of the workgroup [d][key]
  int cnt[6];                // waves per SIMD, then per group (group assignment)
};
static_assert(sizeof(PpLds) <= 160 * 1024, "LDS of one CU");

template <int MODE, bool FAST, bool BOUNDED, int L2N>
__device__ __forceinline__ void pp_body(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const bf16* __restrict__ dout,
    float* __restrict__ dq_acc, bf16* __restrict__ dk, bf16* __restrict__ dv, int T_,
    const KVariant& var, PpLds& L) {
  const int nkb = (T_ + BKN - 1) / BKN;
  const int nheads = gridDim.x / nkb;
  int bh, kb;
  map_block(blockIdx.x, nheads, nkb, false, bh, kb);
  // The wave index goes through readfirstlane so that the compiler treats it,
  // and every branch on it, as wave-uniform: each group's loop then holds only
  // its own registers, and no barrier sits in lane-divergent control flow.
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 4, i16 = lane & 15, j4 = i16 >> 2, m4 = i16 & 3;
  // Group = rank of the wave among the two waves on its SIMD (hardware id
  // register HW_ID bits 5:4), so that the two waves of every SIMD are in
  // different groups whatever the wave-to-SIMD placement; if the placement is
  // not two waves per SIMD, waves 0-3 and 4-7. gt numbers the 256 threads of
  // the group (the loaders' thread index).
  const int simd = (__builtin_amdgcn_s_getreg((1 << 11) | (4 << 6) | 4)) & 3;
  if (tid < 6) L.cnt[tid] = 0;
  __syncthreads();
  int rank = 0;
  if (lane == 0) rank = atomicAdd(&L.cnt[simd], 1);
  rank = __builtin_amdgcn_readfirstlane(__shfl(rank, 0, 64));
  __syncthreads();
  const bool two_per_simd = L.cnt[0] == 2 && L.cnt[1] == 2 && L.cnt[2] == 2 && L.cnt[3] == 2;
  const int grp = two_per_simd ? rank : w >> 2;
  int gidx = 0;
  if (lane == 0) gidx = atomicAdd(&L.cnt[4 + grp], 1);
  gidx = __builtin_amdgcn_readfirstlane(__shfl(gidx, 0, 64));
  const int gt = 64 * gidx + lane;
  const int64_t base = (int64_t)bh * T_ * HD;
  const int64_t rbase = (int64_t)bh * T_;
  const int key0 = kb * BKN, kw = key0 + 32 * w, kcol = kw + c32;
  const bool wave_keys = kw < T_;  // T % 64 == 0: a wave's 32 keys are all valid or none
  const int log2n = var.log2n;
  const bool stat_pow = MODE == MODE_NOSHIFT && !var.inv_stat;
  const float clamp = var.clamp;

  // B operands: lane holds K[kcol][16ks + 8g ..] and V[kcol][16ks + 8g ..].
  bf16x8 kreg[4], vreg[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (wave_keys) {
      kreg[ks] = *reinterpret_cast<const bf16x8*>(k + base + (int64_t)kcol * HD + 16 * ks + 8 * g);
      vreg[ks] = *reinterpret_cast<const bf16x8*>(v + base + (int64_t)kcol * HD + 16 * ks + 8 * g);
    } else {
      kreg[ks] = bf16x8{};
      vreg[ks] = bf16x8{};
    }
  }
  // Ones in the k rows 64, 65 of the extended V^T (dP's -di block).
  const bf16 one = (bf16)1.0f, zero = (bf16)0.0f;
  const bf16x8 ones = g == 0 ? bf16x8{one, one, zero, zero, zero, zero, zero, zero} : bf16x8{};
  const float neg_g0 = g == 0 ? -1.0f : 0.0f;
  // K^T of the workgroup's keys for the dQ product (8 lanes share a key row,
  // so the global reads coalesce).
#pragma unroll
  for (int i = 0; i < BKN * HD / 8 / NTHR; ++i) {
    const int c = tid + NTHR * i, row = c >> 3, col = 8 * (c & 7);
    const bf16x8 val =
        key0 + row < T_ ? *reinterpret_cast<const bf16x8*>(k + base + (int64_t)(key0 + row) * HD + col)
                        : bf16x8{};
#pragma unroll
    for (int e = 0; e < 8; ++e) L.kt[(col + e) * KTR + row] = val[e];
  }

  f32x16 dka[2], dva[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    zero16(dka[dt]);
    zero16(dva[dt]);
  }

  const int qt0 = key0 / BQ, nqt = T_ / BQ;
  const int u0 = 2 * qt0, u_end = 2 * nqt;  // 32-query units (halves of tiles)
  auto qbuf = [&](int t) { return (t - qt0) & 1; };
  auto dbuf = [&](int t) { return (t - qt0) & 1; };
  // The wave has unmasked scores in unit u / unit u crosses its keys.
  auto active = [&](int u) { return wave_keys && u * 32 + 31 >= kw; };
  auto crosses = [&](int u) { return u * 32 < kw + 31; };

  // Loader of this thread's group: group 0 moves Q_s, group 1 dO, di and the
  // row statistic. Thread gt moves rows gt/8 and 32 + gt/8, chunk gt%8.
  const bf16* lsrc = grp ? dout : q;
  const int lrow = gt >> 3, lch = gt & 7;
  bf16x8 pre[2];
  float pst = 0.0f, pdi = 0.0f;
  auto gload = [&](int t) {
    t = t < nqt ? t : nqt - 1;
#pragma unroll
    for (int c = 0; c < 2; ++c)
      pre[c] = *reinterpret_cast<const bf16x8*>(lsrc + base + (int64_t)(t * BQ + lrow + 32 * c) * HD +
                                                8 * lch);
    if (grp) {
      pst = stat[rbase + t * BQ + (gt & 63)];
      pdi = di[rbase + t * BQ + (gt & 63)];
    }
  };
  auto lstore = [&](int t) {
    if (t >= nqt) return;
    bf16* dst = grp ? L.g[qbuf(t)] : L.q[qbuf(t)];
#pragma unroll
    for (int c = 0; c < 2; ++c)
      *reinterpret_cast<bf16x8*>(&dst[(lrow + 32 * c) * RSTR + 8 * lch]) = pre[c];
    if (grp && gt < 64) {
      L.st[qbuf(t)][gt] = stat_pow ? powN<L2N>(pst, log2n) : pst;
      L.dd[qbuf(t)][gt] = pdi;
    }
  };

  // SDP(u): acc[r] <-> query 32u + 8(r/4) + 4g + r%4, key kcol.
  auto sdp = [&](int u, f32x16& s, f32x16& dp) {
    const int t = u >> 1, mq = u & 1;
    const bf16* Q = L.q[qbuf(t)];
    const bf16* Gd = L.g[qbuf(t)];
    zero16(s);
    zero16(dp);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int e = (32 * mq + c32) * RSTR + 16 * ks + 8 * g;
      s = mfma32(*reinterpret_cast<const bf16x8*>(&Q[e]), kreg[ks], s);
      dp = mfma32(*reinterpret_cast<const bf16x8*>(&Gd[e]), vreg[ks], dp);
    }
    // Lanes g = 1 feed zeros; a multiply by a lane mask (not a branch around
    // the load) keeps the block in one basic block.
    const float dd = L.dd[qbuf(t)][32 * mq + c32] * neg_g0;
    const bf16 hi = (bf16)dd;
    const bf16 lo = (bf16)(dd - (float)hi);
    dp = mfma32(bf16x8{hi, lo, zero, zero, zero, zero, zero, zero}, ones, dp);
  };
  // GRAD(u): p, ds -> bf16 k-slot packs pb[kcl], db[kcl]. Lane 16rho + i
  // reads the row factor of query 32u + 8(i/4) + 4(rho/2) + i%4, and a DPP
  // broadcast of lane i hands every lane that of its accumulator row i. Only
  // units that cross the diagonal evaluate the mask.
  const int stq = 8 * (i16 >> 2) + 4 * g + (lane & 3);
  auto grad = [&](auto diag_tag, int u, const f32x16& s, const f32x16& dp, bf16x8 (&pb)[2],
                  bf16x8 (&db)[2]) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    const int t = u >> 1, mq = u & 1;
    const float st_r = L.st[qbuf(t)][32 * mq + stq];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p, ds;
      tile_grad<MODE, FAST, BOUNDED, L2N>(s[r], dp[r], row_bcast(st_r, r), clamp, log2n, p, ds);
      if (DIAG && 32 * u + 8 * (r >> 2) + 4 * g + (r & 3) < kcol) {
        p = 0.0f;
        ds = 0.0f;
      }
      pb[r >> 3][r & 7] = (bf16)p;
      db[r >> 3][r & 7] = (bf16)ds;
    }
  };
  // UPD(u): dS^T of the wave's rows -> LDS, then dV^T += dO^T P and
  // dK^T += Q_s^T dS over the unit's two 16-query chunks (transposing reads:
  // lane 4j+m of group G addresses query row 16(2mq+kcl) + 4(G/2) + j (+8),
  // d 32dt + 16(G%2) + 4m .. +3).
  auto upd = [&](int u, const bf16x8 (&pb)[2], const bf16x8 (&db)[2]) {
    const int t = u >> 1, mq = u & 1;
    // db[kcl][e] is query 32u + 16kcl + 8(e/4) + 4g + e%4.
    bf16* drow = &L.dst[dbuf(t)][(32 * w + c32) * DSTR + 32 * mq + 4 * g];
#pragma unroll
    for (int kcl = 0; kcl < 2; ++kcl) {
      const bf16x8 x = db[kcl];
      *reinterpret_cast<bf16x4*>(drow + 16 * kcl) = bf16x4{x[0], x[1], x[2], x[3]};
      *reinterpret_cast<bf16x4*>(drow + 16 * kcl + 8) = bf16x4{x[4], x[5], x[6], x[7]};
    }
    const bf16* Q = L.q[qbuf(t)];
    const bf16* Gd = L.g[qbuf(t)];
#pragma unroll
    for (int kcl = 0; kcl < 2; ++kcl) {
      const int qr = 16 * (2 * mq + kcl) + 4 * (G >> 1) + j4;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const int e0 = qr * RSTR + 32 * dt + 16 * (G & 1) + 4 * m4, e1 = e0 + 8 * RSTR;
        const bf16x8 ag = join(read_tr(&Gd[e0]), read_tr(&Gd[e1]));
        const bf16x8 aq = join(read_tr(&Q[e0]), read_tr(&Q[e1]));
        dva[dt] = mfma32(ag, pb[kcl], dva[dt]);
        dka[dt] = mfma32(aq, db[kcl], dka[dt]);
      }
    }
  };
  auto zero_rows = [&](int u) {
    bf16* drow = &L.dst[dbuf(u >> 1)][(32 * w + c32) * DSTR + 32 * (u & 1) + 4 * g];
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<bf16x4*>(drow + 8 * j) = bf16x4{};
  };
  // DQ of tile t, keys 128h .. 128h + 127: wave w forms queries 16(w%4).., d
  // 32(w/4).. (16x16x32 MFMAs); the second half adds the block to the
  // float32 accumulator.
  f32x4 qa0, qa1;
  auto dq_half = [&](int t, int h) {
    const bf16* D = L.dst[dbuf(t)];
    const int qr = 16 * (w & 3), dc = 32 * (w >> 2);
    if (h == 0) {
      qa0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      qa1 = qa0;
    }
#pragma unroll
    for (int k2 = 0; k2 < BKN / 64; ++k2) {
      const int kk = 4 * h + k2;
      const int krow = 32 * kk + 8 * G + j4;
      const bf16x8 a = join(read_tr(&D[krow * DSTR + qr + 4 * m4]),
                            read_tr(&D[(krow + 4) * DSTR + qr + 4 * m4]));
      const bf16* kc = &L.kt[(dc + i16) * KTR + 32 * kk + 8 * G];
      qa0 = mfma16(a, *reinterpret_cast<const bf16x8*>(kc), qa0);
      qa1 = mfma16(a, *reinterpret_cast<const bf16x8*>(kc + 16 * KTR), qa1);
    }
    if (h == 1) {
      // qa[i]: dQ[t*64 + qr + 4G + i][dc + 16nb + i16]
      float* out = dq_acc + base + (int64_t)(t * BQ + qr + 4 * G) * HD + dc + i16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        atomicAdd(out + (int64_t)i * HD, qa0[i]);
        atomicAdd(out + (int64_t)i * HD + 16, qa1[i]);
      }
    }
  };

  f32x16 s, dp;
  bf16x8 pb[2], db[2];
  // VALU phase of unit u: this group's tile store and next fetch (group 1
  // stores tile u/2 + 1 in its even units, group 0 tile (u+1)/2 in its odd
  // ones), then GRAD(u).
  auto alpha = [&](int u) {
    if ((u & 1) == (grp ^ 1)) {
      lstore((u + 1) / 2 + grp);
      gload((u + 1) / 2 + grp + 1);
    }
    if (active(u)) {
      if (crosses(u))
        grad(std::true_type{}, u, s, dp, pb, db);
      else
        grad(std::false_type{}, u, s, dp, pb, db);
    }
  };
  // MFMA phase after GRAD(u): UPD(u), half u%2 of DQ of tile u/2 - 1,
  // SDP(u + 1).
  auto beta = [&](int u) {
    if (u >= u0) {
      if (active(u))
        upd(u, pb, db);
      else
        zero_rows(u);
      if ((u >> 1) - 1 >= qt0) dq_half((u >> 1) - 1, u & 1);
    }
    if (u + 1 < u_end && active(u + 1)) sdp(u + 1, s, dp);
  };

  // Prologue: tile qt0 in LDS, tile qt0 + 1 of each group's tensor in
  // registers (stored in the first units: group 1 in unit u0, group 0 in
  // u0 + 1). The explicit drains keep the loop's memory-counter waits from
  // covering prologue loads.
  gload(qt0);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  lstore(qt0);
  gload(qt0 + 1);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();
  // Group 0 forms SDP(u0) ahead of its first GRAD; group 1 forms it in its
  // first MFMA phase, beside group 0's first GRAD. One loop per group (the
  // group is fixed for the whole kernel), so each loop carries only its own
  // live state across the back edge.
  if (grp == 0 && active(u0)) sdp(u0, s, dp);
  __syncthreads();
  if (grp == 0) {
    for (int u = u0; u < u_end; ++u) {
      alpha(u);
      __syncthreads();
      beta(u);
      __syncthreads();
    }
  } else {
    for (int u = u0; u < u_end; ++u) {
      beta(u - 1);
      __syncthreads();
      alpha(u);
      __syncthreads();
    }
    beta(u_end - 1);
  }
  __syncthreads();
  dq_half(nqt - 1, 0);
  dq_half(nqt - 1, 1);

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
__global__ __launch_bounds__(NTHR, 1) void bwd_pp_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ stat, const float* __restrict__ di, const bf16* __restrict__ dout,
    float* __restrict__ dq_acc, bf16* __restrict__ dk, bf16* __restrict__ dv, int T_,
    KVariant lo, KVariant hi, const int32_t* __restrict__ guard) {
  __shared__ __attribute__((aligned(16))) PpLds lds;
  if (LO == HI || guard_in_range(guard))
    pp_body<LO & 3, (LO & 4) != 0, (LO & 8) != 0, (LO >> 4)>(q, k, v, stat, di, dout, dq_acc, dk,
                                                             dv, T_, lo, lds);
  else
    pp_body<HI & 3, (HI & 4) != 0, (HI & 8) != 0, (HI >> 4)>(q, k, v, stat, di, dout, dq_acc, dk,
                                                             dv, T_, hi, lds);
}

typedef void (*PpFn)(const bf16*, const bf16*, const bf16*, const float*, const float*,
                     const bf16*, float*, bf16*, bf16*, int, KVariant, KVariant, const int32_t*);

PpFn pick_pp(int cl, int ch) { ALGX_PICK_ALL(bwd_pp_kernel) }

}  // namespace
}  // namespace mfma

int32_t launch_bwd_pp(const void* q, const void* k, const void* v, const float* stat,
                      const float* di, const void* dout, float* dq_acc, void* dk, void* dv, int B,
                      int H, int T, const KVariant& lo, const KVariant& hi, const int32_t* guard,
                      hipStream_t s) {
  using namespace mfma;
  if (T % BQ != 0 || T < BQ) return fail("attn_bwd: MFMA kernel needs T % 64 == 0");
  const int grid = B * H * ((T + BKN - 1) / BKN);
  PpFn fn = pick_pp(cfg_for(lo), guard != nullptr ? cfg_for(hi) : cfg_for(lo));
  if (fn == nullptr) return fail("attn_bwd: no MFMA kernel for this variant pair");
  launch_k(probe_for(ALGX_PROBE_ATTN_BWD), fn, dim3(grid), dim3(NTHR), s, (const bf16*)q,
           (const bf16*)k, (const bf16*)v, stat, di, (const bf16*)dout, dq_acc, (bf16*)dk,
           (bf16*)dv, T, lo, hi, guard);
  return check_launch("attn_bwd_pp");
}

}  // namespace algx
