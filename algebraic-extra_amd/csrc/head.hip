// Fused tied-embedding projection + likelihood loss (fused_head.py) on gfx950.
//
// Forward (fused_head.py:72-117, :174-191): logits z^T = E h^T are formed
// tile by tile (256 vocab x 256 tokens, d streamed through LDS in 32-wide
// stages, v_mfma_f32_32x32x16_bf16) and never stored. Vocabulary rows sit on
// the MFMA M axis so every lane holds 16 vocabulary values of one token; the
// per-token statistic (online max/sum-exp for "ce", sum of rho(min(z/c,X))^n
// for "alg_ce") is kept per lane, merged across lanes at the end of a
// workgroup's vocabulary chunk, and merged across chunks by a small kernel.
// The target logit is written by the one lane that meets it.
//
// Backward (fused_head.py:120-156, :194-216): the same tiles are recomputed
// and the scaled bf16 logit gradient dz (fused_head.py:145) is written for a
// chunk of tokens; dh = dz E and dE += dz^T h are then plain MFMA GEMMs over
// that chunk (the reference also materialises dz and runs an XLA GEMM for dE).
#include <cstdlib>
#include <type_traits>

#include "head_f32.h"

namespace algx {

namespace {

constexpr int BM = 256, BN = 256, BK = 32;  // output tile and k stage of every GEMM
constexpr int LSTR = BK + 8;   // LDS row stride (bf16) of k-contiguous tiles: 80 B
constexpr int TSTR = BM + 16;  // LDS row stride (bf16) of [k][mn] tiles: 544 B
constexpr int NWM = 2, NWN = 4;               // waves along m and n
constexpr int kThreads = 64 * NWM * NWN;
constexpr int WTM = BM / NWM, WTN = BN / NWN;  // outputs per wave: 128 x 64
constexpr int TI = WTM / 32, TJ = WTN / 32;    // 32x32 MFMA tiles per wave along m and n
constexpr int kStageElems = BM * LSTR > BK * TSTR ? BM * LSTR : BK * TSTR;
constexpr int kChunks = BM * BK / 8 / kThreads;  // 16-byte chunks per thread per tile stage
static_assert(BM == BN && (BM / 8) * (kThreads / (BM / 8)) == kThreads &&
                  kChunks * (kThreads / (BM / 8)) == BK,
              "[k][mn] loader: BM/8 threads per k row group, kChunks k rows each");
constexpr int kFwdWorkgroups = 256;  // forward grid target: one workgroup per CU

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Operand of a GEMM C[m][n] = sum_k A(m,k) B(n,k). KC: stored as [MN][K]
// (k contiguous, leading dimension ld); otherwise stored as [K][MN].
struct Operand {
  const bf16* p;
  int64_t ld;
  int rows;  // extent along m (or n)
  int K;
};

// Stages one 256 x 64 (mn x k) tile of an operand into registers (zero
// outside): four 16-byte loads per thread.
// Per-thread addressing of one operand tile (set once per output tile): the
// thread's chunks of a 256 x BK (mn x k) stage.
template <bool KC>
struct TileAddr {
  const bf16* base[kChunks];  // chunk address at k stage 0 (op.p when its mn is outside)
  int koff[kChunks];          // k of the chunk within a stage
  bool mn_in[kChunks];
  __device__ __forceinline__ void init(const Operand& op, int mn0, int tid) {
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (KC) {
        // [mn][k]: BK / 8 chunks per row.
        const int id = tid + kThreads * c;
        const int row = mn0 + id / (BK / 8);
        koff[c] = (id % (BK / 8)) * 8;
        mn_in[c] = row < op.rows;
        base[c] = op.p + (mn_in[c] ? (int64_t)row * op.ld + koff[c] : 0);
      } else {
        // [k][mn]: kChunks consecutive k rows x 8 consecutive mn per thread.
        const int kg = tid / (BM / 8), mg = tid % (BM / 8);
        const int mm = mn0 + 8 * mg;
        koff[c] = kChunks * kg + c;
        mn_in[c] = mm < op.rows;
        base[c] = op.p + (mn_in[c] ? (int64_t)koff[c] * op.ld + mm : 0);
      }
    }
  }
};

template <bool KC>
struct TileLoader {
  bf16x8 r[kChunks];
  uint32_t ok;  // bit c: chunk c is inside the operand
  // Branch-free: an out-of-range chunk reads the operand's first 16 bytes and
  // is replaced by zeros when stored, so no wait for the load sits here.
  __device__ __forceinline__ void load(const Operand& op, const TileAddr<KC>& ad, int k0) {
    ok = 0;
    const int64_t step = KC ? (int64_t)k0 : (int64_t)k0 * op.ld;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const bool in = ad.mn_in[c] && k0 + ad.koff[c] < op.K;
      ok |= in ? 1u << c : 0u;
      r[c] = *reinterpret_cast<const bf16x8*>(in ? ad.base[c] + step : op.p);
    }
  }
  __device__ __forceinline__ void store(bf16* lds, int tid) const {
    if (KC) {
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        const int id = tid + kThreads * c;
        *reinterpret_cast<bf16x8*>(lds + (id / (BK / 8)) * LSTR + (id % (BK / 8)) * 8) =
            (ok >> c) & 1 ? r[c] : bf16x8{};
      }
    } else {
      // Kept as stored in memory, [k][mn]; the MFMA operand is read through
      // transposing LDS reads.
      const int kg = tid / (BM / 8), mg = tid % (BM / 8);
#pragma unroll
      for (int i = 0; i < kChunks; ++i)
        *reinterpret_cast<bf16x8*>(lds + (kChunks * kg + i) * TSTR + 8 * mg) =
            (ok >> i) & 1 ? r[i] : bf16x8{};
    }
  }
};

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// MFMA operand (rows mn0 + (lane % 32), k-slots k0 + 8(lane / 32) .. +7) of a
// tile in LDS: one 16-byte read from a [mn][k] tile, or two transposing reads
// (ds_read_b64_tr_b16) from a [k][mn] tile, in which lane 4j+m of each
// 16-lane group addresses row j, columns 4m .. 4m+3.
template <bool KC>
__device__ __forceinline__ bf16x8 operand(const bf16* tile, int mn0, int k0, int lane) {
  if (KC) {
    return *reinterpret_cast<const bf16x8*>(tile + (mn0 + (lane & 31)) * LSTR + k0 + 8 * (lane >> 5));
  } else {
    const int G = lane >> 4, j = (lane >> 2) & 3, m = lane & 3;
    const bf16* p = tile + (k0 + 8 * (G >> 1) + j) * TSTR + mn0 + 16 * (G & 1) + 4 * m;
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p + 4 * TSTR));
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
}

// Wave w = (wm, wn) = (w / NWN, w % NWN) owns outputs m0 + WTM wm .. + WTM - 1,
// n0 + WTN wn .. + WTN - 1:
// acc.v[i][j][r] = C[m0 + WTM wm + 32i + 8(r/4) + 4g + r%4][n0 + WTN wn + 32j + c32].
struct Acc {
  f32x16 v[TI][TJ];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) v[i][j][r] = 0.0f;
  }
};

template <bool AKC, bool BKC>
__device__ __forceinline__ void mma_stage(const bf16* As, const bf16* Bs, Acc& acc, int wm,
                                          int wn, int lane) {
#pragma unroll
  for (int ks = 0; ks < BK / 16; ++ks) {
    bf16x8 a[TI], b[TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i) a[i] = operand<AKC>(As, WTM * wm + 32 * i, 16 * ks, lane);
#pragma unroll
    for (int j = 0; j < TJ; ++j) b[j] = operand<BKC>(Bs, WTN * wn + 32 * j, 16 * ks, lane);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc.v[i][j] = mfma32(a[i], b[j], acc.v[i][j]);
  }
}

// Full-K product of one output tile: LDS double-buffered, global loads two
// k stages ahead (two register sets, so a stage's HBM latency spans two
// stages of MFMA work).
template <bool AKC, bool BKC>
__device__ __forceinline__ void gemm_tile(const Operand& A, const Operand& B, int m0, int n0,
                                          bf16* As, bf16* Bs, Acc& acc, int tid) {
  const int w = tid >> 6, lane = tid & 63;
  const int wm = w / NWN, wn = w % NWN;
  const int K = A.K;
  const int nk = (K + BK - 1) / BK;
  TileAddr<AKC> aa;
  TileAddr<BKC> ab;
  aa.init(A, m0, tid);
  ab.init(B, n0, tid);
  TileLoader<AKC> la0, la1;
  TileLoader<BKC> lb0, lb1;
  acc.zero();
  // Every step issues the same loads (stage indices past the end are clamped
  // to the last stage and never stored), so each wait before a store covers
  // exactly the loads of the stage it stores.
  const int klast = (nk - 1) * BK;
  la0.load(A, aa, 0);
  lb0.load(B, ab, 0);
  la1.load(A, aa, min(BK, klast));
  lb1.load(B, ab, min(BK, klast));
  __syncthreads();  // previous users of the LDS buffers are done
  la0.store(As, tid);
  lb0.store(Bs, tid);
  __syncthreads();
  // Stage kk sits in LDS buffer kk % 2; register set kk % 2 held it and is
  // refilled with stage kk + 2 while stage kk + 1 waits in the other set.
  auto step = [&](int kk, TileLoader<AKC>& la_cur, TileLoader<BKC>& lb_cur,
                  TileLoader<AKC>& la_nxt, TileLoader<BKC>& lb_nxt) {
    const int buf = kk & 1;
    la_cur.load(A, aa, min((kk + 2) * BK, klast));
    lb_cur.load(B, ab, min((kk + 2) * BK, klast));
    mma_stage<AKC, BKC>(As + buf * kStageElems, Bs + buf * kStageElems, acc, wm, wn, lane);
    if (kk + 1 < nk) {
      la_nxt.store(As + (buf ^ 1) * kStageElems, tid);
      lb_nxt.store(Bs + (buf ^ 1) * kStageElems, tid);
    }
    __syncthreads();
  };
  for (int kk = 0; kk < nk; kk += 2) {
    step(kk, la0, lb0, la1, lb1);
    if (kk + 1 < nk) step(kk + 1, la1, lb1, la0, lb0);
  }
}

// ------------------------------------------------ direct-to-LDS GEMM core
// The same product with the stages moved from memory straight into LDS by
// LDS-DMA loads (global_load_lds_dwordx4: lane i of a wave's load writes its
// 16 bytes at the destination + 16 i), so no registers stage them and no LDS
// stores are issued; a ring of four stages keeps the loads two stages ahead
// of the operand reads, with one barrier per stage. Stages are unpadded, with their
// 16-byte chunks XOR-permuted so that the operand reads meet every LDS bank
// once per pass: [mn][k] tiles (64-byte rows) keep chunk c of row r at
// c ^ ((r >> 2) & 3), [k][mn] tiles (512-byte rows) at c ^ 4 (r & 3). Needs
// K % BK == 0 (no partial stage); rows (or columns) past the operand's extent
// load the operand's first bytes, which only reach outputs that are never
// stored.
constexpr int kDmaStages = 4;
constexpr int kDmaOpElems = BM * BK;            // one operand stage: 8192 bf16

// Source of this lane's 16 bytes in 1 KB block `blk` of a stage at k = 0.
template <bool KC>
__device__ __forceinline__ const bf16* dma_src(const Operand& op, int mn0, int blk, int lane) {
  if (KC) {
    const int r = 16 * blk + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
    const int row = mn0 + r;
    return row < op.rows ? op.p + (int64_t)row * op.ld + 8 * c : op.p;
  } else {
    const int r = 2 * blk + (lane >> 5), c = (lane & 31) ^ (4 * (r & 3));
    const int col = mn0 + 8 * c;
    return col < op.rows ? op.p + (int64_t)r * op.ld + col : op.p;
  }
}

// MFMA operand (as `operand`) from a swizzled DMA stage.
template <bool KC>
__device__ __forceinline__ bf16x8 operand_dma(const bf16* tile, int mn0, int k0, int lane) {
  if (KC) {
    const int r = mn0 + (lane & 31), c = (k0 >> 3) + (lane >> 5);
    return *reinterpret_cast<const bf16x8*>(tile + r * BK + 8 * (c ^ ((r >> 2) & 3)));
  } else {
    const int G = lane >> 4, j = (lane >> 2) & 3, m = lane & 3;
    const int r = k0 + 8 * (G >> 1) + j;
    const int col = mn0 + 16 * (G & 1) + 4 * m;
    const bf16* p = tile + r * BM + 8 * ((col >> 3) ^ (4 * (r & 3))) + (col & 7);
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p + 4 * BM));
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
}

// One LDS-DMA load of a wave: lane i's 16 bytes at src go to dst + 16 i (dst
// wave-uniform). Issued as inline assembly so that the compiler does not
// track it: its waitcnt pass cannot tell which LDS buffer such a load writes
// and would wait for all of them before every LDS read; the ring below waits
// for its own loads explicitly (wait_vm) before the barrier that publishes
// them.
__device__ __forceinline__ void dma16(const bf16* src, unsigned lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src)
               : "memory", "m0");
}

// s_waitcnt immediates: vmcnt(n) with expcnt and lgkmcnt unconstrained.
template <int N> __device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// Ring of stage buffers (32 KB each: the A stage, then the B stage).
struct DmaRing {
  bf16* slot[kDmaStages];
};

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Products of `ntiles` output tiles that share the B rows n0: tile t uses A
// rows m0 + t BM; epi(t, m0 + t BM, acc) receives each finished tile. The
// ring streams across the tiles, so a tile's first stages load during the
// previous tile's last stages and epilogue. Several tiles need the tile's
// stage count to be a multiple of the ring's (every tile starts at slot 0).
template <bool AKC, bool BKC, typename Epi>
__device__ __forceinline__ void gemm_seq_dma(const Operand& A, const Operand& B, int m0,
                                             int ntiles, int n0, const DmaRing& ring, Acc& acc,
                                             int tid, Epi&& epi) {
  constexpr int S = kDmaStages, L = S - 2;  // stages in flight beyond the one being read
  const int w = tid >> 6, lane = tid & 63;
  const int wm = w / NWN, wn = w % NWN;
  const int nk = A.K / BK;
  const int G = ntiles * nk;  // stages of the whole sequence
  const bf16* sa0 = dma_src<AKC>(A, m0, 2 * w, lane);  // A sources of the tile being issued
  const bf16* sa1 = dma_src<AKC>(A, m0, 2 * w + 1, lane);
  const bf16* sb0 = dma_src<BKC>(B, n0, 2 * w, lane);
  const bf16* sb1 = dma_src<BKC>(B, n0, 2 * w + 1, lane);
  const int64_t stepA = AKC ? BK : (int64_t)BK * A.ld;
  const int64_t stepB = BKC ? BK : (int64_t)BK * B.ld;
  // Byte offset of the wave's two 1 KB blocks in an operand stage (uniform).
  const unsigned wofs = 2048u * __builtin_amdgcn_readfirstlane(w);
  // The wave's two 1 KB blocks of each operand of stage kk (A sources a0/a1)
  // -> slot.
  auto issue = [&](const bf16* a0, const bf16* a1, int kk, bf16* slot) {
    const unsigned dA = lds_addr(slot) + wofs, dB = dA + 2 * kDmaOpElems;
    // Stage offsets as scalars computed here (the compiler would otherwise
    // keep one vector induction variable per unrolled stage).
    int64_t oa = kk * stepA, ob = kk * stepB;
    asm volatile("" : "+s"(oa), "+s"(ob));
    dma16(a0 + oa, dA);
    dma16(a1 + oa, dA + 1024);
    dma16(sb0 + ob, dB);
    dma16(sb1 + ob, dB + 1024);
  };
  // Wait until at most `later` of this wave's stages are still loading (four
  // loads a stage; the loads complete in issue order, and any later vector
  // memory operation only makes the wait stricter).
  auto wait_stages = [](int later) {
    static_assert(L <= 4, "the vmcnt immediates below cover up to three later stages");
    if (later <= 0)
      wait_vm<0>();
    else if (later == 1)
      wait_vm<4>();
    else if (later == 2)
      wait_vm<8>();
    else
      wait_vm<12>();
  };
  // Operands of one 16-wide k step (ks) of a stage into registers.
  auto rd = [&](const bf16* As, int ks, bf16x8 (&a)[TI], bf16x8 (&b)[TJ]) {
    const bf16* Bs = As + kDmaOpElems;
#pragma unroll
    for (int j = 0; j < TJ; ++j) b[j] = operand_dma<BKC>(Bs, WTN * wn + 32 * j, 16 * ks, lane);
#pragma unroll
    for (int i = 0; i < TI; ++i) a[i] = operand_dma<AKC>(As, WTM * wm + 32 * i, 16 * ks, lane);
  };
  auto mm = [&](const bf16x8 (&a)[TI], const bf16x8 (&b)[TJ]) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc.v[i][j] = mfma32(a[i], b[j], acc.v[i][j]);
  };
  acc.zero();
  wait_vm<0>();     // nothing older is counted with the ring's loads
  __syncthreads();  // previous users of the ring are done
  // Stages 0 .. S-2 now (all of the first tile when there are several), then
  // stage g + S - 1 at the barrier of stage g (into the slot of stage g - 1),
  // so every stage is issued two stages before its operands are read.
#pragma unroll
  for (int u = 0; u < S - 1; ++u)
    if (u < nk) issue(sa0, sa1, u, ring.slot[u]);
  wait_stages(min(S - 2, G - 1));
  __syncthreads();
  // Register double buffer over half stages: the operands of the next half
  // stage are read while the MFMAs of the current one run. The barrier sits
  // between a stage's halves: it publishes stage g + 1 (whose first half is
  // read next). It does not wait for this wave's LDS reads: those in flight
  // read the slot of stage g, which no load refills before the next barrier.
  // On the last stage the reads of "stage G" fetch a stale slot and are unused.
  bf16x8 xa[TI], xb[TJ], ya[TI], yb[TJ];
  rd(ring.slot[0], 0, xa, xb);
  for (int t = 0; t < ntiles; ++t) {
    // A sources of the next tile, for the stages issued near this tile's end.
    const bf16* na0 = sa0;
    const bf16* na1 = sa1;
    if (t + 1 < ntiles) {
      na0 = dma_src<AKC>(A, m0 + (t + 1) * BM, 2 * w, lane);
      na1 = dma_src<AKC>(A, m0 + (t + 1) * BM, 2 * w + 1, lane);
    }
    const int g0 = t * nk;
    auto step = [&](int kk, const bf16* cur, const bf16* nxt, bf16* refill) {
      rd(cur, 1, ya, yb);
      __builtin_amdgcn_sched_barrier(0);
      mm(xa, xb);
      __builtin_amdgcn_sched_barrier(0);
      // Wait for stage g + 1; the stages issued after it may stay in flight.
      const int g = g0 + kk;
      wait_stages(min(g + S - 2, G - 1) - (g + 1));
      asm volatile("s_barrier" ::: "memory");
      if (kk + S - 1 < nk)
        issue(sa0, sa1, kk + S - 1, refill);
      else if (t + 1 < ntiles)
        issue(na0, na1, kk + S - 1 - nk, refill);
      rd(nxt, 0, xa, xb);
      __builtin_amdgcn_sched_barrier(0);
      mm(ya, yb);
    };
    // Slots are named statically: S stages a turn.
    for (int kk = 0; kk < nk; kk += S) {
#pragma unroll
      for (int u = 0; u < S; ++u)
        if (kk + u < nk)
          step(kk + u, ring.slot[u], ring.slot[(u + 1) % S], ring.slot[(u + S - 1) % S]);
    }
    epi(t, m0 + t * BM, acc);
    acc.zero();
    sa0 = na0;
    sa1 = na1;
  }
}

// Full-K product of one output tile on the direct-to-LDS ring.
template <bool AKC, bool BKC>
__device__ __forceinline__ void gemm_tile_dma(const Operand& A, const Operand& B, int m0, int n0,
                                              const DmaRing& ring, Acc& acc, int tid) {
  Acc out;
  gemm_seq_dma<AKC, BKC>(A, B, m0, 1, n0, ring, out, tid,
                         [&](int, int, Acc& a) { acc = a; });
}

// LDS of a kernel built on the GEMM cores (DMA: a compile-time bool in
// scope): four 32 KB stage buffers of the direct-to-LDS ring, or the two
// double-buffered operand stages of gemm_tile in the first of them.
#define GEMM_LDS_STAGES                                                                  \
  __shared__ __attribute__((aligned(16))) bf16 s0[DMA ? 2 * kDmaOpElems : 4 * kStageElems]; \
  __shared__ __attribute__((aligned(16))) bf16 s1[DMA ? 2 * kDmaOpElems : 8];               \
  __shared__ __attribute__((aligned(16))) bf16 s2[DMA ? 2 * kDmaOpElems : 8];               \
  __shared__ __attribute__((aligned(16))) bf16 s3[DMA ? 2 * kDmaOpElems : 8];               \
  const DmaRing ring{{s0, s1, s2, s3}}

// x^n, n = 2^log2n: unrolled squarings for a compile-time L2N > 0 (a runtime
// loop inside the per-logit epilogue would cost a branch per logit).
template <int L2N> __device__ __forceinline__ float pow_n(float x, int log2n) {
  if (L2N > 0) {
#pragma unroll
    for (int i = 0; i < L2N; ++i) x = x * x;
    return x;
  }
  return pow2n(x, log2n);
}

// alg_ce weight w = (x + sqrt(1+x^2))^n with x = min(z/c, clamp) (fused_head.py:98-100).
template <int L2N>
__device__ __forceinline__ float alg_weight(float z, float inv_c, float clamp, int log2n,
                                            float& r) {
  const float x = __builtin_fminf(z * inv_c, clamp);
  return pow_n<L2N>(rho_fast(x, r), log2n);
}

// Forward statistics. grid = (token blocks) x (vocabulary chunks of
// chunk_tiles tiles).
// partial[(chunk * N + token) * 2 + {0,1}] = (m, l) for ce, (-, l) for alg_ce.
// DMA: the direct-to-LDS ring streamed over the chunk's tiles (d a multiple
// of BK * kDmaStages).
template <int KIND, int L2N, bool DMA>
__global__ __launch_bounds__(kThreads) void head_fwd_kernel(
    const bf16* __restrict__ h, const bf16* __restrict__ e, const int32_t* __restrict__ targets,
    float* __restrict__ zt, float* __restrict__ partial, int N, int d, int V, int log2n,
    float inv_c, float clamp, int chunk_tiles) {
  GEMM_LDS_STAGES;
  __shared__ float red_m[2][BN], red_l[2][BN];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int wm = w / NWN, wn = w % NWN;
  const int n0 = blockIdx.x * BN;
  const int chunk = blockIdx.y;
  const int ntiles_v = (V + BM - 1) / BM;
  const int t_begin = chunk * chunk_tiles;
  const int t_end = min(ntiles_v, t_begin + chunk_tiles);
  const Operand A{e, d, V, d};
  const Operand B{h, d, N, d};
  int tok[TJ], tgt[TJ];
  float m_st[TJ], l_st[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    tok[j] = n0 + WTN * wn + 32 * j + c32;
    tgt[j] = tok[j] < N ? targets[tok[j]] : -1;
    m_st[j] = -1e30f;
    l_st[j] = 0.0f;
  }
  // Statistic update of one vocabulary tile; FULL: every row of the tile is
  // inside the vocabulary (all but the last tile), so no row mask is formed.
  auto consume = [&](auto full_tag, int m0, const Acc& acc) {
    constexpr bool FULL = decltype(full_tag)::value;
    const int mw = m0 + WTM * wm;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      // The target logit: one lane of one 32-row block holds it.
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const int off = tgt[j] - (mw + 32 * i);
        if (off >= 0 && off < 32 && ((off >> 2) & 1) == g) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (8 * (r >> 2) + (r & 3) == (off & ~4)) zt[tok[j]] = acc.v[i][j][r];
        }
      }
      float tile_max = -1e30f;
      if (KIND == ALGX_HEAD_CE) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = mw + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
            if (FULL || m < V) tile_max = __builtin_fmaxf(tile_max, acc.v[i][j][r]);
          }
      }
      const float m_new = __builtin_fmaxf(m_st[j], tile_max);
      float lsum = 0.0f;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = mw + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
          const float z = acc.v[i][j][r];
          float wgt;
          if (KIND == ALGX_HEAD_CE) {
            wgt = __builtin_amdgcn_exp2f((z - m_new) * 1.4426950408889634f);
          } else {
            float rr;
            wgt = alg_weight<L2N>(z, inv_c, clamp, log2n, rr);
          }
          lsum += (FULL || m < V) ? wgt : 0.0f;
        }
      if (KIND == ALGX_HEAD_CE) {
        l_st[j] = l_st[j] * __builtin_amdgcn_exp2f((m_st[j] - m_new) * 1.4426950408889634f) + lsum;
        m_st[j] = m_new;
      } else {
        l_st[j] += lsum;
      }
    }
  };
  Acc acc;
  if constexpr (DMA) {
    gemm_seq_dma<true, true>(A, B, t_begin * BM, t_end - t_begin, n0, ring, acc, tid,
                             [&](int, int m0, const Acc& a) {
                               if (m0 + BM <= V)
                                 consume(std::true_type{}, m0, a);
                               else
                                 consume(std::false_type{}, m0, a);
                             });
  } else {
    for (int t = t_begin; t < t_end; ++t) {
      const int m0 = t * BM;
      gemm_tile<true, true>(A, B, m0, n0, s0, s0 + 2 * kStageElems, acc, tid);
      if (m0 + BM <= V)
        consume(std::true_type{}, m0, acc);
      else
        consume(std::false_type{}, m0, acc);
    }
  }
  // Merge the 4 partial states of each token: lane halves g, then waves wm.
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    float mo = __shfl_xor(m_st[j], 32, 64), lo = __shfl_xor(l_st[j], 32, 64);
    if (KIND == ALGX_HEAD_CE) {
      const float mm = __builtin_fmaxf(m_st[j], mo);
      l_st[j] = l_st[j] * __builtin_amdgcn_exp2f((m_st[j] - mm) * 1.4426950408889634f) +
                lo * __builtin_amdgcn_exp2f((mo - mm) * 1.4426950408889634f);
      m_st[j] = mm;
    } else {
      l_st[j] += lo;
    }
    if (g == 0) {
      red_m[wm][WTN * wn + 32 * j + c32] = m_st[j];
      red_l[wm][WTN * wn + 32 * j + c32] = l_st[j];
    }
  }
  __syncthreads();
  if (tid < BN) {
    const int col = tid;
    const float m_a = red_m[0][col], l_a = red_l[0][col];
    const float m_b = red_m[1][col], l_b = red_l[1][col];
    float m_out, l_out;
    if (KIND == ALGX_HEAD_CE) {
      m_out = __builtin_fmaxf(m_a, m_b);
      l_out = l_a * __builtin_amdgcn_exp2f((m_a - m_out) * 1.4426950408889634f) +
              l_b * __builtin_amdgcn_exp2f((m_b - m_out) * 1.4426950408889634f);
    } else {
      m_out = 0.0f;
      l_out = l_a + l_b;
    }
    const int token = n0 + col;
    if (token < N) {
      partial[((int64_t)chunk * N + token) * 2 + 0] = m_out;
      partial[((int64_t)chunk * N + token) * 2 + 1] = l_out;
    }
  }
}

// stat = m + log l (ce) or l^(-1/n) (alg_ce) from the chunk partials
// (fused_head.py:113-116).
template <int KIND>
__global__ __launch_bounds__(256) void head_stat_kernel(const float* __restrict__ partial,
                                                        int nchunks, int N, int log2n,
                                                        float* __restrict__ stat) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= N) return;
  float m = -1e30f, l = 0.0f;
  for (int c = 0; c < nchunks; ++c) {
    const float mc = partial[((int64_t)c * N + t) * 2 + 0];
    const float lc = partial[((int64_t)c * N + t) * 2 + 1];
    if (KIND == ALGX_HEAD_CE) {
      const float mm = __builtin_fmaxf(m, mc);
      l = l * __expf(m - mm) + lc * __expf(mc - mm);
      m = mm;
    } else {
      l += lc;
    }
  }
  stat[t] = KIND == ALGX_HEAD_CE ? m + __logf(l) : inv_root(l, log2n);
}

// dz tile of a token chunk: dz[t][v] = bf16(f(z) * scale), 0 for padded v.
template <int KIND, int L2N, bool DMA>
__global__ __launch_bounds__(kThreads) void head_dz_kernel(
    const bf16* __restrict__ h, const bf16* __restrict__ e, const int32_t* __restrict__ targets,
    const float* __restrict__ stat, const float* __restrict__ scale, bf16* __restrict__ dz,
    int64_t ldz, int tok0, int ntok, int d, int V, int log2n, float inv_c, float clamp,
    int chunk_tiles) {
  GEMM_LDS_STAGES;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int wm = w / NWN, wn = w % NWN;
  const int n0 = blockIdx.x * BN;  // token offset inside the chunk
  const int ntiles_v = (V + BM - 1) / BM;
  const int t_begin = blockIdx.y * chunk_tiles;
  const int t_end = min(ntiles_v, t_begin + chunk_tiles);
  const Operand A{e, d, V, d};
  const Operand B{h + (int64_t)tok0 * d, d, ntok, d};
  // The lane's tokens (the same for every vocabulary tile), read before the
  // loads of the stage ring start.
  int tgt_j[TJ];
  float st_j[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int tl = n0 + WTN * wn + 32 * j + c32;
    tgt_j[j] = tl < ntok ? targets[tok0 + tl] : -1;
    st_j[j] = tl < ntok ? stat[tok0 + tl] : 0.0f;
  }
  const float sc = scale[0];
  // FULL: every row of the tile is inside the vocabulary (all but the last
  // vocabulary tile), so no row mask is formed.
  auto emit = [&](auto full_tag, int m0, const Acc& acc) {
    constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int tl = n0 + WTN * wn + 32 * j + c32;
      if (tl >= ntok) continue;
      const int tgt = tgt_j[j];
      const float st = st_j[j];
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int mb = m0 + WTM * wm + 32 * i + 8 * q4 + 4 * g;
          bf16x4 out;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int m = mb + u;
            const float z = acc.v[i][j][4 * q4 + u];
            const float y = m == tgt ? 1.0f : 0.0f;
            float g_z;
            if (KIND == ALGX_HEAD_CE) {
              g_z = __builtin_amdgcn_exp2f((z - st) * 1.4426950408889634f) - y;
            } else {
              const float x = __builtin_fminf(z * inv_c, clamp);
              float r;
              const float p = pow_n<L2N>(rho_fast(x, r) * st, log2n);
              g_z = (p - y) * r;
            }
            out[u] = (bf16)((FULL || m < V) ? g_z * sc : 0.0f);
          }
          *reinterpret_cast<bf16x4*>(dz + (int64_t)tl * ldz + mb) = out;
        }
    }
  };
  auto emit_tile = [&](int, int m0, const Acc& a) {
    if (m0 + BM <= V)
      emit(std::true_type{}, m0, a);
    else
      emit(std::false_type{}, m0, a);
  };
  Acc acc;
  if constexpr (DMA) {
    gemm_seq_dma<true, true>(A, B, t_begin * BM, t_end - t_begin, n0, ring, acc, tid, emit_tile);
  } else {
    for (int t = t_begin; t < t_end; ++t) {
      gemm_tile<true, true>(A, B, t * BM, n0, s0, s0 + 2 * kStageElems, acc, tid);
      emit_tile(t, t * BM, acc);
    }
  }
}

// One GEMM of a grouped launch: C[m][n] (+)= sum_k A(m,k) B(n,k).
struct GemmJob {
  Operand A, B;
  void* C;
  int64_t ldc;
  int M, N;
  int tiles_n;  // output tiles along n
};

template <bool AKC, bool BKC, typename TOut, bool ACCUM, bool DMA>
__device__ __forceinline__ void gemm_job(const GemmJob& jb, int tile, bf16* lds,
                                         const DmaRing& ring, int tid) {
  const int w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int wm = w / NWN, wn = w % NWN;
  const int m0 = (tile / jb.tiles_n) * BM, n0 = (tile % jb.tiles_n) * BN;
  Acc acc;
  if (DMA)
    gemm_tile_dma<AKC, BKC>(jb.A, jb.B, m0, n0, ring, acc, tid);
  else
    gemm_tile<AKC, BKC>(jb.A, jb.B, m0, n0, lds, lds + 2 * kStageElems, acc, tid);
  TOut* C = reinterpret_cast<TOut*>(jb.C);
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int n = n0 + WTN * wn + 32 * j + c32;
      if (n >= jb.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + WTM * wm + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m >= jb.M) continue;
        TOut* dst = C + (int64_t)m * jb.ldc + n;
        if (ACCUM)
          *dst = from_f<TOut>(to_f(*dst) + acc.v[i][j][r]);
        else
          *dst = from_f<TOut>(acc.v[i][j][r]);
      }
    }
}

// XCD-aware tile order of a grouped GEMM: workgroups are dealt to the 8 XCDs
// round-robin by index, so the tiles_n output tiles that share one row block
// of A (one dz block) go to indices 8 apart, i.e. to one XCD and its L2, and
// run at about the same time. Index `b` counts from a multiple of 8; a
// trailing partial group keeps the plain order.
__device__ __forceinline__ int xcd_tile(int b, int ntiles, int tiles_n) {
  const int grp = 8 * tiles_n;
  const int full = ntiles / grp * grp;
  if (b >= full) return b;
  const int r = b % grp;
  return ((b / grp) * 8 + (r & 7)) * tiles_n + (r >> 3);
}

// The backward's two products of a token chunk in one launch (the long-K dh
// tiles first): dh[t][c] = sum_v dz[t][v] E[v][c] in the first dh_slots
// workgroups (n_dh tiles; dh_slots is n_dh rounded up to a multiple of 8),
// then dE[v][c] (+)= sum_t dz[t][v] h[t][c].
template <bool ACCUM, bool DMA>
__global__ __launch_bounds__(kThreads) void head_grad_kernel(GemmJob dh, GemmJob de, int n_dh,
                                                             int dh_slots, int n_de) {
  GEMM_LDS_STAGES;
  const int b = blockIdx.x;
  if (b < dh_slots) {
    if (b < n_dh)
      gemm_job<true, false, bf16, false, DMA>(dh, xcd_tile(b, n_dh, dh.tiles_n), s0, ring,
                                              threadIdx.x);
  } else {
    gemm_job<false, false, float, ACCUM, DMA>(de, xcd_tile(b - dh_slots, n_de, de.tiles_n), s0,
                                              ring, threadIdx.x);
  }
}

int64_t vpad_of(int V) { return ((int64_t)V + BM - 1) / BM * BM; }

// Token chunk of the backward: bounds the bf16 dz scratch to 2 GiB (all
// 16384 tokens of a 50304-word vocabulary in one chunk), or to
// ALGX_HEAD_CHUNK_BYTES when that is set.
int chunk_tokens(int N, int V) {
  const int64_t per_tok = vpad_of(V) * 2;
  int64_t limit = (int64_t)2 << 30;
  if (const char* env = std::getenv("ALGX_HEAD_CHUNK_BYTES")) {
    const long long v = std::atoll(env);
    if (v > 0) limit = v;
  }
  int64_t c = limit / per_tok;
  c = c / BN * BN;
  if (c < BN) c = BN;
  return (int)(c > N ? ((N + BN - 1) / BN) * BN : c);
}

int32_t check_head(const void* h, const void* E, const int32_t* targets, int N, int d, int V,
                   int kind, int n, int dtype) {
  if (N < 0 || d <= 0 || V <= 0) return fail("head: invalid sizes");
  if (dtype != ALGX_BF16 && dtype != ALGX_F32) return fail("head: dtype must be bf16 or f32");
  if (dtype == ALGX_BF16 && d % 8) return fail("head: hidden width must be a multiple of 8");
  if (kind != ALGX_HEAD_CE && kind != ALGX_HEAD_ALG_CE) return fail("head: unknown kind");
  if (kind == ALGX_HEAD_ALG_CE && (n < 1 || (n & (n - 1)))) return fail("head: n must be a power of two");
  if (N > 0 && (h == nullptr || E == nullptr || targets == nullptr)) return fail("head: null input");
  return 0;
}

typedef void (*HeadFwdFn)(const bf16*, const bf16*, const int32_t*, float*, float*, int, int,
                          int, int, float, float, int);
typedef void (*HeadDzFn)(const bf16*, const bf16*, const int32_t*, const float*, const float*,
                         bf16*, int64_t, int, int, int, int, int, float, float, int);

// Kernel instance for (kind, n): alg_ce with n = 8, 16 or 32 gets unrolled
// powers. DMA (the direct-to-LDS ring) when d is a multiple of BK.
template <bool DMA> HeadFwdFn pick_head_fwd_as(int kind, int log2n) {
  if (kind == ALGX_HEAD_CE) return head_fwd_kernel<ALGX_HEAD_CE, 0, DMA>;
  switch (log2n) {
    case 3: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 3, DMA>;
    case 4: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 4, DMA>;
    case 5: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 5, DMA>;
    default: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 0, DMA>;
  }
}
template <bool DMA> HeadDzFn pick_head_dz_as(int kind, int log2n) {
  if (kind == ALGX_HEAD_CE) return head_dz_kernel<ALGX_HEAD_CE, 0, DMA>;
  switch (log2n) {
    case 3: return head_dz_kernel<ALGX_HEAD_ALG_CE, 3, DMA>;
    case 4: return head_dz_kernel<ALGX_HEAD_ALG_CE, 4, DMA>;
    case 5: return head_dz_kernel<ALGX_HEAD_ALG_CE, 5, DMA>;
    default: return head_dz_kernel<ALGX_HEAD_ALG_CE, 0, DMA>;
  }
}
HeadFwdFn pick_head_fwd(int kind, int log2n, int d) {
  return d % (BK * kDmaStages) == 0 ? pick_head_fwd_as<true>(kind, log2n)
                                    : pick_head_fwd_as<false>(kind, log2n);
}
HeadDzFn pick_head_dz(int kind, int log2n, int d) {
  return d % (BK * kDmaStages) == 0 ? pick_head_dz_as<true>(kind, log2n)
                                    : pick_head_dz_as<false>(kind, log2n);
}

// Vocabulary tiles per forward workgroup: the token blocks x vocabulary tiles
// dealt out in about kFwdWorkgroups equal chunks (one round of the CUs), so
// no partial last round of workgroups is left.
int chunk_tiles_of(int N, int V) {
  const int64_t ntv = (V + BM - 1) / BM, ntb = (N + BN - 1) / BN;
  const int64_t per = (ntv * ntb + kFwdWorkgroups - 1) / kFwdWorkgroups;
  const int64_t nch = (ntv + per - 1) / per;
  return (int)((ntv + nch - 1) / nch);
}
int nchunks_of(int N, int V) {
  const int nt = (V + BM - 1) / BM, ct = chunk_tiles_of(N, V);
  return (nt + ct - 1) / ct;
}

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int64_t algx_head_fwd_workspace_bytes(int32_t N, int32_t d, int32_t V, int32_t dtype) {
  (void)d;
  if (N <= 0 || V <= 0) return 0;
  if (dtype == ALGX_F32) return head_f32_fwd_workspace(N, V);
  return (int64_t)nchunks_of(N, V) * N * 2 * sizeof(float);
}

extern "C" int32_t algx_head_fwd(const void* h, const void* E, const int32_t* targets,
                                 float* stat, float* zt, void* workspace, int32_t N, int32_t d,
                                 int32_t V, int32_t kind, int32_t n, float inv_c, float clamp,
                                 int32_t dtype, void* stream) {
  if (int32_t rc = check_head(h, E, targets, N, d, V, kind, n, dtype)) return rc;
  if (N == 0) return 0;
  if (stat == nullptr || zt == nullptr || workspace == nullptr) return fail("head_fwd: null output");
  hipStream_t s = (hipStream_t)stream;
  const int nch = nchunks_of(N, V);
  dim3 grid((N + BN - 1) / BN, nch);
  const int log2n = kind == ALGX_HEAD_ALG_CE ? ilog2(n) : 0;
  float* partial = (float*)workspace;
  // The target logit starts at 0 as in fused_head.py:80 (a target outside
  // the vocabulary tiles is never met).
  if (int32_t rc = fill_f32(zt, N, 0.0f, s)) return rc;
  if (dtype == ALGX_F32)
    return head_f32_fwd((const float*)h, (const float*)E, targets, stat, zt, partial, N, d, V,
                        kind, log2n, inv_c, clamp, s);
  {
    const Probe probe = probe_for(ALGX_PROBE_HEAD_FWD);
    launch_k(probe, pick_head_fwd(kind, log2n, d),
             grid, dim3(kThreads), s, (const bf16*)h, (const bf16*)E, targets, zt, partial, N, d,
             V, log2n, inv_c, clamp, chunk_tiles_of(N, V));
  }
  if (int32_t rc = check_launch("head_fwd")) return rc;
  const int nb = (N + 255) / 256;
  if (kind == ALGX_HEAD_CE)
    head_stat_kernel<ALGX_HEAD_CE><<<nb, 256, 0, s>>>(partial, nch, N, log2n, stat);
  else
    head_stat_kernel<ALGX_HEAD_ALG_CE><<<nb, 256, 0, s>>>(partial, nch, N, log2n, stat);
  return check_launch("head_stat");
}

extern "C" int64_t algx_head_bwd_workspace_bytes(int32_t N, int32_t d, int32_t V, int32_t dtype) {
  (void)d;
  if (N <= 0 || V <= 0) return 0;
  if (dtype == ALGX_F32) return head_f32_bwd_workspace(N, V);
  return (int64_t)chunk_tokens(N, V) * vpad_of(V) * 2;
}

extern "C" int32_t algx_head_bwd(const void* h, const void* E, const int32_t* targets,
                                 const float* stat, const float* scale, void* dh, float* dE,
                                 void* workspace, int32_t N, int32_t d, int32_t V, int32_t kind,
                                 int32_t n, float inv_c, float clamp, int32_t dtype,
                                 void* stream) {
  if (int32_t rc = check_head(h, E, targets, N, d, V, kind, n, dtype)) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (dE == nullptr) return fail("head_bwd: null dE");
  if (N == 0) return fill_f32(dE, (int64_t)V * d, 0.0f, s);
  if (stat == nullptr || scale == nullptr || dh == nullptr || workspace == nullptr)
    return fail("head_bwd: null pointer");
  const int log2n = kind == ALGX_HEAD_ALG_CE ? ilog2(n) : 0;
  if (dtype == ALGX_F32)
    return head_f32_bwd((const float*)h, (const float*)E, targets, stat, scale, (float*)dh, dE,
                        (float*)workspace, N, d, V, kind, log2n, inv_c, clamp, s);
  const int64_t ldz = vpad_of(V);
  const int csize = chunk_tokens(N, V);
  bf16* dz = (bf16*)workspace;
  const bf16* hb = (const bf16*)h;
  const bf16* eb = (const bf16*)E;
  for (int tok0 = 0; tok0 < N; tok0 += csize) {
    const int ntok = min(csize, N - tok0);
    const int ct = chunk_tiles_of(ntok, V);
    dim3 gdz((ntok + BN - 1) / BN, ((V + BM - 1) / BM + ct - 1) / ct);
    launch_k(probe_for(ALGX_PROBE_HEAD_DZ),
             pick_head_dz(kind, log2n, d),
             gdz, dim3(kThreads), s, hb, eb, targets, stat, scale, dz, ldz, tok0, ntok, d, V, log2n,
             inv_c, clamp, ct);
    if (int32_t rc = check_launch("head_dz")) return rc;
    // dh[t][c] = sum_v dz[t][v] E[v][c]: A = dz (k-contiguous), B(n=c,k=v) = E stored [v][c].
    // dE[v][c] (+)= sum_t dz[t][v] h[t][c]: A(m=v,k=t) = dz stored [t][v], B(n=c,k=t) = h [t][c].
    const int tn = (d + BN - 1) / BN;
    const GemmJob jdh{Operand{dz, ldz, ntok, V}, Operand{eb, d, d, V},
                      (bf16*)dh + (int64_t)tok0 * d, (int64_t)d, ntok, d, tn};
    const GemmJob jde{Operand{dz, ldz, V, ntok}, Operand{hb + (int64_t)tok0 * d, d, d, ntok},
                      dE, (int64_t)d, V, d, tn};
    const int n_dh = ((ntok + BM - 1) / BM) * tn;
    const int n_de = ((V + BM - 1) / BM) * tn;
    const int dh_slots = (n_dh + 7) / 8 * 8;
    // LDS-DMA stages when both products have whole k stages (V and the
    // chunk's token count multiples of BK).
    const bool dma = V % BK == 0 && ntok % BK == 0;
    auto gk = dma ? (tok0 == 0 ? head_grad_kernel<false, true> : head_grad_kernel<true, true>)
                  : (tok0 == 0 ? head_grad_kernel<false, false> : head_grad_kernel<true, false>);
    launch_k(probe_for(ALGX_PROBE_HEAD_DE), gk, dim3(dh_slots + n_de), dim3(kThreads), s, jdh, jde,
             n_dh, dh_slots, n_de);
    if (int32_t rc = check_launch("head_grad")) return rc;
  }
  return 0;
}
