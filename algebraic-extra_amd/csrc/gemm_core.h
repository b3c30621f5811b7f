// The bf16 MFMA GEMM core of the gfx950 kernels (fused head, batched GEMMs):
// 256 x 256 output tiles of 8 waves (each 128 x 64, v_mfma_f32_32x32x16_bf16),
// operands k-contiguous ([mn][k]) or [k][mn] (read through transposing LDS
// reads), k streamed through LDS in 32-wide stages, either staged through
// registers (gemm_tile: any K) or moved by LDS-DMA loads in a four-stage ring
// (gemm_seq_dma / gemm_tile_dma: K a multiple of 32).
#pragma once

#include "common.h"

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
  // 0: plain row-major storage. Otherwise the operand is stored in blocks of
  // 32 contiguous columns of the row-major matrix ([cols / 32][rows][32],
  // ld = 32) and bstride is the distance between blocks; the direct-to-LDS
  // path reads it (whole 64-byte row pieces per 32-wide k stage), the
  // register-staged path does not.
  int64_t bstride = 0;
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
#ifndef ALGX_DMA_SLOTS
#define ALGX_DMA_SLOTS 4
#endif
constexpr int kDmaStages = ALGX_DMA_SLOTS;
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
    const int64_t at = op.bstride ? (int64_t)(col >> 5) * op.bstride + (col & 31) : col;
    return col < op.rows ? op.p + (int64_t)r * op.ld + at : op.p;
  }
}

// Elements between consecutive 32-wide k stages of an operand.
template <bool KC>
__device__ __forceinline__ int64_t kstep(const Operand& op) {
  if (KC) return op.bstride ? op.bstride : BK;  // the next 32-column block
  return (int64_t)BK * op.ld;                    // the next 32 rows
}

// Bytes from op.p to the end of the last 16-byte piece the direct-to-LDS
// loads of a (KC or [k][mn]-stored) operand can read (k stages of BK up to
// op.K, mn up to op.rows), and whether that fits the loads' 32-bit offsets
// (with their 1024-byte bias and room to spare). Operands beyond it take the
// register-staged stages.
__host__ __device__ inline int64_t dma_span_bytes(const Operand& op, bool kc) {
  const int64_t stages = (op.K + BK - 1) / BK;
  int64_t last;  // element offset of the last element read
  if (kc) {
    const int64_t step = op.bstride ? op.bstride : BK;
    last = (stages - 1) * step + (int64_t)(op.rows - 1) * op.ld + (BK - 1);
  } else {
    const int64_t col = op.rows - 1 + 7;  // a piece may run to 7 past the last column
    const int64_t at = op.bstride ? (col >> 5) * op.bstride + (col & 31) : col;
    last = (stages * BK - 1) * op.ld + at;
  }
  return (last + 8) * (int64_t)sizeof(bf16);
}
__host__ __device__ inline bool dma_span_ok(const Operand& op, bool kc) {
  return op.rows > 0 && op.K > 0 && dma_span_bytes(op, kc) <= (int64_t(1) << 32) - 4096;
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

// One LDS-DMA load of a wave: lane i's 16 bytes at sbase + voff (a uniform
// 64-bit base in SGPRs plus the lane's 32-bit byte offset, the instruction's
// scalar-base form) go to lds + 16 i (lds wave-uniform). The scalar-base
// form hands the address unit one 32-bit offset per lane instead of a 64-bit
// address, which a standalone copy of the k loop measured 1-5 % faster.
// Issued as inline assembly so that the compiler does not track it: its
// waitcnt pass cannot tell which LDS buffer such a load writes and would wait
// for all of them before every LDS read; the ring below waits for its own
// loads explicitly (wait_vm) before the barrier that publishes them. The
// assembly sets M0 itself and names it as clobbered; the compiler treats M0
// as reserved and uses it nowhere in these kernels (no indirect register
// indexing, GWS or compiler-issued LDS DMA: every M0 write in their generated
// code is one of these loads), so no value of its own lives in M0 across the
// statement.
__device__ __forceinline__ void dma16s(const void* sbase, unsigned voff, unsigned lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff),
               "s"(sbase)
               : "memory", "m0");
}

// Two such loads under one M0: the first block's 16-byte lanes go to
// lds + 16 i, the second's to lds + 1024 + 16 i through the instruction
// offset, which the global address takes too (so voff1m is the second
// block's byte offset minus 1024).
__device__ __forceinline__ void dma16x2s(const void* sbase, unsigned voff0, unsigned voff1m,
                                         unsigned lds) {
  asm volatile(
      "s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %3\n\t"
      "global_load_lds_dwordx4 %2, %3 offset:1024" ::"s"(lds),
      "v"(voff0), "v"(voff1m), "s"(sbase)
      : "memory", "m0");
}

// s_waitcnt immediates: vmcnt(n) with expcnt and lgkmcnt unconstrained.
template <int N> __device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// Ring of stage buffers (32 KB each: the A stage, then the B stage).
struct DmaRing {
  bf16* slot[5];
};

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Products of a sequence of `ntiles` output tiles with nk k stages each:
// src(t, a0, a1, b0, b1) gives the wave's four LDS-DMA sources of tile t at
// k = 0 (dma_src of its A and B blocks 2w and 2w + 1, inside the operands
// that start at baseA / baseB, each spanning less than 4 GiB - 2 KiB; the
// operands' k steps stepA / stepB are the same for every tile), epi(t, acc)
// receives each finished tile. The ring streams across the tiles, so a tile's first stages
// load during the previous tile's last stages and epilogue. Several tiles
// need nk to be a multiple of the ring's stage count (every tile starts at
// slot 0).
//
// Each step's refill (four loads of the stage two ahead, as two pairs that
// share one M0 write) is issued between the MFMAs of the step's second half,
// not in a burst ahead of them. With STORE_HEAVY false the loop has no
// branch: a step with nothing to refill (a tile's first step, whose refill
// ran before the previous epilogue, and the steps past the sequence's end)
// repeats a load that changes nothing: the stage already in flight into the
// same slot, or the stage being read into the slot just consumed, which
// nothing reads again. Kernels whose epilogue stores a whole output tile pass
// STORE_HEAVY: such a repeated load would queue behind those stores and hold
// up the next wait, so they skip it with a branch instead. The loads take
// the scalar-base form: the lane's source as a 32-bit byte offset from the
// operand base, biased by 1024 (with the scalar base 1024 bytes low), so that
// a pair's second block, whose offset is passed 1024 bytes low for the
// instruction offset to add back, stays non-negative even for a source
// clamped to the base itself (dma_src's op.p).
template <bool AKC, bool BKC, bool STORE_HEAVY = false, typename Src, typename Epi>
__device__ __forceinline__ void gemm_stream_dma(int nk, int64_t stepA, int64_t stepB,
                                                const bf16* baseA, const bf16* baseB, int ntiles,
                                                Src&& src, const DmaRing& ring, Acc& acc,
                                                int tid, Epi&& epi) {
  constexpr int S = kDmaStages, L = S - 2;  // stages in flight beyond the one being read
  const int w = tid >> 6, lane = tid & 63;
  const int wm = w / NWN, wn = w % NWN;
  const int G = ntiles * nk;  // stages of the whole sequence
  // The lane's biased byte offsets of a source pair from its operand base,
  // and the scalar base of stage kk (1024 bytes below the stage's start).
  auto boff = [](const bf16* q, const bf16* base) { return (unsigned)((q - base) * 2) + 1024u; };
  auto sbase = [](const bf16* base, int64_t koff) {
    return reinterpret_cast<const void*>(reinterpret_cast<uintptr_t>(base + koff) - 1024u);
  };
  unsigned oa0, oa1, ob0, ob1;  // sources of the tile being issued
  {
    const bf16 *a0, *a1, *b0, *b1;
    src(0, a0, a1, b0, b1);
    oa0 = boff(a0, baseA), oa1 = boff(a1, baseA), ob0 = boff(b0, baseB), ob1 = boff(b1, baseB);
  }
  // Byte offset of the wave's two 1 KB blocks in an operand stage (uniform).
  const unsigned wofs = 2048u * __builtin_amdgcn_readfirstlane(w);
  // The wave's two 1 KB blocks of each operand of stage kk -> slot.
  auto issue = [&](unsigned a0, unsigned a1, unsigned b0, unsigned b1, int kk, bf16* slot) {
    const unsigned dA = lds_addr(slot) + wofs, dB = dA + 2 * kDmaOpElems;
    // Stage offsets as scalars computed here (the compiler would otherwise
    // keep one vector induction variable per unrolled stage).
    int64_t ka = kk * stepA, kb = kk * stepB;
    asm volatile("" : "+s"(ka), "+s"(kb));
    const void* sA = sbase(baseA, ka);
    const void* sB = sbase(baseB, kb);
    dma16s(sA, a0, dA);
    dma16s(sA, a1, dA + 1024);
    dma16s(sB, b0, dB);
    dma16s(sB, b1, dB + 1024);
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
    if (u < nk) issue(oa0, oa1, ob0, ob1, u, ring.slot[u]);
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
    // Sources of the next tile, for the stages issued near this tile's end.
    unsigned na0 = oa0, na1 = oa1, nb0 = ob0, nb1 = ob1;
    if (t + 1 < ntiles) {
      const bf16 *a0, *a1, *b0, *b1;
      src(t + 1, a0, a1, b0, b1);
      na0 = boff(a0, baseA), na1 = boff(a1, baseA), nb0 = boff(b0, baseB), nb1 = boff(b1, baseB);
    }
    const int g0 = t * nk;
    // `synced`: this stage's wait, barrier and refill already ran before the
    // previous tile's epilogue (the first stage of every tile but the first);
    // `landed`: this wave's loads of the stage it waits for are known to have
    // landed (the second stage of such a tile), so only the barrier remains.
    auto step = [&](int kk, const bf16* cur, const bf16* nxt, bf16* refill, bool synced,
                    bool landed) {
      rd(cur, 1, ya, yb);
      __builtin_amdgcn_sched_barrier(0);
      mm(xa, xb);
      __builtin_amdgcn_sched_barrier(0);
      if (!synced) {
        // Wait for stage g + 1; the stages issued after it may stay in flight.
        const int g = g0 + kk;
        if (!landed) wait_stages(min(g + S - 2, G - 1) - (g + 1));
        asm volatile("s_barrier" ::: "memory");
      }
      rd(nxt, 0, xa, xb);
      // The refill: stage kk + S - 1 of this tile, else of the next tile, else
      // (past the end) a repeat of stage kk into the slot just consumed.
      const bool here = kk + S - 1 < nk, next = !here && t + 1 < ntiles;
      const bool fill = !STORE_HEAVY || (!synced && (here || next));
      const unsigned p0 = next ? na0 : oa0, p1 = next ? na1 : oa1;
      const unsigned q0 = next ? nb0 : ob0, q1 = next ? nb1 : ob1;
      const int ks = here ? kk + S - 1 : next ? kk + S - 1 - nk : kk;
      const unsigned dA = lds_addr(refill) + wofs, dB = dA + 2 * kDmaOpElems;
      int64_t ka = ks * stepA, kb = ks * stepB;
      asm volatile("" : "+s"(ka), "+s"(kb));
      const void* sA = sbase(baseA, ka);
      const void* sB = sbase(baseB, kb);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          acc.v[i][j] = mfma32(ya[i], yb[j], acc.v[i][j]);
          if (j == TJ - 1 && fill) {
            if (i == 1) dma16x2s(sA, p0, p1 - 1024u, dA);
            if (i == 3) dma16x2s(sB, q0, q1 - 1024u, dB);
          }
        }
    };
    // Slots are named statically: S stages a turn.
    for (int kk = 0; kk < nk; kk += S) {
#pragma unroll
      for (int u = 0; u < S; ++u)
        if (kk + u < nk)
          step(kk + u, ring.slot[u], ring.slot[(u + 1) % S], ring.slot[(u + S - 1) % S],
               u == 0 && kk == 0 && t > 0, S >= 4 && u == 1 && kk == 0 && t > 0);
    }
    if (t + 1 < ntiles) {
      // Global stores count in vmcnt, and the loads and stores of one wave
      // are not known to retire in order, so a vmcnt wait only bounds the
      // loads still in flight. A wait issued after this tile's epilogue stores
      // would therefore also wait for them to land. So the next tile's first
      // wait, barrier and refill (stage S - 1 of that tile; nk >= S here) run
      // before the epilogue, and so does the wait for the next tile's stage 2
      // (with S >= 4: only stage S - 1 may stay in flight), which the second
      // stage would otherwise wait for. The stores then have two stages of
      // MFMA work before a wait can meet them.
      const int g = g0 + nk;
      wait_stages(min(g + S - 2, G - 1) - (g + 1));
      asm volatile("s_barrier" ::: "memory");
      issue(na0, na1, nb0, nb1, S - 1, ring.slot[S - 1]);
      if (S >= 4) wait_vm<4>();
    } else if (!STORE_HEAVY) {
      // The last step's repeated load may still be writing the ring: let it
      // land before the workgroup can end and its LDS be reassigned.
      wait_vm<0>();
    }
    epi(t, acc);
    acc.zero();
    oa0 = na0;
    oa1 = na1;
    ob0 = nb0;
    ob1 = nb1;
  }
}

// Products of `ntiles` output tiles that share the B rows n0: tile t uses A
// rows m0 + t BM; epi(t, m0 + t BM, acc) receives each finished tile.
template <bool AKC, bool BKC, bool STORE_HEAVY = false, typename Epi>
__device__ __forceinline__ void gemm_seq_dma(const Operand& A, const Operand& B, int m0,
                                             int ntiles, int n0, const DmaRing& ring, Acc& acc,
                                             int tid, Epi&& epi) {
  const int w = tid >> 6, lane = tid & 63;
  const bf16* b0 = dma_src<BKC>(B, n0, 2 * w, lane);
  const bf16* b1 = dma_src<BKC>(B, n0, 2 * w + 1, lane);
  gemm_stream_dma<AKC, BKC, STORE_HEAVY>(
      A.K / BK, kstep<AKC>(A), kstep<BKC>(B), A.p, B.p, ntiles,
      [&](int t, const bf16*& a0, const bf16*& a1, const bf16*& sb0, const bf16*& sb1) {
        a0 = dma_src<AKC>(A, m0 + t * BM, 2 * w, lane);
        a1 = dma_src<AKC>(A, m0 + t * BM, 2 * w + 1, lane);
        sb0 = b0;
        sb1 = b1;
      },
      ring, acc, tid, [&](int t, Acc& a) { epi(t, m0 + t * BM, a); });
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
  __shared__ __attribute__((aligned(16))) bf16 s4[DMA && kDmaStages > 4 ? 2 * kDmaOpElems : 8]; \
  const DmaRing ring{{s0, s1, s2, s3, s4}}

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

}  // namespace
}  // namespace algx
