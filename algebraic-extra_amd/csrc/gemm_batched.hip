// Batched bf16 GEMM with a fused linear combination, on the MFMA GEMM core:
//   C[b] = alpha * opA(A[b]) opB(B[b])^T + beta * D[b]
// with opA(m, k) = A[m*lda + k] (k-contiguous) or A[k*lda + m], opB(n, k)
// likewise. It carries Muon's Newton-Schulz products (optimizers.py:27-65):
// the Gram matrix X X^T (both operands k-contiguous, so no transpose is
// formed), b A + c A A and a X + B X (the second operand [k][n], read through
// transposing LDS reads), each written to its own buffer with the
// combination in the epilogue.
#include <utility>

#include "gemm_core.h"

namespace algx {
namespace {

struct BatchGemm {
  const bf16* A;
  const bf16* B;
  const bf16* D;  // null: beta is not applied
  bf16* C;
  int64_t lda, ldb, ldd, ldc;
  int64_t sa, sb, sd, sc;  // batch strides (elements)
  int M, N, K;
  float alpha, beta;
  int tiles_m, tiles_n;
  int batch;
  int ntiles;  // tiles per matrix (upper triangle only when symmetric)
};

// Up to kMaxGroups batches of one launch. Group i owns workgroups
// [start[i], start[i + 1]); every start is a multiple of 8, so a workgroup's
// XCD (index mod 8) is the same counted from the launch or from its group.
constexpr int kMaxGroups = 4;
struct GemmGroups {
  BatchGemm g[kMaxGroups];
  int start[kMaxGroups + 1];
  int ngroups;
};

// Workgroup b -> (matrix, tile). Workgroups are dealt to the 8 XCDs
// round-robin by index; when the batch is a multiple of 8, matrix j's tiles
// go to indices congruent to j mod 8, i.e. all to one XCD and its L2, in
// consecutive order there.
__device__ __forceinline__ void batch_tile(int b, const BatchGemm& p, int& mat, int& tile) {
  const int T = p.ntiles;
  if (p.batch % 8 == 0) {
    const int x = b & 7, r = b >> 3;  // XCD, index within it
    mat = (r / T) * 8 + x;
    tile = r % T;
  } else {
    mat = b / T;
    tile = b % T;
  }
}

// Row-major index of tile (a, b), a <= b, of the upper triangle of t x t
// tiles -> (a, b).
__device__ __forceinline__ void upper_tile(int idx, int t, int& a, int& b) {
  a = 0;
  int row = t;  // tiles in row a of the triangle
  while (idx >= row) {
    idx -= row;
    --row;
    ++a;
  }
  b = a + idx;
}

// C[m][n] (+ beta D) of a finished 256 x 256 tile of C^T at (n0, m0):
// acc.v[i][j][4q + u] = C[m][n + u], m = m0 + WTN wn + 32 j + c32,
// n = n0 + WTM wm + 32 i + 8 q + 4 g (N % 8 == 0: a run is whole or absent).
// Each run's bf16 values also go to mirror(r, col, value4) when given. The
// D runs of one j are all loaded before any is used (outside rows and
// columns read D's first run instead), so a lane waits for D once per j
// rather than once per run.
template <typename Mirror>
__device__ __forceinline__ void store_tile(const BatchGemm& p, int mat, int m0, int n0,
                                           const Acc& acc, int tid, Mirror&& mirror) {
  const int w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int wm = w / NWN, wn = w % NWN;
  bf16* C = p.C + mat * p.sc;
  const bf16* D = p.D != nullptr ? p.D + mat * p.sd : nullptr;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int m = m0 + WTN * wn + 32 * j + c32;
    const bool m_in = m < p.M;
    bf16x4 d[TI][4];
    if (D != nullptr) {
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + WTM * wm + 32 * i + 8 * q + 4 * g;
          const int64_t at = m_in && n < p.N ? (int64_t)m * p.ldd + n : 0;
          d[i][q] = *reinterpret_cast<const bf16x4*>(D + at);
        }
    }
    if (!m_in) continue;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + WTM * wm + 32 * i + 8 * q + 4 * g;
        if (n >= p.N) continue;
        f32x4 v;
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = p.alpha * acc.v[i][j][4 * q + u];
        if (D != nullptr) {
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = __builtin_fmaf(p.beta, (float)d[i][q][u], v[u]);
        }
        const bf16x4 o = {(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
        *reinterpret_cast<bf16x4*>(C + (int64_t)m * p.ldc + n) = o;
        mirror(n - n0, m - m0, o);
      }
  }
}

// Each workgroup forms a 256 x 256 tile of C^T (the kernel's M axis runs
// over C's columns n, its N axis over C's rows m), so every lane holds runs
// of four consecutive columns of one row: C and D move in 8-byte pieces.
// SYM (C symmetric, M == N, D symmetric when present): only the tiles on and
// above the diagonal are formed; an off-diagonal tile's values also go to
// the mirrored tile, transposed through the idle stage buffers.
template <bool AKC, bool BKC, bool DMA, bool SYM>
__global__ __launch_bounds__(kThreads) void batched_gemm_kernel(GemmGroups gp) {
  GEMM_LDS_STAGES;
  const int tid = threadIdx.x;
  int gi = 0;
#pragma unroll
  for (int i = 1; i < kMaxGroups; ++i)
    if (i < gp.ngroups && (int)blockIdx.x >= gp.start[i]) gi = i;
  const BatchGemm p = gp.g[gi];
  const int local = (int)blockIdx.x - gp.start[gi];
  if (local >= p.batch * p.ntiles) return;  // padding of the group to a multiple of 8
  int mat, tile;
  batch_tile(local, p, mat, tile);
  int n0, m0;
  if (SYM) {
    int a, b;
    upper_tile(tile, p.tiles_m, a, b);
    m0 = a * BN;
    n0 = b * BM;
  } else {
    n0 = (tile / p.tiles_m) * BM;
    m0 = (tile % p.tiles_m) * BN;
  }
  const Operand Bop{p.B + mat * p.sb, p.ldb, p.N, p.K};  // the kernel's A: C^T rows
  const Operand Aop{p.A + mat * p.sa, p.lda, p.M, p.K};  // the kernel's B: C^T columns
  Acc acc;
  if constexpr (DMA)
    gemm_tile_dma<BKC, AKC>(Bop, Aop, n0, m0, ring, acc, tid);
  else
    gemm_tile<BKC, AKC>(Bop, Aop, n0, m0, s0, s0 + 2 * kStageElems, acc, tid);
  const bool mirror = SYM && m0 != n0;  // uniform over the workgroup
  // stage buffer k of the ring (constant indices only: a runtime index would
  // place the ring in a static initializer)
  auto buf = [&](int k) -> bf16* {
    return k == 0 ? ring.slot[0] : k == 1 ? ring.slot[1] : k == 2 ? ring.slot[2] : ring.slot[3];
  };
  static_assert(!SYM || DMA, "the mirrored tile is staged in the four 32 KB stage buffers");
  // every wave's last LDS reads of the k loop are done before staging
  if (mirror) __syncthreads();
  store_tile(p, mat, m0, n0, acc, tid, [&](int r, int col, const bf16x4& o) {
    // row r + u of the mirrored tile (256 columns m), 64 rows per stage buffer
    if (mirror) {
#pragma unroll
      for (int u = 0; u < 4; ++u) buf((r + u) >> 6)[((r + u) & 63) * BN + col] = o[u];
    }
  });
  bf16* C = p.C + mat * p.sc;
  if (mirror) {
    __syncthreads();
    // C[n][m] = C[m][n] for the staged rows, 16-byte pieces (M % 8 == 0)
    for (int c = tid; c < BM * BN / 8; c += kThreads) {
      const int r = c / (BN / 8), col = 8 * (c % (BN / 8));
      if (n0 + r < p.M && m0 + col < p.M)
        *reinterpret_cast<bf16x8*>(C + (int64_t)(n0 + r) * p.ldc + m0 + col) =
            *reinterpret_cast<const bf16x8*>(buf(r >> 6) + (r & 63) * BN + col);
    }
  }
}

typedef void (*BatchFn)(GemmGroups);
template <bool DMA, bool SYM> BatchFn pick_batched_as(bool akc, bool bkc) {
  if (akc)
    return bkc ? batched_gemm_kernel<true, true, DMA, SYM> : batched_gemm_kernel<true, false, DMA, SYM>;
  return bkc ? batched_gemm_kernel<false, true, DMA, SYM> : batched_gemm_kernel<false, false, DMA, SYM>;
}
BatchFn pick_batched(bool akc, bool bkc, bool dma, bool sym) {
  if (sym) return pick_batched_as<true, true>(akc, bkc);
  return dma ? pick_batched_as<true, false>(akc, bkc) : pick_batched_as<false, false>(akc, bkc);
}

// Split-K product (the weight gradients of the model's projections, K = the
// token count): C[m][n] = cast(sum_k opA(m, k) opB(n, k)) with K cut into
// `splits` chunks of Kc. Workgroup b forms chunk b / ntiles of tile
// b % ntiles (256 x 256, m along the core's M axis, so a lane's sixteen
// accumulators are sixteen rows of one column and each store instruction
// covers 32 consecutive columns of two rows) and stores it in float32 to the
// chunk's slice of the workspace; a second pass adds the slices in chunk
// order and casts (so the result does not depend on workgroup timing).
struct SplitK {
  const bf16* A;
  const bf16* B;
  float* P;  // workspace: splits x M x N float32
  int64_t lda, ldb;
  int M, N, Kc, splits, tiles_n;
};

template <bool AKC, bool BKC, bool DMA>
__global__ __launch_bounds__(kThreads) void splitk_gemm_kernel(SplitK p) {
  GEMM_LDS_STAGES;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int wm = w / NWN, wn = w % NWN;
  const int ntiles = (int)gridDim.x / p.splits;
  const int split = (int)blockIdx.x / ntiles, tile = (int)blockIdx.x % ntiles;
  const int m0 = (tile / p.tiles_n) * BM, n0 = (tile % p.tiles_n) * BN;
  const int64_t k0 = (int64_t)split * p.Kc;
  const Operand Aop{p.A + (AKC ? k0 : k0 * p.lda), p.lda, p.M, p.Kc};
  const Operand Bop{p.B + (BKC ? k0 : k0 * p.ldb), p.ldb, p.N, p.Kc};
  Acc acc;
  if constexpr (DMA)
    gemm_tile_dma<AKC, BKC>(Aop, Bop, m0, n0, ring, acc, tid);
  else
    gemm_tile<AKC, BKC>(Aop, Bop, m0, n0, s0, s0 + 2 * kStageElems, acc, tid);
  // acc.v[i][j][r] = partial C[m0 + WTM wm + 32 i + 8 (r / 4) + 4 g + r % 4][n0 + WTN wn + 32 j + c32]
  float* P = p.P + (int64_t)split * p.M * p.N;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int n = n0 + WTN * wn + 32 * j + c32;
    if (n >= p.N) continue;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + WTM * wm + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m < p.M) P[(int64_t)m * p.N + n] = acc.v[i][j][r];
      }
  }
}

// C[m][n] = cast(sum over the chunks of P[s][m][n]), four columns a thread.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ P,
                                                            bf16* __restrict__ C, int M, int N,
                                                            int64_t ldc, int splits) {
  const int64_t mn = (int64_t)M * N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
  for (int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; e < mn; e += stride) {
    f32x4 v = *reinterpret_cast<const f32x4*>(P + e);
    for (int sp = 1; sp < splits; ++sp) {
      const f32x4 u = *reinterpret_cast<const f32x4*>(P + sp * mn + e);
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] += u[c];
    }
    const int64_t m = e / N, n = e % N;
    *reinterpret_cast<bf16x4*>(C + m * ldc + n) = bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
  }
}

typedef void (*SplitFn)(SplitK);
template <bool DMA> SplitFn pick_splitk_as(bool akc, bool bkc) {
  if (akc) return bkc ? splitk_gemm_kernel<true, true, DMA> : splitk_gemm_kernel<true, false, DMA>;
  return bkc ? splitk_gemm_kernel<false, true, DMA> : splitk_gemm_kernel<false, false, DMA>;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Checks one batch's arguments and fills its descriptor (tile counts are set
// by the launch, which knows whether the symmetric schedule runs).
int32_t fill_batch(const algx_gemm_batch& b, bool a_kc, bool b_kc, bool symmetric, float alpha,
                   float beta, BatchGemm& p) {
  if (b.batch < 0 || b.M < 0 || b.N < 0 || b.K < 0) return fail("gemm_bf16_batched: negative size");
  p = BatchGemm{};
  p.batch = b.batch;
  p.M = b.M;
  p.N = b.N;
  p.K = b.K;
  if (b.batch == 0 || b.M == 0 || b.N == 0) return 0;  // nothing to form
  if (b.A == nullptr || b.B == nullptr || b.C == nullptr) return fail("gemm_bf16_batched: null pointer");
  // Every operand is moved in 16-byte chunks along its contiguous axis.
  if (b.M % 8 || b.N % 8 || b.K % 8)
    return fail("gemm_bf16_batched: M, N and K must be multiples of 8");
  const bool d = b.D != nullptr;
  if (b.lda % 8 || b.ldb % 8 || b.ldc % 8 || (d && b.ldd % 8) || b.stride_a % 8 ||
      b.stride_b % 8 || (d && b.stride_d % 8) || b.stride_c % 8)
    return fail("gemm_bf16_batched: leading dimensions and batch strides must be multiples of 8");
  if (!aligned16(b.A) || !aligned16(b.B) || !aligned16(b.C) || (d && !aligned16(b.D)))
    return fail("gemm_bf16_batched: operands must be 16-byte aligned");
  if (b.lda < (a_kc ? b.K : b.M) || b.ldb < (b_kc ? b.K : b.N) || b.ldc < b.N || (d && b.ldd < b.N))
    return fail("gemm_bf16_batched: leading dimension below the row length");
  if (b.K == 0) return fail("gemm_bf16_batched: K must be positive");
  if (symmetric && b.M != b.N) return fail("gemm_bf16_batched: a symmetric product needs M == N");
  p.A = (const bf16*)b.A;
  p.B = (const bf16*)b.B;
  p.D = (const bf16*)b.D;
  p.C = (bf16*)b.C;
  p.lda = b.lda;
  p.ldb = b.ldb;
  p.ldd = b.ldd;
  p.ldc = b.ldc;
  p.sa = b.stride_a;
  p.sb = b.stride_b;
  p.sd = b.stride_d;
  p.sc = b.stride_c;
  p.alpha = alpha;
  p.beta = beta;
  p.tiles_m = (b.M + BN - 1) / BN;  // the kernel's N tiles
  p.tiles_n = (b.N + BM - 1) / BM;  // the kernel's M tiles
  return 0;
}

// One launch over live groups of one stage kind.
int32_t launch_kind(BatchGemm* all, int live, bool a_kc, bool b_kc, bool dma, bool symmetric,
                    hipStream_t s) {
  // the triangle-only schedule of a symmetric C stages its mirrored tiles in
  // the direct-to-LDS stage buffers (without them every tile is formed)
  const bool sym = symmetric && dma;
  // Longest k loops first, so the short ones fill the launch's tail.
  for (int i = 1; i < live; ++i)
    for (int j = i; j > 0 && all[j].K > all[j - 1].K; --j) std::swap(all[j], all[j - 1]);
  GemmGroups gp{};
  int64_t start = 0;
  for (int i = 0; i < live; ++i) {
    BatchGemm& p = all[i];
    p.ntiles = sym ? p.tiles_m * (p.tiles_m + 1) / 2 : p.tiles_m * p.tiles_n;
    gp.g[i] = p;
    gp.start[i] = (int)start;
    start += ((int64_t)p.batch * p.ntiles + 7) / 8 * 8;
    if (start > 0x7fffffff) return fail("gemm_bf16_batched: too many tiles");
  }
  gp.start[live] = (int)start;
  gp.ngroups = live;
  hipLaunchKernelGGL(pick_batched(a_kc, b_kc, dma, sym), dim3((unsigned)start), dim3(kThreads),
                     0, s, gp);
  return check_launch("gemm_bf16_batched");
}

// Groups whose K is a whole number of 32-wide stages run direct-to-LDS, the
// others register-staged, as in one call per group; the two kinds go to
// separate launches so that every group takes the path its own call takes.
int32_t launch_groups(const algx_gemm_batch* groups, int ngroups, bool a_kc, bool b_kc,
                      bool symmetric, float alpha, float beta, hipStream_t s) {
  if (ngroups < 0 || ngroups > kMaxGroups)
    return fail("gemm_bf16_grouped: between 0 and 4 groups");
  if (ngroups > 0 && groups == nullptr) return fail("gemm_bf16_grouped: null group array");
  BatchGemm dma[kMaxGroups], reg[kMaxGroups];
  int nd = 0, nr = 0;
  for (int i = 0; i < ngroups; ++i) {
    BatchGemm p;
    if (int32_t rc = fill_batch(groups[i], a_kc, b_kc, symmetric, alpha, beta, p)) return rc;
    if (p.batch == 0 || p.M == 0 || p.N == 0) continue;
    // (the kernel's A is the caller's B and vice versa)
    if (p.K % BK == 0 && dma_span_ok(Operand{nullptr, p.ldb, p.N, p.K}, b_kc) &&
        dma_span_ok(Operand{nullptr, p.lda, p.M, p.K}, a_kc))
      dma[nd++] = p;
    else
      reg[nr++] = p;
  }
  if (nd > 0)
    if (int32_t rc = launch_kind(dma, nd, a_kc, b_kc, true, symmetric, s)) return rc;
  if (nr > 0)
    if (int32_t rc = launch_kind(reg, nr, a_kc, b_kc, false, symmetric, s)) return rc;
  return 0;
}

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int32_t algx_gemm_bf16_batched(const void* A, const void* B, const void* D, void* C,
                                          int32_t batch, int32_t M, int32_t N, int32_t K,
                                          int32_t a_kc, int32_t b_kc, int32_t symmetric,
                                          int64_t lda, int64_t ldb,
                                          int64_t ldd, int64_t ldc, int64_t stride_a,
                                          int64_t stride_b, int64_t stride_d, int64_t stride_c,
                                          float alpha, float beta, void* stream) {
  const algx_gemm_batch g{A, B, D, C, batch, M, N, K, lda, ldb, ldd, ldc,
                          stride_a, stride_b, stride_d, stride_c};
  return launch_groups(&g, 1, a_kc != 0, b_kc != 0, symmetric != 0, alpha, beta,
                       (hipStream_t)stream);
}

extern "C" int64_t algx_gemm_bf16_splitk_workspace_bytes(int32_t M, int32_t N,
                                                        int32_t splits) {
  if (M <= 0 || N <= 0 || splits <= 0) return 0;
  return (int64_t)splits * M * N * (int64_t)sizeof(float);
}

extern "C" int32_t algx_gemm_bf16_splitk(const void* A, const void* B, void* C, void* workspace,
                                         int32_t M, int32_t N, int32_t K, int32_t a_kc,
                                         int32_t b_kc, int64_t lda, int64_t ldb, int64_t ldc,
                                         int32_t splits, void* stream) {
  if (M < 0 || N < 0 || K < 0) return fail("gemm_bf16_splitk: negative size");
  if (splits < 1 || splits > 1024) return fail("gemm_bf16_splitk: splits must be in 1 .. 1024");
  if (M == 0 || N == 0) return 0;
  if (A == nullptr || B == nullptr || C == nullptr || workspace == nullptr)
    return fail("gemm_bf16_splitk: null pointer");
  if (K == 0 || K % splits) return fail("gemm_bf16_splitk: K must be a positive multiple of splits");
  const int Kc = K / splits;
  if (M % 8 || N % 8 || Kc % 8)
    return fail("gemm_bf16_splitk: M, N and K / splits must be multiples of 8");
  if (lda % 8 || ldb % 8 || ldc % 8)
    return fail("gemm_bf16_splitk: leading dimensions must be multiples of 8");
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || !aligned16(workspace))
    return fail("gemm_bf16_splitk: operands must be 16-byte aligned");
  if (lda < (a_kc ? K : M) || ldb < (b_kc ? K : N) || ldc < N)
    return fail("gemm_bf16_splitk: leading dimension below the row length");
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int64_t grid = (int64_t)tiles_m * tiles_n * splits;
  if (grid > 0x7fffffff) return fail("gemm_bf16_splitk: too many tiles");
  hipStream_t s = (hipStream_t)stream;
  const SplitK p{(const bf16*)A, (const bf16*)B, (float*)workspace, lda, ldb, M, N, Kc, splits,
                 tiles_n};
  const bool dma = Kc % BK == 0 && dma_span_ok(Operand{nullptr, lda, M, Kc}, a_kc != 0) &&
                   dma_span_ok(Operand{nullptr, ldb, N, Kc}, b_kc != 0);
  SplitFn fn = dma ? pick_splitk_as<true>(a_kc != 0, b_kc != 0)
                   : pick_splitk_as<false>(a_kc != 0, b_kc != 0);
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(kThreads), 0, s, p);
  if (int32_t rc = check_launch("gemm_bf16_splitk")) return rc;
  int64_t nb = ((int64_t)M * N / 4 + 255) / 256;
  if (nb > 4096) nb = 4096;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)nb), dim3(256), 0, s,
                     (const float*)workspace, (bf16*)C, M, N, (int64_t)ldc, splits);
  return check_launch("gemm_bf16_splitk_reduce");
}

extern "C" int32_t algx_gemm_bf16_grouped(const algx_gemm_batch* groups, int32_t ngroups,
                                          int32_t a_kc, int32_t b_kc, int32_t symmetric,
                                          float alpha, float beta, void* stream) {
  return launch_groups(groups, ngroups, a_kc != 0, b_kc != 0, symmetric != 0, alpha, beta,
                       (hipStream_t)stream);
}
