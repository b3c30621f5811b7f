// Batched bf16 GEMM with a fused linear combination, on the MFMA GEMM core:
//   C[b] = alpha * opA(A[b]) opB(B[b])^T + beta * D[b]
// with opA(m, k) = A[m*lda + k] (k-contiguous) or A[k*lda + m], opB(n, k)
// likewise. It carries Muon's Newton-Schulz products (optimizers.py:27-65):
// the Gram matrix X X^T (both operands k-contiguous, so no transpose is
// formed), b A + c A A and a X + B X (the second operand [k][n], read through
// transposing LDS reads), each written to its own buffer with the
// combination in the epilogue.
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
// Each run's bf16 values also go to mirror(r, col, value4) when given.
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
    if (m >= p.M) continue;
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
          const bf16x4 d = *reinterpret_cast<const bf16x4*>(D + (int64_t)m * p.ldd + n);
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = __builtin_fmaf(p.beta, (float)d[u], v[u]);
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
__global__ __launch_bounds__(kThreads) void batched_gemm_kernel(BatchGemm p) {
  GEMM_LDS_STAGES;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int wm = w / NWN, wn = w % NWN;
  int mat, tile;
  batch_tile(blockIdx.x, p, mat, tile);
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

typedef void (*BatchFn)(BatchGemm);
template <bool DMA, bool SYM> BatchFn pick_batched_as(bool akc, bool bkc) {
  if (akc)
    return bkc ? batched_gemm_kernel<true, true, DMA, SYM> : batched_gemm_kernel<true, false, DMA, SYM>;
  return bkc ? batched_gemm_kernel<false, true, DMA, SYM> : batched_gemm_kernel<false, false, DMA, SYM>;
}
BatchFn pick_batched(bool akc, bool bkc, bool dma, bool sym) {
  if (sym) return pick_batched_as<true, true>(akc, bkc);
  return dma ? pick_batched_as<true, false>(akc, bkc) : pick_batched_as<false, false>(akc, bkc);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

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
  if (batch < 0 || M < 0 || N < 0 || K < 0) return fail("gemm_bf16_batched: negative size");
  if (batch == 0 || M == 0 || N == 0) return 0;
  if (A == nullptr || B == nullptr || C == nullptr) return fail("gemm_bf16_batched: null pointer");
  // Every operand is moved in 16-byte chunks along its contiguous axis.
  if (M % 8 || N % 8 || K % 8) return fail("gemm_bf16_batched: M, N and K must be multiples of 8");
  if (lda % 8 || ldb % 8 || ldc % 8 || (D != nullptr && ldd % 8) || stride_a % 8 ||
      stride_b % 8 || (D != nullptr && stride_d % 8) || stride_c % 8)
    return fail("gemm_bf16_batched: leading dimensions and batch strides must be multiples of 8");
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || (D != nullptr && !aligned16(D)))
    return fail("gemm_bf16_batched: operands must be 16-byte aligned");
  if (lda < (a_kc ? K : M) || ldb < (b_kc ? K : N) || ldc < N || (D != nullptr && ldd < N))
    return fail("gemm_bf16_batched: leading dimension below the row length");
  if (K == 0) return fail("gemm_bf16_batched: K must be positive");
  BatchGemm p;
  p.A = (const bf16*)A;
  p.B = (const bf16*)B;
  p.D = (const bf16*)D;
  p.C = (bf16*)C;
  p.lda = lda;
  p.ldb = ldb;
  p.ldd = ldd;
  p.ldc = ldc;
  p.sa = stride_a;
  p.sb = stride_b;
  p.sd = stride_d;
  p.sc = stride_c;
  p.M = M;
  p.N = N;
  p.K = K;
  p.alpha = alpha;
  p.beta = beta;
  p.tiles_m = (M + BN - 1) / BN;  // the kernel's N tiles
  p.tiles_n = (N + BM - 1) / BM;  // the kernel's M tiles
  p.batch = batch;
  if (symmetric && M != N) return fail("gemm_bf16_batched: a symmetric product needs M == N");
  // Direct-to-LDS stages when K is a whole number of 32-wide stages; the
  // triangle-only schedule of a symmetric C stages its mirrored tiles in
  // their buffers (without them every tile is formed).
  const bool dma = K % BK == 0;
  const bool sym = symmetric && dma;
  p.ntiles = sym ? p.tiles_m * (p.tiles_m + 1) / 2 : p.tiles_m * p.tiles_n;
  const int64_t ntot = (int64_t)batch * p.ntiles;
  if (ntot > 0x7fffffff) return fail("gemm_bf16_batched: too many tiles");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(pick_batched(a_kc != 0, b_kc != 0, dma, sym), dim3((unsigned)ntot),
                     dim3(kThreads), 0, s, p);
  return check_launch("gemm_bf16_batched");
}
