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
};

// Workgroup b -> (matrix, tile). Workgroups are dealt to the 8 XCDs
// round-robin by index; when the batch is a multiple of 8, matrix j's tiles
// go to indices congruent to j mod 8, i.e. all to one XCD and its L2, in
// consecutive order there.
__device__ __forceinline__ void batch_tile(int b, const BatchGemm& p, int& mat, int& tile) {
  const int T = p.tiles_m * p.tiles_n;
  if (p.batch % 8 == 0) {
    const int x = b & 7, r = b >> 3;  // XCD, index within it
    mat = (r / T) * 8 + x;
    tile = r % T;
  } else {
    mat = b / T;
    tile = b % T;
  }
}

// Each workgroup forms a 256 x 256 tile of C^T (the kernel's M axis runs
// over C's columns n, its N axis over C's rows m), so every lane holds runs
// of four consecutive columns of one row: C and D move in 8-byte pieces.
template <bool AKC, bool BKC, bool DMA>
__global__ __launch_bounds__(kThreads) void batched_gemm_kernel(BatchGemm p) {
  GEMM_LDS_STAGES;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int wm = w / NWN, wn = w % NWN;
  int mat, tile;
  batch_tile(blockIdx.x, p, mat, tile);
  const int n0 = (tile / p.tiles_m) * BM, m0 = (tile % p.tiles_m) * BN;
  const Operand Bop{p.B + mat * p.sb, p.ldb, p.N, p.K};  // the kernel's A: C^T rows
  const Operand Aop{p.A + mat * p.sa, p.lda, p.M, p.K};  // the kernel's B: C^T columns
  Acc acc;
  if constexpr (DMA)
    gemm_tile_dma<BKC, AKC>(Bop, Aop, n0, m0, ring, acc, tid);
  else
    gemm_tile<BKC, AKC>(Bop, Aop, n0, m0, s0, s0 + 2 * kStageElems, acc, tid);
  bf16* C = p.C + mat * p.sc;
  const bf16* D = p.D != nullptr ? p.D + mat * p.sd : nullptr;
  // acc.v[i][j][4q + u] = C[m][n + u], m = m0 + WTN wn + 32 j + c32,
  // n = n0 + WTM wm + 32 i + 8 q + 4 g (N % 8 == 0: a run is whole or absent).
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
        *reinterpret_cast<bf16x4*>(C + (int64_t)m * p.ldc + n) =
            bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
      }
  }
}

typedef void (*BatchFn)(BatchGemm);

BatchFn pick_batched(bool akc, bool bkc, bool dma) {
  if (dma) {
    if (akc) return bkc ? batched_gemm_kernel<true, true, true> : batched_gemm_kernel<true, false, true>;
    return bkc ? batched_gemm_kernel<false, true, true> : batched_gemm_kernel<false, false, true>;
  }
  if (akc) return bkc ? batched_gemm_kernel<true, true, false> : batched_gemm_kernel<true, false, false>;
  return bkc ? batched_gemm_kernel<false, true, false> : batched_gemm_kernel<false, false, false>;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int32_t algx_gemm_bf16_batched(const void* A, const void* B, const void* D, void* C,
                                          int32_t batch, int32_t M, int32_t N, int32_t K,
                                          int32_t a_kc, int32_t b_kc, int64_t lda, int64_t ldb,
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
  const int64_t nwg = (int64_t)batch * p.tiles_m * p.tiles_n;
  if (nwg > 0x7fffffff) return fail("gemm_bf16_batched: too many tiles");
  // Direct-to-LDS stages when K is a whole number of 32-wide stages.
  const bool dma = K % BK == 0;
  hipLaunchKernelGGL(pick_batched(a_kc != 0, b_kc != 0, dma), dim3((unsigned)nwg), dim3(kThreads),
                     0, (hipStream_t)stream, p);
  return check_launch("gemm_bf16_batched");
}
