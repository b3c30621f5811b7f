// Layout changes of the model step that XLA folds into its fusions in the
// reference and torch would run as strided element copies:
//
// * swap_axes: (B, P, Q, row) -> (B, Q, P, row) with rows moved whole, as
//   16-byte vectors: the attention output's (B, H, T, D) -> (B, T, H*D) of
//   model.py:182, and its inverse for the gradient.
// * transpose: batched [K][M][N] -> [K][N][M] of 2- or 4-byte elements: the
//   swapaxes of Muon's Newton-Schulz (optimizers.py:41, :49, :58, :62). With
//   M and N multiples of the 16-byte vector (8 bf16 or 4 float32) every lane
//   transposes one square block in registers (no LDS); other shapes go
//   through a 64 x 64 LDS tile.
// * concat_cast / split_cast: float32 [rows][C_i] parts (up to 4) written as
//   one [rows][sum C_i] bf16 or float32 matrix, and the inverse for the
//   gradient: the per-step casts and concatenations of the layer-stacked
//   weights for the fused [w_q | w_k | w_v] and [w_g | w_u] GEMMs
//   (model.py:167-169, :184-189 cast each weight to the compute dtype).
//
// All are HBM-bound byte moves: every source byte is read once and every
// destination byte written once, in 128-byte (or longer) runs per wave.
#include "common.h"

namespace algx {

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;

// dst vector i = ((b * Q + q) * P + p) * vpr + c  <-  src ((b * P + p) * Q + q) * vpr + c.
__global__ __launch_bounds__(kThreads) void swap_axes_kernel(const i32x4* __restrict__ src,
                                                             i32x4* __restrict__ dst, uint32_t P,
                                                             uint32_t Q, uint32_t vpr,
                                                             uint32_t total) {
  const uint32_t i = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
  if (i >= total) return;
  const uint32_t c = i % vpr;
  uint32_t r = i / vpr;
  const uint32_t p = r % P;
  r /= P;
  const uint32_t q = r % Q, b = r / Q;
  dst[i] = src[((b * P + p) * Q + q) * vpr + c];
}

// One 64 x 64 tile of one matrix: row-contiguous reads of the source (one
// 64-element run per wave instruction) into LDS, row-contiguous writes of the
// destination read down the LDS columns (row pitch 65 elements, so the 64
// lanes of a column read fall in distinct banks).
template <typename E>
__global__ __launch_bounds__(kThreads) void transpose_kernel(const E* __restrict__ src,
                                                             E* __restrict__ dst, int M, int N,
                                                             int tiles_n) {
  __shared__ E tile[kTile][kTile + 1];
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int m0 = tm * kTile, n0 = tn * kTile;
  const int64_t base = (int64_t)blockIdx.y * M * N;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int r = w; r < kTile; r += kThreads / 64) {
    const int m = m0 + r, n = n0 + lane;
    if (m < M && n < N) tile[r][lane] = src[base + (int64_t)m * N + n];
  }
  __syncthreads();
#pragma unroll
  for (int r = w; r < kTile; r += kThreads / 64) {
    const int n = n0 + r, m = m0 + lane;
    if (n < N && m < M) dst[base + (int64_t)n * M + m] = tile[lane][r];
  }
}

// One wave per 64 x 64 (bf16) or 32 x 32 (float32) tile; lane (i, j) =
// (lane / 8, lane % 8) owns the square block of V x V elements (V = 16 bytes /
// element size) at rows V i, columns V j of the tile: V 16-byte row loads,
// the block transposed in registers, V 16-byte row stores. Each load or store
// instruction moves 8 runs of 128 contiguous bytes.
template <int V>
__global__ __launch_bounds__(kThreads) void transpose_block_kernel(const i32x4* __restrict__ src,
                                                                   i32x4* __restrict__ dst,
                                                                   int M, int N, int tiles_n,
                                                                   int tiles) {
  constexpr int T = 8 * V;  // tile edge in elements
  const int lane = threadIdx.x & 63;
  const int tile = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (tile >= tiles) return;
  const int m0 = (tile / tiles_n) * T + V * (lane >> 3);
  const int n0 = (tile % tiles_n) * T + V * (lane & 7);
  if (m0 >= M || n0 >= N) return;
  // In 16-byte vectors: a row of the source holds N / V, of the destination M / V.
  const int64_t base = (int64_t)blockIdx.y * M * (N / V);
  const int64_t nv = N / V, mv = M / V;
  i32x4 in[V];
#pragma unroll
  for (int r = 0; r < V; ++r) in[r] = src[base + (int64_t)(m0 + r) * nv + n0 / V];
  i32x4 out[V];
  if (V == 8) {
    // bf16: out row c, word k = (element c of row 2k) | (element c of row 2k+1) << 16.
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t a = (uint32_t)in[2 * k][c >> 1], b = (uint32_t)in[2 * k + 1][c >> 1];
        out[c][k] = (int)((c & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16)));
      }
  } else {
#pragma unroll
    for (int c = 0; c < V; ++c)
#pragma unroll
      for (int k = 0; k < V; ++k) out[c][k] = in[k][c];
  }
#pragma unroll
  for (int c = 0; c < V; ++c) dst[base + (int64_t)(n0 + c) * mv + m0 / V] = out[c];
}

constexpr int kMaxParts = 4;

struct Parts {
  void* p[kMaxParts];   // float32 parts
  int64_t c[kMaxParts];  // columns of each part (multiples of 4)
  int64_t off[kMaxParts + 1];  // column offset of each part in the joined matrix
  int n;
};

// One 4-column group of the joined matrix per thread: the group lies inside
// one part (its columns are multiples of 4). TO_JOINED: parts -> joined
// (float32 read, T written); otherwise joined -> parts (T read, float32 written).
template <typename T, bool TO_JOINED>
__global__ __launch_bounds__(kThreads) void concat_cast_kernel(Parts parts, T* __restrict__ joined,
                                                               int64_t rows) {
  const int64_t w = parts.off[parts.n];
  const int64_t groups = w / 4;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= rows * groups) return;
  const int64_t r = i / groups, col = (i % groups) * 4;
  int q = 0;
#pragma unroll
  for (int t = 1; t < kMaxParts; ++t) q += (t < parts.n && col >= parts.off[t]) ? 1 : 0;
  float* part = (float*)parts.p[q] + r * parts.c[q] + (col - parts.off[q]);
  T* jp = joined + r * w + col;
  if (TO_JOINED) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(part);
    if (sizeof(T) == 2) {
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (bf16)v[e];
      *reinterpret_cast<bf16x4*>(jp) = o;
    } else {
      *reinterpret_cast<f32x4*>(jp) = v;
    }
  } else {
    f32x4 v;
    if (sizeof(T) == 2) {
      const bf16x4 b = *reinterpret_cast<const bf16x4*>(jp);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (float)b[e];
    } else {
      v = *reinterpret_cast<const f32x4*>(jp);
    }
    *reinterpret_cast<f32x4*>(part) = v;
  }
}

int32_t concat_cast_any(void* const* parts, const int64_t* cols, int32_t nparts, void* joined,
                        int64_t rows, int32_t dtype, bool to_joined, void* stream) {
  const char* what = to_joined ? "concat_cast" : "split_cast";
  if (nparts < 1 || nparts > kMaxParts) return fail(std::string(what) + ": 1 to 4 parts");
  if (rows < 0) return fail(std::string(what) + ": negative row count");
  if (dtype != ALGX_BF16 && dtype != ALGX_F32) return fail(std::string(what) + ": dtype must be bf16 or f32");
  Parts ps{};
  ps.n = nparts;
  ps.off[0] = 0;
  for (int i = 0; i < nparts; ++i) {
    if (cols[i] <= 0 || cols[i] % 4) return fail(std::string(what) + ": part widths must be positive multiples of 4");
    ps.p[i] = parts[i];
    ps.c[i] = cols[i];
    ps.off[i + 1] = ps.off[i] + cols[i];
  }
  const int64_t total = rows * (ps.off[nparts] / 4);
  if (total == 0) return 0;
  if (joined == nullptr || ((uintptr_t)joined & (dtype == ALGX_BF16 ? 7 : 15)))
    return fail(std::string(what) + ": joined matrix null or misaligned");
  for (int i = 0; i < nparts; ++i)
    if (parts[i] == nullptr || !((((uintptr_t)parts[i]) & 15) == 0))
      return fail(std::string(what) + ": parts must be 16-byte aligned float32");
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks >= ((int64_t)1 << 31)) return fail(std::string(what) + ": too many elements");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ALGX_BF16) {
    if (to_joined)
      hipLaunchKernelGGL((concat_cast_kernel<bf16, true>), dim3((uint32_t)blocks), dim3(kThreads),
                         0, s, ps, (bf16*)joined, rows);
    else
      hipLaunchKernelGGL((concat_cast_kernel<bf16, false>), dim3((uint32_t)blocks), dim3(kThreads),
                         0, s, ps, (bf16*)joined, rows);
  } else {
    if (to_joined)
      hipLaunchKernelGGL((concat_cast_kernel<float, true>), dim3((uint32_t)blocks),
                         dim3(kThreads), 0, s, ps, (float*)joined, rows);
    else
      hipLaunchKernelGGL((concat_cast_kernel<float, false>), dim3((uint32_t)blocks),
                         dim3(kThreads), 0, s, ps, (float*)joined, rows);
  }
  return check_launch(what);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool overlaps(const void* a, const void* b, int64_t bytes) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + (uintptr_t)bytes && y < x + (uintptr_t)bytes;
}

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int32_t algx_swap_axes(const void* src, void* dst, int64_t B, int64_t P, int64_t Q,
                                  int64_t row_bytes, void* stream) {
  if (B < 0 || P < 0 || Q < 0) return fail("swap_axes: negative extent");
  if (row_bytes <= 0 || row_bytes % 16) return fail("swap_axes: row_bytes must be a positive multiple of 16");
  const int64_t vpr = row_bytes / 16;
  const int64_t total = B * P * Q * vpr;
  if (total == 0) return 0;
  if (total >= ((int64_t)1 << 32) - kThreads) return fail("swap_axes: more than 2^32 16-byte vectors");
  if (src == nullptr || dst == nullptr) return fail("swap_axes: null pointer");
  if (!aligned16(src) || !aligned16(dst)) return fail("swap_axes: pointers must be 16-byte aligned");
  if (overlaps(src, dst, total * 16)) return fail("swap_axes: source and destination overlap");
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(swap_axes_kernel, dim3((uint32_t)blocks), dim3(kThreads), 0,
                     (hipStream_t)stream, (const i32x4*)src, (i32x4*)dst, (uint32_t)P,
                     (uint32_t)Q, (uint32_t)vpr, (uint32_t)total);
  return check_launch("swap_axes");
}

extern "C" int32_t algx_transpose(const void* src, void* dst, int64_t K, int64_t M, int64_t N,
                                  int32_t elem_bytes, void* stream) {
  if (K < 0 || M < 0 || N < 0) return fail("transpose: negative extent");
  if (elem_bytes != 2 && elem_bytes != 4) return fail("transpose: elem_bytes must be 2 or 4");
  if (K == 0 || M == 0 || N == 0) return 0;
  if (K > 65535) return fail("transpose: at most 65535 matrices");
  if (M >= ((int64_t)1 << 31) || N >= ((int64_t)1 << 31)) return fail("transpose: extent too large");
  const int64_t tiles_n = (N + kTile - 1) / kTile;
  const int64_t tiles = (M + kTile - 1) / kTile * tiles_n;
  if (tiles >= ((int64_t)1 << 31)) return fail("transpose: too many tiles");
  if (src == nullptr || dst == nullptr) return fail("transpose: null pointer");
  if (overlaps(src, dst, K * M * N * elem_bytes)) return fail("transpose: source and destination overlap");
  hipStream_t s = (hipStream_t)stream;
  const int V = 16 / elem_bytes;
  const int64_t bt_n = (N + 8 * V - 1) / (8 * V);
  const int64_t bt = (M + 8 * V - 1) / (8 * V) * bt_n;
  if (M % V == 0 && N % V == 0 && aligned16(src) && aligned16(dst) && bt < ((int64_t)1 << 31)) {
    const dim3 bgrid((uint32_t)((bt + kThreads / 64 - 1) / (kThreads / 64)), (uint32_t)K);
    if (V == 8)
      hipLaunchKernelGGL(transpose_block_kernel<8>, bgrid, dim3(kThreads), 0, s,
                         (const i32x4*)src, (i32x4*)dst, (int)M, (int)N, (int)bt_n, (int)bt);
    else
      hipLaunchKernelGGL(transpose_block_kernel<4>, bgrid, dim3(kThreads), 0, s,
                         (const i32x4*)src, (i32x4*)dst, (int)M, (int)N, (int)bt_n, (int)bt);
    return check_launch("transpose");
  }
  const dim3 grid((uint32_t)tiles, (uint32_t)K);
  if (elem_bytes == 2)
    hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, dim3(kThreads), 0, s,
                       (const uint16_t*)src, (uint16_t*)dst, (int)M, (int)N, (int)tiles_n);
  else
    hipLaunchKernelGGL(transpose_kernel<uint32_t>, grid, dim3(kThreads), 0, s,
                       (const uint32_t*)src, (uint32_t*)dst, (int)M, (int)N, (int)tiles_n);
  return check_launch("transpose");
}

extern "C" int32_t algx_concat_cast(void* const* parts, const int64_t* cols, int32_t nparts,
                                   void* joined, int64_t rows, int32_t dtype, void* stream) {
  return concat_cast_any(parts, cols, nparts, joined, rows, dtype, true, stream);
}

extern "C" int32_t algx_split_cast(const void* joined, void* const* parts, const int64_t* cols,
                                  int32_t nparts, int64_t rows, int32_t dtype, void* stream) {
  return concat_cast_any(parts, cols, nparts, (void*)joined, rows, dtype, false, stream);
}
