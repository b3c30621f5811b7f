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

#include "gemm_core.h"
#include "head_f32.h"

namespace algx {

namespace {

constexpr int kFwdWorkgroups = 256;  // forward grid target: one workgroup per CU

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
      // The target logit: one lane of one 32-row block holds it. The wave's
      // 128 rows hold a target of its 32 tokens in ~8 % of the (tile,
      // column) pairs at V = 50304, so one wave-wide vote skips the search.
      if (__any((unsigned)(tgt[j] - mw) < (unsigned)WTM)) {
#pragma unroll
        for (int i = 0; i < TI; ++i) {
          const int off = tgt[j] - (mw + 32 * i);
          if (off >= 0 && off < 32 && ((off >> 2) & 1) == g) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (8 * (r >> 2) + (r & 3) == (off & ~4)) zt[tok[j]] = acc.v[i][j][r];
          }
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
// BLK = false: dz row-major with row stride ldz. BLK: dz is stored in blocks
// of 32 vocabulary columns, [v / 32][t][32] with blocks bstride apart (the
// layout the backward's GEMMs read in whole 64-byte row pieces).
template <int KIND, int L2N, bool DMA, bool BLK>
__global__ __launch_bounds__(kThreads) void head_dz_kernel(
    const bf16* __restrict__ h, const bf16* __restrict__ e, const int32_t* __restrict__ targets,
    const float* __restrict__ stat, const float* __restrict__ scale, bf16* __restrict__ dz,
    int64_t ldz, int64_t bstride, int tok0, int ntok, int d, int V, int log2n, float inv_c,
    float clamp, int chunk_tiles) {
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
    // dz of columns mb0 + 8 q4 + 4 g .. + 3 of token column j
    // d loss / d z of one logit, y the target indicator (fused_head.py:137-145)
    auto grad = [&](float z, float y, float st) {
      if (KIND == ALGX_HEAD_CE)
        return __builtin_amdgcn_exp2f((z - st) * 1.4426950408889634f) - y;
      const float x = __builtin_fminf(z * inv_c, clamp);
      float r;
      const float p = pow_n<L2N>(rho_fast(x, r) * st, log2n);
      return (p - y) * r;
    };
    // TGT: some lane of the wave has its token's target among the rows it
    // holds for this token column, so each logit takes the indicator y; else
    // y = 0 everywhere ((p - 0) r = p r exactly, so both forms agree bitwise).
    auto run = [&](auto tgt_tag, int mb0, int i, int j, int q4, int tgt, float st) {
      constexpr bool TGT = decltype(tgt_tag)::value;
      bf16x4 out;
      const int mr = mb0 + 8 * q4 + 4 * g;  // the run's first column
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float y = TGT && mr + u == tgt ? 1.0f : 0.0f;
        out[u] = (bf16)((FULL || mr + u < V) ? grad(acc.v[i][j][4 * q4 + u], y, st) * sc : 0.0f);
      }
      return out;
    };
    auto column = [&](auto tgt_tag, int j) {
      const int tl = n0 + WTN * wn + 32 * j + c32;  // the same in lanes c32 and c32 + 32
      const int tgt = tgt_j[j];
      const float st = st_j[j];
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const int mb0 = m0 + WTM * wm + 32 * i;  // a 32-column block of dz
        if (tl >= ntok) continue;  // both lanes of a swap pair
        if constexpr (BLK) {
          // Lanes c32 and c32 + 32 hold alternate 4-column runs of one
          // token's 32 columns. Per pair of runs, two swaps between the lane
          // halves give each lane 8 consecutive columns, stored as 16 bytes:
          // columns 16 h + 8 g .. + 7 of the block.
          bf16* row = dz + (int64_t)(mb0 >> 5) * bstride + (int64_t)tl * 32 + 8 * g;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            u32x2 d0 = __builtin_bit_cast(u32x2, run(tgt_tag, mb0, i, j, 2 * h, tgt, st));
            u32x2 d1 = __builtin_bit_cast(u32x2, run(tgt_tag, mb0, i, j, 2 * h + 1, tgt, st));
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              // upper half of d0[e] <-> lower half of d1[e]
              const auto r = __builtin_amdgcn_permlane32_swap(d0[e], d1[e], false, false);
              d0[e] = r[0];
              d1[e] = r[1];
            }
            *reinterpret_cast<u32x4*>(row + 16 * h) = u32x4{d0[0], d0[1], d1[0], d1[1]};
          }
        } else {
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            *reinterpret_cast<bf16x4*>(dz + (int64_t)tl * ldz + mb0 + 8 * q4 + 4 * g) =
                run(tgt_tag, mb0, i, j, q4, tgt, st);
        }
      }
    };
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      // A wave's 128 rows hold a target of its 32 tokens in ~8 % of the
      // (tile, column) pairs at V = 50304; the test is one wave-wide vote.
      const bool hit = (unsigned)(tgt_j[j] - (m0 + WTM * wm)) < (unsigned)WTM;
      if (__any(hit))
        column(std::true_type{}, j);
      else
        column(std::false_type{}, j);
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
    gemm_seq_dma<true, true, true>(A, B, t_begin * BM, t_end - t_begin, n0, ring, acc, tid,
                                   emit_tile);
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
                         bf16*, int64_t, int64_t, int, int, int, int, int, float, float, int);

// Kernel instance for (kind, n): alg_ce with n = 8, 16 or 32 gets unrolled
// powers in both kernels, and the forward also for n = 2, 4 and 64 (its
// runtime power loop, kept for n >= 128, spills registers). DMA (the
// direct-to-LDS ring) when d is a multiple of BK.
template <bool DMA> HeadFwdFn pick_head_fwd_as(int kind, int log2n) {
  if (kind == ALGX_HEAD_CE) return head_fwd_kernel<ALGX_HEAD_CE, 0, DMA>;
  switch (log2n) {
    case 1: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 1, DMA>;
    case 2: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 2, DMA>;
    case 3: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 3, DMA>;
    case 4: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 4, DMA>;
    case 5: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 5, DMA>;
    case 6: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 6, DMA>;
    default: return head_fwd_kernel<ALGX_HEAD_ALG_CE, 0, DMA>;
  }
}
template <bool DMA, bool BLK> HeadDzFn pick_head_dz_as(int kind, int log2n) {
  if (kind == ALGX_HEAD_CE) return head_dz_kernel<ALGX_HEAD_CE, 0, DMA, BLK>;
  switch (log2n) {
    case 3: return head_dz_kernel<ALGX_HEAD_ALG_CE, 3, DMA, BLK>;
    case 4: return head_dz_kernel<ALGX_HEAD_ALG_CE, 4, DMA, BLK>;
    case 5: return head_dz_kernel<ALGX_HEAD_ALG_CE, 5, DMA, BLK>;
    default: return head_dz_kernel<ALGX_HEAD_ALG_CE, 0, DMA, BLK>;
  }
}
// The logit products run direct-to-LDS when d is a whole number of ring
// turns and E and the token rows fit the loads' 32-bit offsets.
bool logits_dma(int d, int V, int ntok) {
  return d % (BK * kDmaStages) == 0 && dma_span_ok(Operand{nullptr, d, V, d}, true) &&
         dma_span_ok(Operand{nullptr, d, ntok, d}, true);
}
HeadFwdFn pick_head_fwd(int kind, int log2n, int d, int V, int N) {
  return logits_dma(d, V, N) ? pick_head_fwd_as<true>(kind, log2n)
                             : pick_head_fwd_as<false>(kind, log2n);
}
HeadDzFn pick_head_dz(int kind, int log2n, int d, bool blocked, int V, int ntok) {
  const bool dma = logits_dma(d, V, ntok);
  if (blocked)
    return dma ? pick_head_dz_as<true, true>(kind, log2n) : pick_head_dz_as<false, true>(kind, log2n);
  return dma ? pick_head_dz_as<true, false>(kind, log2n) : pick_head_dz_as<false, false>(kind, log2n);
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
    launch_k(probe, pick_head_fwd(kind, log2n, d, V, N),
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
    // LDS-DMA stages in the dh/dE launch when both products have whole k
    // stages (V and the chunk's token count multiples of BK). dz is then
    // stored in 32-column blocks ([v / 32][t][32]): dh's 32-wide k stage
    // reads one 64-byte piece per token row, dE's reads 32 token rows of one
    // block contiguously (2 KB), instead of half lines of 100 KB rows.
    const int64_t blk = (int64_t)32 * ntok;
    const bool dma = V % BK == 0 && ntok % BK == 0 &&
                     dma_span_ok(Operand{nullptr, 32, ntok, V, blk}, true) &&
                     dma_span_ok(Operand{nullptr, 32, V, ntok, blk}, false) &&
                     dma_span_ok(Operand{nullptr, d, d, V}, false) &&
                     dma_span_ok(Operand{nullptr, d, d, ntok}, false);
    const int64_t bstride = dma ? blk : 0;
    dim3 gdz((ntok + BN - 1) / BN, ((V + BM - 1) / BM + ct - 1) / ct);
    launch_k(probe_for(ALGX_PROBE_HEAD_DZ),
             pick_head_dz(kind, log2n, d, bstride != 0, V, ntok),
             gdz, dim3(kThreads), s, hb, eb, targets, stat, scale, dz, ldz, bstride, tok0, ntok, d,
             V, log2n, inv_c, clamp, ct);
    if (int32_t rc = check_launch("head_dz")) return rc;
    // dh[t][c] = sum_v dz[t][v] E[v][c]: A = dz (k-contiguous), B(n=c,k=v) = E stored [v][c].
    // dE[v][c] (+)= sum_t dz[t][v] h[t][c]: A(m=v,k=t) = dz stored [t][v], B(n=c,k=t) = h [t][c].
    const int tn = (d + BN - 1) / BN;
    const Operand dz_t = dma ? Operand{dz, 32, ntok, V, bstride} : Operand{dz, ldz, ntok, V};
    const Operand dz_v = dma ? Operand{dz, 32, V, ntok, bstride} : Operand{dz, ldz, V, ntok};
    const GemmJob jdh{dz_t, Operand{eb, d, d, V}, (bf16*)dh + (int64_t)tok0 * d, (int64_t)d,
                      ntok, d, tn};
    const GemmJob jde{dz_v, Operand{hb + (int64_t)tok0 * d, d, d, ntok}, dE, (int64_t)d, V, d, tn};
    const int n_dh = ((ntok + BM - 1) / BM) * tn;
    const int n_de = ((V + BM - 1) / BM) * tn;
    const int dh_slots = (n_dh + 7) / 8 * 8;
    auto gk = dma ? (tok0 == 0 ? head_grad_kernel<false, true> : head_grad_kernel<true, true>)
                  : (tok0 == 0 ? head_grad_kernel<false, false> : head_grad_kernel<true, false>);
    launch_k(probe_for(ALGX_PROBE_HEAD_DE), gk, dim3(dh_slots + n_de), dim3(kThreads), s, jdh, jde,
             n_dh, dh_slots, n_de);
    if (int32_t rc = check_launch("head_grad")) return rc;
  }
  return 0;
}
