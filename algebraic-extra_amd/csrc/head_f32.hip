// Fused head for float32 hidden states (fused_head.py:160-216 with h.dtype =
// float32: the embedding is cast to float32, the logits, their gradient dz and
// the products dh = dz E, dE = dz^T h are all float32).
//
// This is the parity path of float32 models, not a benchmarked one: 64 x 64
// output tiles of 256 threads, each thread 4 x 4 outputs by scalar FMA, with
// 16-wide k stages staged in LDS as [k][mn] so that a thread's four operands
// of a k step sit in four banks. Thread t owns rows (t % 16) + 16 i and
// columns (t / 16) + 16 j of its tile, i, j = 0..3.
//
// Forward: grid (token tiles, vocabulary chunks of kF32ChunkTiles tiles);
// per-token online statistics merged inside the 16-lane groups sharing a
// token and written as (chunk, token) partials for head_f32_stat_kernel.
// Backward: the logit gradient dz (float32, [tokens][V rounded up to 64]) of a
// token chunk, then the two products by one generic float32 GEMM kernel.
#include "head_f32.h"

namespace algx {
namespace {

constexpr int FT = 64;                  // tile extent along m and n
constexpr int FK = 16;                  // k stage
constexpr int FTHR = 256;
constexpr int kF32ChunkTiles = 8;       // vocabulary tiles per forward workgroup
constexpr float kLog2eF = 1.4426950408889634f;

// C-tile operand: element (mn, k) at p[mn * s_mn + k * s_k], valid for
// mn < rows and k < K.
struct F32Op {
  const float* p;
  int64_t s_mn, s_k;
  int rows, K;
};

// One 64 x 16 stage of an operand into LDS as [k][mn]: 4 elements per thread.
__device__ __forceinline__ void stage_f32(const F32Op& op, int mn0, int k0, float (*dst)[FT + 4],
                                          int tid) {
#pragma unroll
  for (int e = 0; e < FT * FK / FTHR; ++e) {
    const int id = tid + FTHR * e;
    // k-contiguous operands read along k first (coalesced along k), others
    // along mn.
    int mn, k;
    if (op.s_k == 1) {
      mn = id / FK;
      k = id % FK;
    } else {
      k = id / FT;
      mn = id % FT;
    }
    const int gm = mn0 + mn, gk = k0 + k;
    dst[k][mn] = (gm < op.rows && gk < op.K) ? op.p[(int64_t)gm * op.s_mn + (int64_t)gk * op.s_k]
                                             : 0.0f;
  }
}

// acc[i][j] = sum_k A(m0 + tm + 16i, k) B(n0 + tn + 16j, k).
__device__ __forceinline__ void tile_f32(const F32Op& A, const F32Op& B, int m0, int n0,
                                         float (*As)[FT + 4], float (*Bs)[FT + 4],
                                         float (&acc)[4][4], int tid) {
  const int tm = tid & 15, tn = tid >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  for (int k0 = 0; k0 < A.K; k0 += FK) {
    __syncthreads();  // the previous stage is no longer read
    stage_f32(A, m0, k0, As, tid);
    stage_f32(B, n0, k0, Bs, tid);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < FK; ++k) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[k][tm + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[k][tn + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
  }
}

__device__ __forceinline__ float rho_fast_f(float x, float& r) {
  const float rad = __builtin_fmaf(x, x, 1.0f);
  r = rsq(rad);
  return __builtin_fmaf(rad, r, x);
}

// Forward statistics over one vocabulary chunk (fused_head.py:72-117).
// partial[(chunk * N + token) * 2 + {0, 1}] = (m, l) for ce, (0, l) for alg_ce.
template <int KIND>
__global__ __launch_bounds__(FTHR) void head_f32_fwd_kernel(
    const float* __restrict__ h, const float* __restrict__ e, const int32_t* __restrict__ targets,
    float* __restrict__ zt, float* __restrict__ partial, int N, int d, int V, int log2n,
    float inv_c, float clamp) {
  __shared__ float As[FK][FT + 4], Bs[FK][FT + 4];
  const int tid = threadIdx.x, tm = tid & 15, tn = tid >> 4;
  const int n0 = blockIdx.x * FT, chunk = blockIdx.y;
  const int ntv = (V + FT - 1) / FT;
  const int t_begin = chunk * kF32ChunkTiles;
  const int t_end = min(ntv, t_begin + kF32ChunkTiles);
  const F32Op A{e, d, 1, V, d}, B{h, d, 1, N, d};
  float m_st[4], l_st[4];
  int tgt[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tok = n0 + tn + 16 * j;
    tgt[j] = tok < N ? targets[tok] : -1;
    m_st[j] = -1e30f;
    l_st[j] = 0.0f;
  }
  float acc[4][4];
  for (int t = t_begin; t < t_end; ++t) {
    const int m0 = t * FT;
    tile_f32(A, B, m0, n0, As, Bs, acc, tid);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tok = n0 + tn + 16 * j;
      float tmax = -1e30f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + tm + 16 * i;
        if (m < V) {
          if (m == tgt[j] && tok < N) zt[tok] = acc[i][j];
          if (KIND == ALGX_HEAD_CE) tmax = __builtin_fmaxf(tmax, acc[i][j]);
        }
      }
      const float m_new = __builtin_fmaxf(m_st[j], tmax);
      float lsum = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + tm + 16 * i;
        float w;
        if (KIND == ALGX_HEAD_CE) {
          w = __builtin_amdgcn_exp2f((acc[i][j] - m_new) * kLog2eF);
        } else {
          float r;
          w = pow2n(rho_fast_f(__builtin_fminf(acc[i][j] * inv_c, clamp), r), log2n);
        }
        lsum += m < V ? w : 0.0f;
      }
      if (KIND == ALGX_HEAD_CE) {
        l_st[j] = l_st[j] * __builtin_amdgcn_exp2f((m_st[j] - m_new) * kLog2eF) + lsum;
        m_st[j] = m_new;
      } else {
        l_st[j] += lsum;
      }
    }
  }
  // Merge the 16 lanes that share a token (tm = lane % 16).
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int msk = 1; msk < 16; msk <<= 1) {
      const float mo = __shfl_xor(m_st[j], msk, 64), lo = __shfl_xor(l_st[j], msk, 64);
      if (KIND == ALGX_HEAD_CE) {
        const float mm = __builtin_fmaxf(m_st[j], mo);
        l_st[j] = l_st[j] * __builtin_amdgcn_exp2f((m_st[j] - mm) * kLog2eF) +
                  lo * __builtin_amdgcn_exp2f((mo - mm) * kLog2eF);
        m_st[j] = mm;
      } else {
        l_st[j] += lo;
      }
    }
    const int tok = n0 + tn + 16 * j;
    if (tm == 0 && tok < N) {
      partial[((int64_t)chunk * N + tok) * 2 + 0] = KIND == ALGX_HEAD_CE ? m_st[j] : 0.0f;
      partial[((int64_t)chunk * N + tok) * 2 + 1] = l_st[j];
    }
  }
}

// stat = m + log l (ce) or l^(-1/n) (alg_ce) from the chunk partials.
template <int KIND>
__global__ __launch_bounds__(256) void head_f32_stat_kernel(const float* __restrict__ partial,
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

// dz[t][v] = f(z) * scale for the tokens [tok0, tok0 + ntok), 0 for v >= V
// (fused_head.py:127-145 with dz in float32).
template <int KIND>
__global__ __launch_bounds__(FTHR) void head_f32_dz_kernel(
    const float* __restrict__ h, const float* __restrict__ e, const int32_t* __restrict__ targets,
    const float* __restrict__ stat, const float* __restrict__ scale, float* __restrict__ dz,
    int64_t ldz, int tok0, int ntok, int d, int V, int log2n, float inv_c, float clamp) {
  __shared__ float As[FK][FT + 4], Bs[FK][FT + 4];
  const int tid = threadIdx.x, tm = tid & 15, tn = tid >> 4;
  const int n0 = blockIdx.x * FT, m0 = blockIdx.y * FT;
  const F32Op A{e, d, 1, V, d}, B{h + (int64_t)tok0 * d, d, 1, ntok, d};
  float acc[4][4];
  tile_f32(A, B, m0, n0, As, Bs, acc, tid);
  const float sc = scale[0];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tl = n0 + tn + 16 * j;
    if (tl >= ntok) continue;
    const int tgt = targets[tok0 + tl];
    const float st = stat[tok0 + tl];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + tm + 16 * i;
      const float z = acc[i][j];
      const float y = m == tgt ? 1.0f : 0.0f;
      float g;
      if (KIND == ALGX_HEAD_CE) {
        g = __builtin_amdgcn_exp2f((z - st) * kLog2eF) - y;
      } else {
        float r;
        const float p = pow2n(rho_fast_f(__builtin_fminf(z * inv_c, clamp), r) * st, log2n);
        g = (p - y) * r;
      }
      dz[(int64_t)tl * ldz + m] = m < V ? g * sc : 0.0f;
    }
  }
}

// C[m][n] (+)= sum_k A(m, k) B(n, k), C row-major with leading dimension ldc.
__global__ __launch_bounds__(FTHR) void gemm_f32_kernel(F32Op A, F32Op B, float* __restrict__ C,
                                                        int64_t ldc, int accumulate) {
  __shared__ float As[FK][FT + 4], Bs[FK][FT + 4];
  const int tid = threadIdx.x, tm = tid & 15, tn = tid >> 4;
  const int m0 = blockIdx.y * FT, n0 = blockIdx.x * FT;
  float acc[4][4];
  tile_f32(A, B, m0, n0, As, Bs, acc, tid);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + tm + 16 * i;
    if (m >= A.rows) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tn + 16 * j;
      if (n >= B.rows) continue;
      float* dst = C + (int64_t)m * ldc + n;
      *dst = accumulate ? *dst + acc[i][j] : acc[i][j];
    }
  }
}

int nchunks_f32(int V) {
  const int nt = (V + FT - 1) / FT;
  return (nt + kF32ChunkTiles - 1) / kF32ChunkTiles;
}

int64_t vpad_f32(int V) { return ((int64_t)V + FT - 1) / FT * FT; }

int32_t launch_gemm_f32(const F32Op& A, const F32Op& B, float* C, int64_t ldc, bool accumulate,
                        hipStream_t s) {
  if (A.rows == 0 || B.rows == 0) return 0;
  dim3 grid((B.rows + FT - 1) / FT, (A.rows + FT - 1) / FT);
  gemm_f32_kernel<<<grid, FTHR, 0, s>>>(A, B, C, ldc, accumulate ? 1 : 0);
  return check_launch("head_f32_gemm");
}

}  // namespace

int64_t head_f32_fwd_workspace(int N, int V) { return (int64_t)nchunks_f32(V) * N * 2 * 4; }

int32_t head_f32_fwd(const float* h, const float* E, const int32_t* targets, float* stat,
                     float* zt, float* partial, int N, int d, int V, int kind, int log2n,
                     float inv_c, float clamp, hipStream_t s) {
  const int nch = nchunks_f32(V);
  dim3 grid((N + FT - 1) / FT, nch);
  if (kind == ALGX_HEAD_CE)
    head_f32_fwd_kernel<ALGX_HEAD_CE><<<grid, FTHR, 0, s>>>(h, E, targets, zt, partial, N, d, V,
                                                            log2n, inv_c, clamp);
  else
    head_f32_fwd_kernel<ALGX_HEAD_ALG_CE><<<grid, FTHR, 0, s>>>(h, E, targets, zt, partial, N, d,
                                                                V, log2n, inv_c, clamp);
  if (int32_t rc = check_launch("head_f32_fwd")) return rc;
  const int nb = (N + 255) / 256;
  if (kind == ALGX_HEAD_CE)
    head_f32_stat_kernel<ALGX_HEAD_CE><<<nb, 256, 0, s>>>(partial, nch, N, log2n, stat);
  else
    head_f32_stat_kernel<ALGX_HEAD_ALG_CE><<<nb, 256, 0, s>>>(partial, nch, N, log2n, stat);
  return check_launch("head_f32_stat");
}

// Tokens per backward chunk: the float32 dz scratch is capped at 2 GiB.
int head_f32_chunk_tokens(int N, int V) {
  const int64_t per_tok = vpad_f32(V) * 4;
  int64_t c = ((int64_t)2 << 30) / per_tok;
  c = c / FT * FT;
  if (c < FT) c = FT;
  return (int)(c > N ? N : c);
}

int64_t head_f32_bwd_workspace(int N, int V) {
  return (int64_t)head_f32_chunk_tokens(N, V) * vpad_f32(V) * 4;
}

int32_t head_f32_bwd(const float* h, const float* E, const int32_t* targets, const float* stat,
                     const float* scale, float* dh, float* dE, float* dz, int N, int d, int V,
                     int kind, int log2n, float inv_c, float clamp, hipStream_t s) {
  const int64_t ldz = vpad_f32(V);
  const int csize = head_f32_chunk_tokens(N, V);
  for (int tok0 = 0; tok0 < N; tok0 += csize) {
    const int ntok = min(csize, N - tok0);
    dim3 gdz((ntok + FT - 1) / FT, (V + FT - 1) / FT);
    if (kind == ALGX_HEAD_CE)
      head_f32_dz_kernel<ALGX_HEAD_CE><<<gdz, FTHR, 0, s>>>(h, E, targets, stat, scale, dz, ldz,
                                                            tok0, ntok, d, V, log2n, inv_c, clamp);
    else
      head_f32_dz_kernel<ALGX_HEAD_ALG_CE><<<gdz, FTHR, 0, s>>>(h, E, targets, stat, scale, dz,
                                                                ldz, tok0, ntok, d, V, log2n,
                                                                inv_c, clamp);
    if (int32_t rc = check_launch("head_f32_dz")) return rc;
    // dh[t][c] = sum_v dz[t][v] E[v][c]: A(m = t, k = v), B(n = c, k = v) = E[v][c].
    const F32Op adh{dz, ldz, 1, ntok, V}, bdh{E, 1, d, d, V};
    if (int32_t rc = launch_gemm_f32(adh, bdh, dh + (int64_t)tok0 * d, d, false, s)) return rc;
    // dE[v][c] (+)= sum_t dz[t][v] h[t][c]: A(m = v, k = t), B(n = c, k = t) = h[t][c].
    const F32Op ade{dz, 1, ldz, V, ntok}, bde{h + (int64_t)tok0 * d, 1, d, d, ntok};
    if (int32_t rc = launch_gemm_f32(ade, bde, dE, d, tok0 > 0, s)) return rc;
  }
  return 0;
}

}  // namespace algx
