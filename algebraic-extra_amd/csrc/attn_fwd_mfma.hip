// gfx950 MFMA attention forward (flash.py:189-284, head_resident.py:24-93).
//
// One workgroup of 4 waves owns 128 queries of one (b, h); each wave owns 32
// of them and walks 64-key tiles up to the diagonal. The score tile is formed
// transposed, S^T = K Q_s^T, with v_mfma_f32_32x32x16_bf16 (K from LDS as the
// A operand, the wave's scaled Q rows in registers as the B operand), so each
// lane holds 16 keys of ONE query row. The asinh/softmax weight, the causal
// mask and the row sum run on those registers; the bf16 weights go straight
// back as the B operand of O^T += V^T P^T, whose A operand is a V^T tile in
// LDS read through transposing LDS reads in the k-slot order the accumulator
// layout implies.
//
// Occupancy rather than software pipelining: each wave forms a tile's
// scores, weights and PV products in order, in at most 128 VGPRs, so four
// workgroups (32 KB of LDS each) run per CU and four waves per SIMD cover each
// other's MFMA, LDS and barrier waits while the VALU (the bound of this
// kernel: about eight VALU operations and one reciprocal square root per score
// against 256 MFMA flops) works. K and V tiles share a two-slot LDS ring:
// step j reads slot j % 2, and after the step's barrier the slot takes
// K_{j+2} and V_{j+2}.
#include <type_traits>

#include "attn_mfma.h"

namespace algx {
namespace mfma {
namespace {

template <int MODE, bool FAST, bool BOUNDED, int L2N, bool POLY, bool EARLY_QS>
__device__ __forceinline__ void fwd_body(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ sink, bf16* __restrict__ o, float* __restrict__ o_precise,
    float* __restrict__ stat, int H, int T_, const KVariant& var, const FwdPrep& prep,
    bf16 (*Kr)[FBN * HD], bf16 (*Vr)[FBN * HD], float (*red)[4], int bid, int nblocks) {
  const int nheads = nblocks / (T_ / FBM);
  int bh, qb;
  map_block(bid, nheads, T_ / FBM, true, bh, qb);
  const int h = bh % H;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
  const int G = lane >> 4, j4 = (lane >> 2) & 3, m4 = lane & 3;
  const int64_t base = (int64_t)bh * T_ * HD;
  const int q0 = qb * FBM, qw = q0 + 32 * w, qrow = qw + c32;
  const int log2n = var.log2n;

  // K and V tiles move straight from global memory into two-slot LDS rings
  // (tile t in slot t % 2), unpadded rows with chunk c of row r at chunk
  // c ^ sw16(r). Each wave issues two 1 KB blocks of each tile (rows 16w ..
  // 16w + 15): lane i of block b fills row 8b + i / 8, physical chunk i % 8,
  // so it reads logical chunk (i % 8) ^ sw16(row) from global memory.
  const int nkb = (q0 + FBM) / FBN;
  unsigned voff[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    const int row = 8 * (2 * w + h2) + (lane >> 3);
    voff[h2] = (unsigned)(row * HD + 8 * ((lane & 7) ^ sw16(row))) * 2u;
  }
  const unsigned wblk = 2048u * (unsigned)__builtin_amdgcn_readfirstlane(w);
  auto issue_k = [&](int t) {
    const bf16* src = k + base + (int64_t)t * FBN * HD;
    const unsigned dst = lds_u32(Kr[t % 2]) + wblk;
    dma16_s(src, voff[0], dst);
    dma16_s(src, voff[1], dst + 1024);
  };
  auto issue_v = [&](int t) {
    const bf16* src = v + base + (int64_t)t * FBN * HD;
    const unsigned dst = lds_u32(Vr[t % 2]) + wblk;
    dma16_s(src, voff[0], dst);
    dma16_s(src, voff[1], dst + 1024);
  };

  // Prologue, issued before anything else the workgroup loads: K_0, V_0,
  // K_1, V_1 resident (nkb >= 2: a workgroup's own two diagonal tiles).
  // The end of step kb waits for K_{kb+1} and V_{kb+1}
  // (issued one step earlier), and after its barrier issues K_{kb+2} and
  // V_{kb+2} into slot kb % 2, which every wave has finished reading.
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    issue_k(t);
    issue_v(t);
  }

  // B operand of S^T = K Q_s^T: lane holds Q_s[qrow][16*ks + 8*g .. +7].
  bf16x8 qreg[4];
  {
    const bf16* qp = q + base + (int64_t)qrow * HD + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qreg[ks] = *reinterpret_cast<const bf16x8*>(qp + 16 * ks);
  }
  // The pre-scale's q_s is stored after the K/V prologue: a store issued
  // before it would make its vmcnt wait also wait for the store to land.
  auto nan_to_inf = [](float x) { return x != x ? __builtin_inff() : x; };
  float sq = 0.0f;  // |q_s|^2 of the lane's row (the guard's partial, below)
  if (prep.q_s != nullptr) {
    // Fused pre-scale: `q` is the raw query; q_s = cast(q * scale)
    // (flash.py:833) is formed in registers and written once for the
    // backward.
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8 x = qreg[ks];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = (bf16)((float)x[e] * prep.q_scale);
        const float f = (float)x[e];
        sq = __builtin_fmaf(f, f, sq);
      }
      qreg[ks] = x;
    }
    sq = nan_to_inf(sq + __shfl_xor(sq, 32, 64));
  }

  const bool has_sink = sink != nullptr;
  float m_row, l_row;
  sink_init(var, has_sink, has_sink ? sink[h] : 0.0f, m_row, l_row);
  if (g == 1) l_row = 0.0f;  // the two lane halves carry partial row sums
  f32x16 oacc[2];
  zero16(oacc[0]);
  zero16(oacc[1]);

  wait_vmcnt<0>();
  __syncthreads();
  // q_s and the guard's partial maxima go out after the prologue's wait, so
  // that wait does not cover them; they land during step 0, whose own wait
  // does. (Two-variant kernels store them at the end instead: there the
  // early store's addresses raise the scalar register count past its limit.)
  auto store_prep = [&] {
    if (prep.q_s != nullptr) {
      bf16* qsp = prep.q_s + base + (int64_t)qrow * HD + 8 * g;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) *reinterpret_cast<bf16x8*>(qsp + 16 * ks) = qreg[ks];
    }
  };
  if (EARLY_QS) store_prep();

  // A operand of S^T: lane reads K[32 mt + c32][16 ks + 8 g ..] (rows 32 mt
  // apart share the chunk placement).
  int koff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = c32 * HD + 8 * ((2 * ks + g) ^ sw16(c32));
  auto scores = [&](int kb, f32x16 (&s)[2]) {
    const bf16* Kt = Kr[kb % 2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      zero16(s[mt]);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&Kt[32 * mt * HD + koff[ks]]);
        s[mt] = mfma32(a, qreg[ks], s[mt]);
      }
    }
  };

  // V^T operand reads: lane reads 4 columns 32 dt + 16 (G & 1) + 4 m4 .. of
  // rows 16 kc + 4 (G >> 1) + j4 and that + 8 (the chunk placement does not
  // depend on kc).
  int voffr[2][2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int r = 4 * (G >> 1) + j4 + 8 * h2, col = 32 * dt + 16 * (G & 1) + 4 * m4;
      voffr[dt][h2] = r * HD + 8 * ((col >> 3) ^ sw16(r)) + (col & 7);
    }

  // Transform tile kb's scores (cur) into weights, accumulate P V. Only tiles
  // that cross the diagonal (diag_tag = true_type) evaluate the causal mask.
  auto consume = [&](auto diag_tag, int kb, f32x16 (&cur)[2]) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    const int k0 = kb * FBN;
    float lsum = 0.0f;
    if (MODE == MODE_NOSHIFT) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float s = cur[mt][r];
          const float x = BOUNDED ? s : __builtin_fminf(s, var.clamp);
          float rr;
          float p = powN<L2N>(POLY ? rho_poly(x, rr) : FAST ? rho_fast(x, rr) : rho_exact(x, rr),
                              log2n);
          if (DIAG && k0 + 32 * mt + 8 * (r >> 2) + 4 * g + (r & 3) > qrow) p = 0.0f;
          cur[mt][r] = p;
          lsum += p;
        }
      l_row += lsum;
    } else {
      float tmax = -__builtin_inff();
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float s = cur[mt][r];
          if (DIAG && k0 + 32 * mt + 8 * (r >> 2) + 4 * g + (r & 3) > qrow) s = -__builtin_inff();
          cur[mt][r] = s;
          tmax = __builtin_fmaxf(tmax, s);
        }
      tmax = __builtin_fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      float m_new = __builtin_fmaxf(m_row, tmax), m_prev = m_row;
      if (!has_sink && kb == 0) {  // flash.py:239-245
        m_new = tmax;
        m_prev = m_new;
      }
      float alpha;
      if (MODE == MODE_SOFTMAX) {
        alpha = __builtin_amdgcn_exp2f((m_prev - m_new) * kLog2e);
        const float mb = m_new * kLog2e;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(cur[mt][r], kLog2e, -mb));
            cur[mt][r] = p;
            lsum += p;
          }
      } else {
        float rr;
        const float shf = rho_exact(-m_new, rr);
        alpha = powN<L2N>(rho_exact(m_prev, rr) * shf, log2n);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float s = cur[mt][r];
            float p = powN<L2N>((FAST ? rho_fast(s, rr) : rho_exact(s, rr)) * shf, log2n);
            if (s == -__builtin_inff()) p = 0.0f;
            cur[mt][r] = p;
            lsum += p;
          }
      }
      l_row = __builtin_fmaf(l_row, alpha, lsum);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
      m_row = m_new;
    }
    // O^T += V^T P^T over four 16-key chunks. k-slot s of lane group g holds
    // key 16kc + 8(s/4) + 4g + s%4 (the accumulator rows the lane owns); the
    // V^T operand is read from the row-major V tile with two transposing
    // reads whose row order matches.
    const bf16* Vt = Vr[kb % 2];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const int mt = kc >> 1, rr = 8 * (kc & 1);
      bf16x8 pb;
#pragma unroll
      for (int s = 0; s < 8; ++s) pb[s] = (bf16)cur[mt][rr + s];
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const bf16* vp = &Vt[16 * kc * HD];
        oacc[dt] = mfma32(join(read_tr(vp + voffr[dt][0]), read_tr(vp + voffr[dt][1])), pb,
                          oacc[dt]);
      }
    }
  };

  auto visible = [&](int kb) { return kb < nkb && kb * FBN <= qw + 31; };
  // Tiles below the workgroup's first query row: no mask and no branch. The
  // next tiles' loads are issued after the barrier, so every wave's only
  // outstanding memory operations at the wait are the previous step's loads.
  static_assert(FBM == 2 * FBN, "a workgroup's query block spans two key tiles");
  const int nfull = q0 / FBN;
  for (int kb = 0; kb < nfull; ++kb) {
    f32x16 sc[2];
    scores(kb, sc);
    consume(std::false_type{}, kb, sc);
    wait_vmcnt<0>();
    __syncthreads();
    issue_k(kb + 2);
    issue_v(kb + 2);
  }
  // The workgroup's two diagonal tiles (nkb = nfull + 2), already loaded or
  // in flight; a wave skips the tiles wholly above its own rows.
  for (int kb = nfull; kb < nkb; ++kb) {
    f32x16 sc[2];
    if (visible(kb)) {
      scores(kb, sc);
      if (kb * FBN + FBN - 1 > qw)
        consume(std::true_type{}, kb, sc);
      else
        consume(std::false_type{}, kb, sc);
    }
    wait_vmcnt<0>();
    __syncthreads();
  }

  if (prep.q_s != nullptr && prep.partial != nullptr) {
    // The range guard's partial maxima (flash.py:841-849): |q_s|^2 over the
    // workgroup's 128 query rows and |k|^2, |v| over the 128 key rows of its
    // diagonal block (so the grid covers every row once), the k and v rows
    // read from the two diagonal tiles still in the LDS ring. Thread t takes
    // physical chunks 4 (t % 2) .. + 3 of row t / 2, so the thread pair
    // covers the row whatever the chunk placement. NaN becomes +inf so that
    // it fails the guard.
    const int r = tid >> 1, slot = (nfull + (r >> 6)) & 1;
    const bf16* kp = &Kr[slot][(r & 63) * HD + 32 * (tid & 1)];
    const bf16* vp = &Vr[slot][(r & 63) * HD + 32 * (tid & 1)];
    float sk = 0.0f, mv = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bf16x8 kx = *reinterpret_cast<const bf16x8*>(kp + 8 * c);
      const bf16x8 vx = *reinterpret_cast<const bf16x8*>(vp + 8 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float kf = (float)kx[e];
        sk = __builtin_fmaf(kf, kf, sk);
        mv = __builtin_fmaxf(mv, nan_to_inf(__builtin_fabsf((float)vx[e])));
      }
    }
    sk = nan_to_inf(sk + __shfl_xor(sk, 1, 64));
    float sqm = sq;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      sqm = __builtin_fmaxf(sqm, __shfl_xor(sqm, m, 64));
      sk = __builtin_fmaxf(sk, __shfl_xor(sk, m, 64));
      mv = __builtin_fmaxf(mv, __shfl_xor(mv, m, 64));
    }
    if (lane == 0) {
      red[0][w] = sqm;
      red[1][w] = sk;
      red[2][w] = mv;
    }
    __syncthreads();
    if (tid < 3)
      prep.partial[(int64_t)bid * 3 + tid] =
          __builtin_fmaxf(__builtin_fmaxf(red[tid][0], red[tid][1]),
                          __builtin_fmaxf(red[tid][2], red[tid][3]));
  }

  const float l_tot = l_row + __shfl_xor(l_row, 32, 64);
  const float inv = 1.0f / l_tot;
  const int64_t orow = base + (int64_t)qrow * HD;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * dt + 8 * j + 4 * g;
      f32x4 val;
#pragma unroll
      for (int i = 0; i < 4; ++i) val[i] = oacc[dt][4 * j + i] * inv;
      bf16x4 ob = {(bf16)val[0], (bf16)val[1], (bf16)val[2], (bf16)val[3]};
      *reinterpret_cast<bf16x4*>(o + orow + d) = ob;
      if (var.precise && o_precise != nullptr)
        *reinterpret_cast<f32x4*>(o_precise + orow + d) = val;
    }
  if (g == 0) stat[(int64_t)bh * T_ + qrow] = final_stat(var, m_row, l_tot);
  if (!EARLY_QS) store_prep();
  if (prep.dq_zero != nullptr) {
    // The workgroup's 128 query rows of the accumulator are one contiguous
    // 32 KB run: eight coalesced 16-byte stores per thread.
    f32x4* z = reinterpret_cast<f32x4*>(prep.dq_zero + base + (int64_t)q0 * HD);
#pragma unroll
    for (int i = 0; i < FBM * HD / 4 / 256; ++i) z[tid + 256 * i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
}

// Four workgroups per CU (four waves per SIMD, at most 128 VGPRs) for the
// single variants whose body fits that budget; three (168 VGPRs) for those
// that would spill at 128: the runtime power loop (n outside 8..32), the
// polynomial radical, the clamped (unbounded) unshifted weights other than
// the fast radical at n = 8 or 16, and the two-variant guarded kernels.
constexpr int fwd_blocks_per_cu(int lo, int hi) {
  return lo != hi || cfg_l2n(lo) == 0 || cfg_poly(lo) ||
                 (cfg_mode(lo) == MODE_NOSHIFT && !cfg_bounded(lo) &&
                  (!cfg_fast(lo) || cfg_l2n(lo) == 5))
             ? 3
             : 4;
}

// The guard word (if any) picks the low or the high variant for the whole
// grid, mirroring lax.cond(in_range, low, high).
template <int LO, int HI>
__global__ __launch_bounds__(256, fwd_blocks_per_cu(LO, HI)) void fwd_mfma_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ sink, bf16* __restrict__ o, float* __restrict__ o_precise,
    float* __restrict__ stat, int H, int T_, KVariant lo, KVariant hi,
    const int32_t* __restrict__ guard, FwdPrep prep) {
  __shared__ __attribute__((aligned(16))) bf16 Kr[2][FBN * HD];
  __shared__ __attribute__((aligned(16))) bf16 Vr[2][FBN * HD];
  __shared__ float red[3][4];
  if (LO == HI || guard_in_range(guard))
    fwd_body<cfg_mode(LO), cfg_fast(LO), cfg_bounded(LO), cfg_l2n(LO), cfg_poly(LO), LO == HI>(
        q, k, v, sink, o, o_precise, stat, H, T_, lo, prep, Kr, Vr, red, blockIdx.x, gridDim.x);
  else
    fwd_body<cfg_mode(HI), cfg_fast(HI), cfg_bounded(HI), cfg_l2n(HI), cfg_poly(HI), LO == HI>(
        q, k, v, sink, o, o_precise, stat, H, T_, hi, prep, Kr, Vr, red, blockIdx.x, gridDim.x);
}

// The guard's closing step and the high half of lax.cond in one launch.
// Every workgroup reduces the low launch's partial maxima to the same
// decision (flash.py:843-849: in range iff max|q_s|^2 max|k|^2 <= (b/1.01)^2,
// max|sink| <= b/1.01 and max|v| <= vmax); workgroup 0 stores the guard word
// for the backward. In range, that is all; otherwise the grid walks every
// (head, query tile) with the high variant.
struct GuardIn {
  const float* partial;
  int nparts;
  float bound_sq, bound_s, vmax;
  int32_t* guard;
};

template <int HI>
__global__ __launch_bounds__(256, 2) void fwd_fallback_kernel(
    const bf16* __restrict__ q_s, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ sink, bf16* __restrict__ o, float* __restrict__ o_precise,
    float* __restrict__ stat, int H, int T_, KVariant hi, GuardIn gin, int ntiles) {
  __shared__ __attribute__((aligned(16))) bf16 Kr[2][FBN * HD];
  __shared__ __attribute__((aligned(16))) bf16 Vr[2][FBN * HD];
  __shared__ float red[3][4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float mx[3] = {0.0f, 0.0f, 0.0f};
  for (int b = tid; b < gin.nparts; b += 256)
#pragma unroll
    for (int j = 0; j < 3; ++j) mx[j] = __builtin_fmaxf(mx[j], gin.partial[(int64_t)b * 3 + j]);
#pragma unroll
  for (int j = 0; j < 3; ++j)
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) mx[j] = __builtin_fmaxf(mx[j], __shfl_xor(mx[j], m, 64));
  if (lane == 0)
#pragma unroll
    for (int j = 0; j < 3; ++j) red[j][w] = mx[j];
  __syncthreads();
  float tot[3];
#pragma unroll
  for (int j = 0; j < 3; ++j)
    tot[j] = __builtin_fmaxf(__builtin_fmaxf(red[j][0], red[j][1]), __builtin_fmaxf(red[j][2], red[j][3]));
  float ms = 0.0f;
  if (sink != nullptr)
    for (int h = 0; h < H; ++h) {
      const float a = __builtin_fabsf(sink[h]);
      ms = __builtin_fmaxf(ms, a != a ? __builtin_inff() : a);
    }
  bool ok = tot[0] * tot[1] <= gin.bound_sq && tot[2] <= gin.vmax;
  if (sink != nullptr) ok = ok && ms <= gin.bound_s;
  if (blockIdx.x == 0 && tid == 0) {
    gin.guard[0] = ok ? 1 : 0;
    float* f = reinterpret_cast<float*>(gin.guard);
    f[1] = tot[0];
    f[2] = tot[1];
    f[3] = tot[2];
    f[4] = ms;
  }
  if (ok) return;
  for (int b = blockIdx.x; b < ntiles; b += gridDim.x) {
    __syncthreads();  // LDS of the previous tile is no longer read
    fwd_body<cfg_mode(HI), cfg_fast(HI), cfg_bounded(HI), cfg_l2n(HI), cfg_poly(HI), false>(
        q_s, k, v, sink, o, o_precise, stat, H, T_, hi, FwdPrep{}, Kr, Vr, red, b, ntiles);
  }
}

typedef void (*FallbackFn)(const bf16*, const bf16*, const bf16*, const float*, bf16*, float*,
                           float*, int, int, KVariant, GuardIn, int);

// The high variants a guarded call pairs with (shifted, exact rho), as for
// the guarded two-variant kernels.
FallbackFn pick_fallback(int ch) {
  if (ch == cfg_of(MODE_SHIFT, false, false, 3)) return fwd_fallback_kernel<cfg_of(MODE_SHIFT, false, false, 3)>;
  if (ch == cfg_of(MODE_SHIFT, false, false, 4)) return fwd_fallback_kernel<cfg_of(MODE_SHIFT, false, false, 4)>;
  if (ch == cfg_of(MODE_SHIFT, false, false, 5)) return fwd_fallback_kernel<cfg_of(MODE_SHIFT, false, false, 5)>;
  if (ch == cfg_of(MODE_SHIFT, false, false, 0)) return fwd_fallback_kernel<cfg_of(MODE_SHIFT, false, false, 0)>;
  return nullptr;
}

typedef void (*FwdFn)(const bf16*, const bf16*, const bf16*, const float*, bf16*, float*, float*,
                      int, int, KVariant, KVariant, const int32_t*, FwdPrep);

FwdFn pick_fwd(int cl, int ch) { ALGX_PICK_ALL(fwd_mfma_kernel) }

}  // namespace
}  // namespace mfma

bool mfma_supported(int T, int D, int dtype) {
  return dtype == ALGX_BF16 && D == mfma::HD && T >= mfma::FBM && T % mfma::FBM == 0;
}

int32_t launch_fwd_mfma(const void* q, const void* k, const void* v, const float* sink, void* o,
                        float* o_precise, float* stat, int B, int H, int T, const KVariant& lo,
                        const KVariant& hi, const int32_t* guard, hipStream_t s) {
  using namespace mfma;
  const int grid = B * H * (T / FBM);
  FwdFn fn = pick_fwd(cfg_for(lo), guard != nullptr ? cfg_for(hi) : cfg_for(lo));
  if (fn == nullptr) return fail("attn_fwd: no MFMA kernel for this variant pair");
  launch_k(probe_for(ALGX_PROBE_ATTN_FWD), fn, dim3(grid), dim3(256), s, (const bf16*)q,
           (const bf16*)k, (const bf16*)v, sink, (bf16*)o, o_precise, stat, H, T, lo, hi, guard,
           FwdPrep{});
  return check_launch("attn_fwd_mfma");
}

int64_t fwd_fused_partials(int B, int H, int T) {
  return (int64_t)B * H * (T / mfma::FBM);
}

int32_t launch_fwd_fused(const void* q, const void* k, const void* v, const float* sink,
                         void* q_s, void* o, float* o_precise, float* stat, int32_t* guard,
                         float* partial, float* dq_zero, int B, int H, int T, float q_scale,
                         float bound, float vmax, const KVariant& lo, const KVariant& hi,
                         hipStream_t s) {
  using namespace mfma;
  const int grid = B * H * (T / FBM);
  // Low variant over the whole grid, fused with the pre-scale and (guarded)
  // the guard's partial maxima. On out-of-range inputs its outputs are
  // overwritten by the high launch below.
  FwdFn fn = pick_fwd(cfg_for(lo), cfg_for(lo));
  if (fn == nullptr) return fail("attn_forward: no MFMA kernel for the low variant");
  FwdPrep pre{(bf16*)q_s, q_scale, guard != nullptr ? partial : nullptr, dq_zero};
  launch_k(probe_for(ALGX_PROBE_ATTN_FWD), fn, dim3(grid), dim3(256), s, (const bf16*)q,
           (const bf16*)k, (const bf16*)v, sink, (bf16*)o, o_precise, stat, H, T, lo, lo,
           (const int32_t*)nullptr, pre);
  if (int32_t rc = check_launch("attn_forward_low")) return rc;
  if (guard == nullptr) return 0;
  FallbackFn fh = pick_fallback(cfg_for(hi));
  if (fh == nullptr) return fail("attn_forward: no MFMA kernel for the high variant");
  const double b101 = (double)bound / 1.01;
  const GuardIn gin{partial, grid, (float)(b101 * b101), (float)b101, vmax, guard};
  const int fgrid = grid < 512 ? grid : 512;  // two workgroups per CU
  launch_k(Probe{}, fh, dim3(fgrid), dim3(256), s, (const bf16*)q_s, (const bf16*)k,
           (const bf16*)v, sink, (bf16*)o, o_precise, stat, H, T, hi, gin, grid);
  return check_launch("attn_forward_high");
}

}  // namespace algx
