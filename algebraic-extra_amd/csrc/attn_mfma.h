// Shared pieces of the gfx950 MFMA attention kernels (bf16, D = 64).
#pragma once

#include "attn_aux.h"

namespace algx {
namespace mfma {

constexpr int HD = 64;
// forward tiles: 128 queries per workgroup (32 per wave), 64-key tiles
constexpr int FBM = 128, FBN = 64;

// Unpadded [row][64] bf16 tiles (128-byte rows) whose 16-byte chunk c of row
// r sits at chunk c ^ sw16(r), a bijection of (r / 2) % 8. Sixteen
// consecutive rows read at one chunk (16-byte reads) and four consecutive
// rows read over four consecutive chunks (8-byte transposing reads) each
// touch the 64 LDS banks once.
__device__ __forceinline__ int sw16(int r) {
  const int m = (r >> 1) & 7;
  return ((m & 1) << 2) | (m >> 1);
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ unsigned lds_u32(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Direct-to-LDS load: lane i's 16 bytes at global `base` + voff land at LDS
// byte address lds + 16 i (M0 = the wave-uniform lds). Issued as assembly so
// that the compiler's wait insertion does not treat every later LDS read as
// depending on it; callers wait for their loads with explicit vmcnt counts.
// M0 is set here and named as clobbered; the compiler uses M0 nowhere in the
// attention kernels (every M0 write in their generated code is one of these
// loads), so it holds no value of its own there across the statement.
__device__ __forceinline__ void dma16_s(const void* base, unsigned voff, unsigned lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(base)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N), expcnt/lgkmcnt unconstrained (N < 16).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

enum { MODE_SOFTMAX = 0, MODE_NOSHIFT = 1, MODE_SHIFT = 2 };

// Extra work of a forward launch: q_s != null -> `q` is the raw query and the
// kernel writes q_s = cast(q * q_scale); partial != null -> it also writes the
// range guard's three partial maxima per workgroup.
struct FwdPrep {
  bf16* q_s = nullptr;
  float q_scale = 1.0f;
  float* partial = nullptr;
  // Non-null: the backward's float32 dQ accumulator ((B, H, T, 64)), whose
  // rows of the workgroup's query block are set to zero in passing.
  float* dq_zero = nullptr;
};

// s_waitcnt immediate for vmcnt(0) with expcnt/lgkmcnt left unconstrained
// (gfx9 encoding: vmcnt[3:0] and [15:14], expcnt[6:4], lgkmcnt[11:8]).
constexpr int kWaitVm0 = 0x0F70;

// Kernel configuration packed in one int:
// MODE | FAST << 2 | BOUNDED << 3 | L2N << 4 (3 bits) | POLY << 7.
constexpr int cfg_of(int mode, bool fast, bool bounded, int l2n, bool poly = false) {
  return mode | (fast ? 4 : 0) | (bounded ? 8 : 0) | (l2n << 4) | (poly ? 128 : 0);
}
constexpr int cfg_mode(int c) { return c & 3; }
constexpr bool cfg_fast(int c) { return (c & 4) != 0; }
constexpr bool cfg_bounded(int c) { return (c & 8) != 0; }
constexpr int cfg_l2n(int c) { return (c >> 4) & 7; }
constexpr bool cfg_poly(int c) { return (c & 128) != 0; }
// Power template argument: n = 8, 16, 32 unrolled; other n by a runtime loop.
inline int l2n_arg(int log2n) { return (log2n >= 3 && log2n <= 5) ? log2n : 0; }
inline int cfg_for(const KVariant& v) {
  if (v.kind == ALGX_SOFTMAX) return cfg_of(MODE_SOFTMAX, false, false, 1);
  if (v.poly) return cfg_of(MODE_NOSHIFT, false, v.bounded != 0, l2n_arg(v.log2n), true);
  if (v.shift) return cfg_of(MODE_SHIFT, v.fast != 0, false, l2n_arg(v.log2n));
  return cfg_of(MODE_NOSHIFT, v.fast != 0, v.bounded != 0, l2n_arg(v.log2n));
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// Transposing LDS read (ds_read_b64_tr_b16): lane 4j+m of each 16-lane group
// addresses 4 consecutive bf16 of row j; lane i of the group receives element
// i%4 of the rows addressed by lanes i/4, i/4+4, i/4+8, i/4+12.
__device__ __forceinline__ bf16x4 read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
}

__device__ __forceinline__ bf16x8 join(bf16x4 a, bf16x4 b) {
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ void zero16(f32x16& a) {
#pragma unroll
  for (int r = 0; r < 16; ++r) a[r] = 0.0f;
}

// Position of key (or query) offset `off` (0..15) inside a 16-wide chunk of
// a transposed operand tile: bits 2 and 3 swapped, i.e. k-slot (g, s) of
// lane group g holds offset 8*(s/4) + 4*g + s%4, which is exactly the set of
// rows a 32x32 accumulator lane holds in registers 8*(j%2)..+7 of chunk j.
__device__ __forceinline__ int slot_pos(int off) {
  return (off & 3) | ((off >> 3) & 1) << 2 | ((off >> 2) & 1) << 3;
}

// blockIdx -> (head, tile): heads are dealt to XCDs (blockIdx % 8) so every
// tile of a head runs on the same XCD and shares its L2; tiles are issued in
// order of decreasing causal work when `descending`.
__device__ __forceinline__ void map_block(int bid, int nheads, int ntiles, bool descending,
                                          int& bh, int& tile) {
  int r;
  if ((nheads & 7) == 0) {
    const int nh8 = nheads >> 3;
    r = bid >> 3;
    bh = (bid & 7) + 8 * (r % nh8);
    r = r / nh8;
  } else {
    bh = bid % nheads;
    r = bid / nheads;
  }
  tile = descending ? ntiles - 1 - r : r;
}

__device__ __forceinline__ bf16x8 scale_bf16x8(bf16x8 x, float s) {
  bf16x8 y;
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = (bf16)((float)x[e] * s);
  return y;
}

// x^(2^log2n) with a compile-time exponent when L2N > 0 (int_pow of flash.py:95-104).
template <int L2N> __device__ __forceinline__ float powN(float x, int log2n) {
  if (L2N > 0) {
#pragma unroll
    for (int i = 0; i < L2N; ++i) x = x * x;
    return x;
  }
  return pow2n(x, log2n);
}

}  // namespace mfma
}  // namespace algx

// Every asinh configuration instantiated as a single-variant kernel.
#define ALGX_ASINH_CFGS(X, K)                                                          \
  X(K, cfg_of(MODE_SHIFT, true, false, 3)) X(K, cfg_of(MODE_SHIFT, true, false, 4))    \
  X(K, cfg_of(MODE_SHIFT, true, false, 5)) X(K, cfg_of(MODE_SHIFT, true, false, 0))    \
  X(K, cfg_of(MODE_SHIFT, false, false, 3)) X(K, cfg_of(MODE_SHIFT, false, false, 4))  \
  X(K, cfg_of(MODE_SHIFT, false, false, 5)) X(K, cfg_of(MODE_SHIFT, false, false, 0))  \
  X(K, cfg_of(MODE_NOSHIFT, true, true, 3)) X(K, cfg_of(MODE_NOSHIFT, true, true, 4))  \
  X(K, cfg_of(MODE_NOSHIFT, true, true, 5)) X(K, cfg_of(MODE_NOSHIFT, true, true, 0))  \
  X(K, cfg_of(MODE_NOSHIFT, false, true, 3)) X(K, cfg_of(MODE_NOSHIFT, false, true, 4)) \
  X(K, cfg_of(MODE_NOSHIFT, false, true, 5)) X(K, cfg_of(MODE_NOSHIFT, false, true, 0)) \
  X(K, cfg_of(MODE_NOSHIFT, true, false, 3)) X(K, cfg_of(MODE_NOSHIFT, true, false, 4)) \
  X(K, cfg_of(MODE_NOSHIFT, true, false, 5)) X(K, cfg_of(MODE_NOSHIFT, true, false, 0)) \
  X(K, cfg_of(MODE_NOSHIFT, false, false, 3)) X(K, cfg_of(MODE_NOSHIFT, false, false, 4)) \
  X(K, cfg_of(MODE_NOSHIFT, false, false, 5)) X(K, cfg_of(MODE_NOSHIFT, false, false, 0)) \
  X(K, cfg_of(MODE_NOSHIFT, false, false, 4, true))

#define ALGX_PICK_SINGLE(K, C) \
  if (cl == (C)) return K<(C), (C)>;
// Guarded launches pair a bounded unshifted low variant with the shifted
// exact-rho high variant of the same n (flash.py:850-852).
#define ALGX_PICK_GUARDED(K, FASTLO, L2)                                                    \
  if (cl == cfg_of(MODE_NOSHIFT, FASTLO, true, L2) && ch == cfg_of(MODE_SHIFT, false, false, L2)) \
    return K<cfg_of(MODE_NOSHIFT, FASTLO, true, L2), cfg_of(MODE_SHIFT, false, false, L2)>;
#define ALGX_PICK_ALL(K)                                                                 \
  if (cl == ch) {                                                                        \
    ALGX_PICK_SINGLE(K, cfg_of(MODE_SOFTMAX, false, false, 1))                           \
    ALGX_ASINH_CFGS(ALGX_PICK_SINGLE, K)                                                 \
    return nullptr;                                                                      \
  }                                                                                      \
  ALGX_PICK_GUARDED(K, true, 3) ALGX_PICK_GUARDED(K, true, 4) ALGX_PICK_GUARDED(K, true, 5) \
  ALGX_PICK_GUARDED(K, true, 0) ALGX_PICK_GUARDED(K, false, 3) ALGX_PICK_GUARDED(K, false, 4) \
  ALGX_PICK_GUARDED(K, false, 5) ALGX_PICK_GUARDED(K, false, 0)                          \
  return nullptr;
