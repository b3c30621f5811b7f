// C ABI of the attention kernels: argument validation, variant conversion
// and dispatch between the MFMA path (bf16, D=64, T%128==0) and the generic
// path (everything else). A guarded MFMA call launches one kernel that reads
// the device guard word and runs the low or the high variant for the whole
// grid; the generic path enqueues both variants and the unselected one
// returns at once. Either way this mirrors lax.cond(in_range, low, high) of
// flash.py:853-856 without a host round trip.
#include <initializer_list>
#include <cstdlib>
#include <mutex>

#include "attn_aux.h"

namespace algx {
namespace {

int32_t to_kvar(const algx_attn_variant* v, KVariant& out, const char* which) {
  if (v == nullptr) return fail(std::string("attn: missing ") + which + " variant");
  if (v->kind != ALGX_SOFTMAX && v->kind != ALGX_ASINH)
    return fail(std::string("attn: unknown kind in ") + which + " variant");
  if (v->kind == ALGX_ASINH && (v->n < 2 || (v->n & (v->n - 1))))
    return fail("attn: asinh kernel needs n to be a power of two");
  if (v->kind == ALGX_ASINH && v->inv_stat && v->shift)
    return fail("attn: inverse-denominator statistic requires shift=False");
  out.kind = v->kind;
  out.log2n = v->kind == ALGX_ASINH ? ilog2(v->n) : 0;
  out.shift = v->kind == ALGX_SOFTMAX ? 1 : (v->shift != 0);
  out.fast = v->fast_rho != 0;
  out.inv_stat = v->inv_stat != 0;
  out.bounded = v->bounded_scores != 0;
  out.precise = v->precise_output != 0;
  out.clamp = v->clamp;
  out.slope = v->kind == ALGX_ASINH ? (float)v->n : 1.0f;
  out.poly = v->kind == ALGX_ASINH && v->poly_rho != 0;
  if (out.poly && (out.shift || v->n != 16))
    return fail("attn: bounded radical approximation requires shift=False and n=16");
  // The guard's unclamped low variant is never paired with the polynomial
  // (flash.py:835-836 refuses range_guard with poly_rho).
  if (out.poly && out.bounded)
    return fail("attn: bounded radical approximation requires bounded_scores=0 "
                "(range_guard is for exact radical evaluation)");
  return 0;
}

// Scratch of algx_attn_forward_noalloc: the guard's partial maxima, one
// triple per forward workgroup, at most kNoAllocParts workgroups (768 KiB).
// Each GPU the library runs on holds its own copy until the process ends.
constexpr int64_t kNoAllocParts = 1 << 16;
static __device__ __align__(256) float scratch[3 * kNoAllocParts];

// Device address of `scratch` on the current device, looked up once per
// device (the host-side name of a __device__ array is not its address).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

int32_t scratch_on_current_device(float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail("attn_forward_noalloc: no current device");
  if (dev < 0 || dev >= kMaxDevices) return fail("attn_forward_noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(std::string("attn_forward_noalloc: hipGetSymbolAddress(scratch): ") +
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = (float*)p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

bool force_generic() {
  const char* e = std::getenv("ALGX_FORCE_GENERIC");
  return e != nullptr && e[0] == '1';
}

// The kernels move (B, H, T, D) rows with 16-byte vector accesses.
int32_t check_aligned(const char* who, std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (p != nullptr && (reinterpret_cast<uintptr_t>(p) & 15) != 0)
      return fail(std::string(who) + ": q, k, v, o, dO and gradient tensors must be 16-byte aligned");
  return 0;
}

int32_t check_shape(int B, int H, int T, int D, int dtype) {
  if (B < 0 || H < 0 || T < 0) return fail("attn: negative size");
  if (dtype != ALGX_BF16 && dtype != ALGX_F32) return fail("attn: dtype must be bf16 or f32");
  if (D != 16 && D != 32 && D != 64) return fail("attn: head dim must be 16, 32 or 64");
  return 0;
}

}  // namespace
}  // namespace algx

using namespace algx;

extern "C" int32_t algx_attn_guard_words(void) { return guard_words(); }

extern "C" int32_t algx_attn_prepare(const void* q, const void* k, const void* v,
                                     const float* sink, void* q_s, int32_t* guard, int32_t B,
                                     int32_t H, int32_t T, int32_t D, int32_t dtype,
                                     float q_scale, float bound, float vmax, void* stream) {
  if (int32_t rc = check_shape(B, H, T, D, dtype)) return rc;
  if ((int64_t)B * H * T == 0) return 0;
  if (q == nullptr || q_s == nullptr) return fail("attn_prepare: null q or q_s");
  if (guard != nullptr && (k == nullptr || v == nullptr))
    return fail("attn_prepare: the guard needs k and v");
  if (int32_t rc = check_aligned("attn_prepare", {q, k, v, q_s})) return rc;
  return launch_prepare(q, k, v, sink, q_s, guard, B, H, T, D, dtype, q_scale, bound, vmax,
                        (hipStream_t)stream);
}

extern "C" int32_t algx_attn_fwd(const void* q, const void* k, const void* v, const float* sink,
                                 void* o, float* o_precise, float* stat, int32_t B, int32_t H,
                                 int32_t T, int32_t D, int32_t dtype,
                                 const algx_attn_variant* low, const algx_attn_variant* high,
                                 const int32_t* guard, void* stream) {
  if (int32_t rc = check_shape(B, H, T, D, dtype)) return rc;
  KVariant kl{}, kh{};
  if (int32_t rc = to_kvar(low, kl, "low")) return rc;
  if (guard != nullptr) {
    if (int32_t rc = to_kvar(high, kh, "high")) return rc;
  } else {
    kh = kl;
  }
  if ((int64_t)B * H * T == 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || stat == nullptr)
    return fail("attn_fwd: null pointer");
  if ((kl.precise || (guard != nullptr && kh.precise)) && o_precise == nullptr)
    return fail("attn_fwd: precise-output variant needs o_precise");
  if (int32_t rc = check_aligned("attn_fwd", {q, k, v, o, o_precise})) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (mfma_supported(T, D, dtype) && !force_generic())
    return launch_fwd_mfma(q, k, v, sink, o, o_precise, stat, B, H, T, kl, kh, guard, s);
  if (int32_t rc = launch_fwd_generic(q, k, v, sink, o, o_precise, stat, B, H, T, D, dtype, kl,
                                      guard, 1, s))
    return rc;
  if (guard != nullptr)
    return launch_fwd_generic(q, k, v, sink, o, o_precise, stat, B, H, T, D, dtype, kh, guard, 0,
                              s);
  return 0;
}

extern "C" int64_t algx_attn_forward_workspace_bytes(int32_t B, int32_t H, int32_t T,
                                                     int32_t D) {
  (void)D;
  if (B <= 0 || H <= 0 || T <= 0) return 0;
  return fwd_fused_partials(B, H, T) * 3 * (int64_t)sizeof(float);
}

extern "C" int32_t algx_attn_forward(const void* q, const void* k, const void* v,
                                     const float* sink, void* q_s, void* o, float* o_precise,
                                     float* stat, int32_t* guard, void* workspace,
                                     void* bwd_workspace, int32_t B, int32_t H, int32_t T,
                                     int32_t D, int32_t dtype, float q_scale, float bound,
                                     float vmax, const algx_attn_variant* low,
                                     const algx_attn_variant* high, void* stream) {
  if (int32_t rc = check_shape(B, H, T, D, dtype)) return rc;
  KVariant kl{}, kh{};
  if (int32_t rc = to_kvar(low, kl, "low")) return rc;
  if (guard != nullptr) {
    if (int32_t rc = to_kvar(high, kh, "high")) return rc;
  } else {
    kh = kl;
  }
  if ((int64_t)B * H * T == 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || q_s == nullptr || o == nullptr ||
      stat == nullptr)
    return fail("attn_forward: null pointer");
  if ((kl.precise || (guard != nullptr && kh.precise)) && o_precise == nullptr)
    return fail("attn_forward: precise-output variant needs o_precise");
  if (int32_t rc = check_aligned("attn_forward", {q, k, v, q_s, o, o_precise, bwd_workspace}))
    return rc;
  hipStream_t s = (hipStream_t)stream;
  if (mfma_supported(T, D, dtype) && !force_generic()) {
    if (guard != nullptr && workspace == nullptr)
      return fail("attn_forward: the guard needs the workspace");
    // The backward workspace starts with its float32 dQ accumulator.
    return launch_fwd_fused(q, k, v, sink, q_s, o, o_precise, stat, guard, (float*)workspace,
                            (float*)bwd_workspace, B, H, T, q_scale, bound, vmax, kl, kh, s);
  }
  if (int32_t rc = launch_prepare(q, k, v, sink, q_s, guard, B, H, T, D, dtype, q_scale, bound,
                                  vmax, s))
    return rc;
  if (int32_t rc = launch_fwd_generic(q_s, k, v, sink, o, o_precise, stat, B, H, T, D, dtype, kl,
                                      guard, 1, s))
    return rc;
  if (guard != nullptr)
    return launch_fwd_generic(q_s, k, v, sink, o, o_precise, stat, B, H, T, D, dtype, kh, guard,
                              0, s);
  return 0;
}

extern "C" int64_t algx_attn_bwd_workspace_bytes(int32_t B, int32_t H, int32_t T, int32_t D) {
  const int64_t rows = (int64_t)B * H * T;
  const int64_t acc = rows * D * (int64_t)sizeof(float);
  const int64_t di = ((rows * (int64_t)sizeof(float) + 255) / 256) * 256;
  return acc + di;
}

extern "C" int32_t algx_attn_bwd(const void* q, const void* k, const void* v, const float* sink,
                                 const void* o, const float* o_precise, const float* stat,
                                 const void* dout, void* dq, void* dk, void* dv, float* dsink,
                                 void* workspace, int32_t workspace_state, int32_t B, int32_t H,
                                 int32_t T, int32_t D, int32_t dtype, float q_scale,
                                 const algx_attn_variant* low, const algx_attn_variant* high,
                                 const int32_t* guard, void* stream) {
  if (int32_t rc = check_shape(B, H, T, D, dtype)) return rc;
  KVariant kl{}, kh{};
  if (int32_t rc = to_kvar(low, kl, "low")) return rc;
  if (guard != nullptr) {
    if (int32_t rc = to_kvar(high, kh, "high")) return rc;
  } else {
    kh = kl;
  }
  if (workspace_state != ALGX_ATTN_WS_RAW && workspace_state != ALGX_ATTN_WS_CLEARED)
    return fail("attn_bwd: workspace_state must be ALGX_ATTN_WS_RAW or ALGX_ATTN_WS_CLEARED");
  hipStream_t s = (hipStream_t)stream;
  const int64_t rows = (int64_t)B * H * T;
  if (rows == 0) {
    if (sink != nullptr && dsink != nullptr) return fill_f32(dsink, H, 0.0f, s);
    return 0;
  }
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || stat == nullptr ||
      dout == nullptr || dq == nullptr || dk == nullptr || dv == nullptr || workspace == nullptr)
    return fail("attn_bwd: null pointer");
  if ((kl.precise || kh.precise) && o_precise == nullptr)
    return fail("attn_bwd: precise-output variant needs o_precise");
  if (int32_t rc = check_aligned("attn_bwd", {q, k, v, o, o_precise, dout, dq, dk, dv, workspace}))
    return rc;
  const bool mfma = mfma_supported(T, D, dtype) && !force_generic();
  float* dq_acc = (float*)workspace;
  float* di = (float*)((char*)workspace + rows * D * (int64_t)sizeof(float));
  // The pre-pass forms di and dsink, and clears the dQ accumulator unless
  // the forward already did (a workspace it prepared).
  const bool cleared = mfma && workspace_state == ALGX_ATTN_WS_CLEARED;
  if (int32_t rc = launch_bwd_pre(dout, o, o_precise, stat, sink, di,
                                  mfma && !cleared ? dq_acc : nullptr, dsink, B, H, T, D, dtype,
                                  kl, kh, guard, s))
    return rc;
  if (mfma) {
    if (int32_t rc = launch_bwd_mfma(q, k, v, stat, di, dout, dq_acc, dk, dv, B, H, T, kl, kh,
                                     guard, s))
      return rc;
    return launch_dq_finish(dq_acc, dq, rows * D, dtype, kl, kh, guard, q_scale, s);
  }
  if (int32_t rc = launch_bwd_generic(q, k, v, stat, di, dout, dq, dk, dv, B, H, T, D, dtype,
                                      q_scale, kl, guard, 1, s))
    return rc;
  if (guard != nullptr)
    return launch_bwd_generic(q, k, v, stat, di, dout, dq, dk, dv, B, H, T, D, dtype, q_scale, kh,
                              guard, 0, s);
  return 0;
}

// algx_attn_forward with the guard partials in the library's per-device
// scratch array instead of a caller workspace: no allocation of any kind.
extern "C" int32_t algx_attn_forward_noalloc(const void* q, const void* k, const void* v,
                                             const float* sink, void* q_s, void* o,
                                             float* o_precise, float* stat, int32_t* guard,
                                             void* bwd_workspace, int32_t B, int32_t H,
                                             int32_t T, int32_t D,
                                             int32_t dtype, float q_scale, float bound,
                                             float vmax, const algx_attn_variant* low,
                                             const algx_attn_variant* high, void* stream) {
  if (int32_t rc = check_shape(B, H, T, D, dtype)) return rc;
  // The limit is checked for every guarded call, whichever path would run,
  // before anything touches the device.
  if (guard != nullptr && fwd_fused_partials(B, H, T) > kNoAllocParts)
    return fail("attn_forward_noalloc: B * H * T / 128 exceeds the scratch limit of 65536 "
                "forward workgroups; use algx_attn_forward with a workspace");
  if ((int64_t)B * H * T > 0 && (q == nullptr || k == nullptr || v == nullptr ||
                                 q_s == nullptr || o == nullptr || stat == nullptr))
    return fail("attn_forward_noalloc: null pointer");
  float* part = nullptr;
  if (guard != nullptr && (int64_t)B * H * T > 0 && mfma_supported(T, D, dtype) &&
      !force_generic()) {
    if (int32_t rc = scratch_on_current_device(&part)) return rc;
  }
  return algx_attn_forward(q, k, v, sink, q_s, o, o_precise, stat, guard, part, bwd_workspace, B,
                           H, T, D, dtype, q_scale, bound, vmax, low, high, stream);
}
