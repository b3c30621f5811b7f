// Error reporting and small utility kernels shared by the algx entry points.
#include <mutex>

#include "common.h"

namespace algx {

namespace {
thread_local std::string g_error;
// Process-wide: frameworks launch backward passes from their own threads.
struct ArmedProbe {
  int which = ALGX_PROBE_NONE;
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
std::mutex g_probe_mu;
ArmedProbe g_probe;
}  // namespace

Probe probe_for(int which) {
  std::lock_guard<std::mutex> lk(g_probe_mu);
  Probe p;
  if (g_probe.which != ALGX_PROBE_NONE && g_probe.which == which) {
    p.start = g_probe.start;
    p.stop = g_probe.stop;
  }
  return p;
}

void set_error(const std::string& msg) { g_error = msg; }

int32_t fail(const std::string& msg) {
  g_error = msg;
  return 1;
}

int32_t check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_error = std::string(what) + ": " + hipGetErrorString(e);
    return 2;
  }
  return 0;
}

__global__ void fill_f32_kernel(float* __restrict__ p, int64_t n, float value) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = value;
}

// Fills n floats with a kernel (graph-capture friendly, unlike a memset node).
int32_t fill_f32(float* p, int64_t n, float value, hipStream_t s) {
  if (n <= 0) return 0;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  fill_f32_kernel<<<(int)blocks, 256, 0, s>>>(p, n, value);
  return check_launch("fill_f32");
}

// One v_mfma_f32_32x32x16_bf16 with the operand/accumulator layout every
// MFMA kernel here assumes: A lane l holds A[l%32][8(l/32)..+7], B lane l
// holds B[8(l/32)..+7][l%32] (read from B^T rows), and accumulator register
// r of lane l is D[8(r/4) + 4(l/32) + r%4][l%32].
__global__ __launch_bounds__(64) void selftest_mfma32_kernel(const bf16* __restrict__ a,
                                                             const bf16* __restrict__ bt,
                                                             float* __restrict__ d) {
  const int l = threadIdx.x, g = l >> 5, c = l & 31;
  const bf16x8 av = *reinterpret_cast<const bf16x8*>(a + c * 16 + 8 * g);
  const bf16x8 bv = *reinterpret_cast<const bf16x8*>(bt + c * 16 + 8 * g);
  f32x16 acc;
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
  for (int r = 0; r < 16; ++r) d[(8 * (r >> 2) + 4 * g + (r & 3)) * 32 + c] = acc[r];
}

}  // namespace algx

extern "C" int32_t algx_selftest_mfma32(const void* a, const void* bt, float* d, void* stream) {
  if (a == nullptr || bt == nullptr || d == nullptr) return algx::fail("selftest: null pointer");
  algx::selftest_mfma32_kernel<<<1, 64, 0, (hipStream_t)stream>>>((const algx::bf16*)a,
                                                                 (const algx::bf16*)bt, d);
  return algx::check_launch("selftest_mfma32");
}

extern "C" int32_t algx_set_probe(int32_t which, void* start_event, void* stop_event) {
  if (which != ALGX_PROBE_NONE && (start_event == nullptr || stop_event == nullptr))
    return algx::fail("set_probe: null event");
  std::lock_guard<std::mutex> lk(algx::g_probe_mu);
  algx::g_probe.which = which;
  algx::g_probe.start = (hipEvent_t)start_event;
  algx::g_probe.stop = (hipEvent_t)stop_event;
  return 0;
}

extern "C" const char* algx_last_error(void) { return algx::g_error.c_str(); }

extern "C" int32_t algx_version(void) { return 3; }
