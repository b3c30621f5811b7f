// Issue rates of the instructions the attention forward's weight loop is made
// of, on gfx950, timed in shader clocks (s_memtime) inside one workgroup per
// CU. Two parts:
//  1. one opcode at a time (v_mul_f32, v_fma_f32, v_rsq_f32, v_exp_f32,
//     v_sqrt_f32), 8 independent registers per lane, 1/2/4 waves per SIMD;
//  2. the forward tile's mix per wave (16 v_mfma_f32_32x32x16_bf16, 240
//     full-rate VALU, 32 v_rsq_f32, all independent) alone, interleaved one
//     MFMA per 15 VALU + 2 rsq, and grouped as 8 MFMA | VALU | 8 MFMA;
// plus the MFMA's own cycle count, which calibrates the counter.
//
// Build and run (one GPU):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       algebraic-extra_amd/microbench/issue_rates.hip -o algebraic-extra_amd/microbench/issue_rates
//   algebraic-extra_amd/microbench/issue_rates
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBlocks = 256;       // one workgroup per CU
constexpr int kMaxThreads = 1024;  // 4 waves per SIMD

#define CHECK(x)                                                               \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));             \
      std::exit(1);                                                            \
    }                                                                          \
  } while (0)

template <int OP>
__device__ __forceinline__ void op1(float& x) {
  if (OP == 0) asm volatile("v_mul_f32 %0, %0, %0" : "+v"(x));
  if (OP == 1) asm volatile("v_fma_f32 %0, %0, %0, %0" : "+v"(x));
  if (OP == 2) asm volatile("v_rsq_f32 %0, %0" : "+v"(x));
  if (OP == 3) asm volatile("v_exp_f32 %0, %0" : "+v"(x));
  if (OP == 4) asm volatile("v_sqrt_f32 %0, %0" : "+v"(x));
}

// Part 1: every lane applies OP to 8 registers per iteration.
template <int OP>
__global__ __launch_bounds__(kMaxThreads) void single_op(int iters, float* out,
                                                         unsigned long long* cyc) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = 1.0f + 0.001f * (threadIdx.x + i);
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) op1<OP>(x[i]);
  }
  __syncthreads();
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}

// 15 full-rate VALU and 2 rsq on the 8 registers.
__device__ __forceinline__ void valu17(float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 15; ++i) {
    if (i & 1)
      op1<0>(x[i & 7]);
    else
      op1<1>(x[i & 7]);
  }
  op1<2>(x[3]);
  op1<2>(x[6]);
}

// Part 2: MODE 0 VALU only, 1 MFMA only, 2 interleaved, 3 grouped.
template <int MODE>
__global__ __launch_bounds__(kMaxThreads) void tile_mix(int iters, float* out,
                                                        unsigned long long* cyc) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = 1.0f + 0.001f * (threadIdx.x + i);
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (__bf16)(0.001f * e);
    b[e] = (__bf16)(0.002f * e);
  }
  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    if (MODE == 0) {
#pragma unroll
      for (int g = 0; g < 16; ++g) valu17(x);
    } else if (MODE == 1) {
#pragma unroll
      for (int g = 0; g < 16; ++g)
        acc[g & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[g & 3], 0, 0, 0);
    } else if (MODE == 2) {
#pragma unroll
      for (int g = 0; g < 16; ++g) {
        acc[g & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[g & 3], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        valu17(x);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int g = 0; g < 8; ++g)
        acc[g & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[g & 3], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int g = 0; g < 16; ++g) valu17(x);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int g = 0; g < 8; ++g)
        acc[g & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[g & 3], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[i][r];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}

typedef void (*Kernel)(int, float*, unsigned long long*);

// Mean over the workgroups of the cycles one launch of `k` took.
double cycles(Kernel k, int threads, int iters, float* out, unsigned long long* cyc,
              float* ms = nullptr) {
  hipLaunchKernelGGL(k, dim3(kBlocks), dim3(threads), 0, 0, 10, out, cyc);  // warm
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  hipLaunchKernelGGL(k, dim3(kBlocks), dim3(threads), 0, 0, iters, out, cyc);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  if (ms != nullptr) CHECK(hipEventElapsedTime(ms, e0, e1));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  unsigned long long c[kBlocks];
  CHECK(hipMemcpy(c, cyc, sizeof(c), hipMemcpyDeviceToHost));
  double avg = 0.0;
  for (int i = 0; i < kBlocks; ++i) avg += (double)c[i];
  return avg / kBlocks;
}

}  // namespace

int main() {
  float* out;
  unsigned long long* cyc;
  CHECK(hipMalloc(&out, (size_t)kBlocks * kMaxThreads * sizeof(float)));
  CHECK(hipMalloc(&cyc, kBlocks * sizeof(unsigned long long)));

  {  // counter calibration: one wave per SIMD, 4 independent accumulators
    const int iters = 20000;
    float ms = 0.0f;
    const double c = cycles(tile_mix<1>, 256, iters / 4, out, cyc, &ms);
    const double per = c / ((iters / 4) * 16.0);
    std::printf("v_mfma_f32_32x32x16_bf16: %.2f counter cycles per instruction per SIMD; "
                "counter %.1f MHz\n", per, c / (ms * 1e3));
  }
  const char* names[] = {"v_mul_f32", "v_fma_f32", "v_rsq_f32", "v_exp_f32", "v_sqrt_f32"};
  const Kernel ops[] = {single_op<0>, single_op<1>, single_op<2>, single_op<3>, single_op<4>};
  for (int waves = 1; waves <= 4; waves *= 2)
    for (int op = 0; op < 5; ++op) {
      const int iters = 20000;
      const double c = cycles(ops[op], 256 * waves, iters, out, cyc);
      std::printf("%-11s waves/SIMD %d: %.2f cycles per wave instruction per SIMD\n", names[op],
                  waves, c / ((double)waves * iters * 8));
    }
  const char* mixes[] = {"VALU only (240 + 32 rsq)", "MFMA only (16)",
                         "interleaved (1 MFMA : 17 VALU)", "grouped 8 MFMA | VALU | 8 MFMA"};
  const Kernel mix[] = {tile_mix<0>, tile_mix<1>, tile_mix<2>, tile_mix<3>};
  for (int waves = 1; waves <= 4; ++waves)
    for (int m = 0; m < 4; ++m) {
      const int iters = 2000;
      const double c = cycles(mix[m], 256 * waves, iters, out, cyc);
      std::printf("tile mix, waves/SIMD %d, %-32s %7.1f cycles per wave-tile per SIMD\n", waves,
                  mixes[m], c / ((double)waves * iters));
    }
  CHECK(hipFree(out));
  CHECK(hipFree(cyc));
  return 0;
}
