// Clock and MFMA-rate probe used by the benchmark to state the fraction of peak at the
// clock the GPU actually sustains under MFMA load (the 2516.6 TFLOP/s dense fp16 peak
// assumes 2.4 GHz).  Every wavefront issues `iters` rounds of four independent
// v_mfma_f32_32x32x16_f16; wavefront 0 of each work-group samples the shader clock
// counter (s_memtime) and the constant 100 MHz counter (s_memrealtime) around its loop.
#include <hip/hip_runtime.h>

#include "../../include/co_alibi.h"
#include "coalibi_common.h"

namespace coalibi {
namespace {

__global__ __launch_bounds__(256) void mfma_probe_kernel(unsigned long long* ticks, float* sink, int iters) {
  const int lane = threadIdx.x & 63;
  f16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = static_cast<_Float16>(0.001f * (lane + e));
    b[e] = static_cast<_Float16>(0.002f * (lane - e));
  }
  f32x16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  const unsigned long long c0 = __builtin_readcyclecounter();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
  }
  const unsigned long long c1 = __builtin_readcyclecounter();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;  // keeps the products live
  if (threadIdx.x == 0) {
    ticks[2 * blockIdx.x] = c1 - c0;
    ticks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

}  // namespace
}  // namespace coalibi

extern "C" int co_alibi_probe_mfma(void* ticks, void* sink, int blocks, int iters, void* stream) {
  if (ticks == nullptr || sink == nullptr || blocks < 1 || iters < 1) return CO_ALIBI_EINVAL;
  hipLaunchKernelGGL(coalibi::mfma_probe_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<unsigned long long*>(ticks), static_cast<float*>(sink), iters);
  return hipGetLastError() == hipSuccess ? CO_ALIBI_OK : CO_ALIBI_ELAUNCH;
}
