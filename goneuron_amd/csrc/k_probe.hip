// Measurement probe: a kernel that does nothing but back-to-back
// v_mfma_f32_32x32x2_f32 on registers, to measure the rate the matrix cores
// sustain on this part (the roofline's practical ceiling next to the
// published peak).  Not used by the training step.
#include "gn_common.h"

namespace gn {

typedef float px16 __attribute__((ext_vector_type(16)));

// 4 independent accumulators per wave, so every MFMA can issue back to back.
__global__ __launch_bounds__(256) void mfma_probe_kernel(float *out, int iters, float a, float b) {
  px16 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = px16{};
  const float x = a + threadIdx.x * 1e-6f, y = b;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[c], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

hipError_t launch_mfma_probe(float *out, int blocks, int iters, hipStream_t s) {
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(256), 0, s, out, iters, 1.0f, 2.0f);
  return hipGetLastError();
}

}  // namespace gn
