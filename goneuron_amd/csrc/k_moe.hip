// Mixture of Experts (moe.go) kernels.
//
// Reference semantics kept (moe.go:140-313):
//  - training mode: each gate logit gets (u*2 - 1)*0.05 with u from the
//    layer's RNG(42) stream, which runs on across samples and steps; every
//    trainBatchParallel worker clone has its own stream (net.go:129-152);
//  - softmax with float64 exp, then sort.Slice by descending probability:
//    for <= 12 experts Go sorts by insertion, which keeps ties in index order;
//    the routing here is that stable order;
//  - out = sum over the top k (in routing order) of expert_out * p;
//  - backward: active experts get grad * p through their Dense (LeakyReLU
//    0.1) backward; gate grad = grad . expert_out for active experts, plus
//    0.2 (p - 1/E) for all in training mode; softmax backward.
#include "gn_common.h"

namespace gn {



// One thread per sample: noisy logits (training), softmax, stable descending
// order; writes probabilities [B][E] and the top-k ids [B][K].
__global__ __launch_bounds__(256) void moe_route_kernel(const float *__restrict__ logits,
                                                        float *__restrict__ prob,
                                                        int32_t *__restrict__ act, MoeRoute rt) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= rt.B) return;
  const int E = rt.E;
  float l[MOE_MAX_E], p[MOE_MAX_E];
  int order[MOE_MAX_E];
  for (int e = 0; e < E; ++e) l[e] = logits[(size_t)b * E + e];
  if (rt.training) {
    int w = 0, j = b;
    if (rt.chunk > 0) {
      w = 1 + b / rt.chunk;
      j = b % rt.chunk;
    }
    uint64_t s = lcg_jump(rt.base[w], (uint64_t)j * E);
    for (int e = 0; e < E; ++e) {
      s = s * LCG_A + LCG_C;
      const float u = (float)(s >> 33) / (float)(1u << 31);
      l[e] = __fadd_rn(l[e], __fmul_rn(__fsub_rn(__fmul_rn(u, 2.0f), 1.0f), 0.05f));
    }
  }
  float mx = l[0];
  for (int e = 1; e < E; ++e) mx = l[e] > mx ? l[e] : mx;
  float sum = 0.f;
  for (int e = 0; e < E; ++e) {
    p[e] = (float)exp((double)(l[e] - mx));
    sum += p[e];
  }
  for (int e = 0; e < E; ++e) {
    p[e] = p[e] / sum;
    prob[(size_t)b * E + e] = p[e];
    order[e] = e;
  }
  for (int i = 1; i < E; ++i)
    for (int j = i; j > 0 && p[order[j]] > p[order[j - 1]]; --j) {
      const int t = order[j];
      order[j] = order[j - 1];
      order[j - 1] = t;
    }
  for (int r = 0; r < rt.K; ++r) act[(size_t)b * rt.K + r] = order[r];
}

// y[b][o] = sum_r eout[act_r][b][o] * p[b][act_r], in routing order
__global__ __launch_bounds__(256) void moe_combine_kernel(const float *__restrict__ eout,
                                                          const float *__restrict__ prob,
                                                          const int32_t *__restrict__ act,
                                                          float *__restrict__ y, int B, int O, int E,
                                                          int K) {
  const int64_t n = (int64_t)B * O;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int b = (int)(i / O), o = (int)(i % O);
    float s = 0.f;
    for (int r = 0; r < K; ++r) {
      const int e = act[(size_t)b * K + r];
      s = __fadd_rn(s, __fmul_rn(eout[((size_t)e * B + b) * O + o], prob[(size_t)b * E + e]));
    }
    y[i] = s;
  }
}

// Expert deltas: edz[e][b][o] = (g * p) * leaky'(eout) for active (b, e), else 0
__global__ __launch_bounds__(256) void moe_expert_dz_kernel(const float *__restrict__ g,
                                                            const float *__restrict__ eout,
                                                            const float *__restrict__ prob,
                                                            const int32_t *__restrict__ act,
                                                            float *__restrict__ edz, int B, int O,
                                                            int E, int K) {
  const int64_t n = (int64_t)E * B * O;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int e = (int)(i / ((int64_t)B * O));
    const int b = (int)((i / O) % B), o = (int)(i % O);
    bool on = false;
    for (int r = 0; r < K; ++r) on |= act[(size_t)b * K + r] == e;
    float v = 0.f;
    if (on) {
      const float d = eout[i] > 0.0f ? 1.0f : 0.1f;
      v = __fmul_rn(__fmul_rn(g[(size_t)b * O + o], prob[(size_t)b * E + e]), d);
    }
    edz[i] = v;
  }
}

// Gate deltas, one thread per sample: gate grad (dot with the active expert
// outputs, + 0.2 (p - 1/E) in training), then the softmax backward.
__global__ __launch_bounds__(256) void moe_gate_grad_kernel(const float *__restrict__ g,
                                                            const float *__restrict__ eout,
                                                            const float *__restrict__ prob,
                                                            const int32_t *__restrict__ act,
                                                            float *__restrict__ dzg, int B, int O,
                                                            int E, int K, int training) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= B) return;
  float gg[MOE_MAX_E];
  for (int e = 0; e < E; ++e) gg[e] = 0.f;
  for (int r = 0; r < K; ++r) {
    const int e = act[(size_t)b * K + r];
    float d = 0.f;
    for (int o = 0; o < O; ++o) d += g[(size_t)b * O + o] * eout[((size_t)e * B + b) * O + o];
    gg[e] = d;
  }
  const float *p = prob + (size_t)b * E;
  if (training) {
    const float target = 1.0f / (float)E;
    for (int e = 0; e < E; ++e) gg[e] = __fadd_rn(gg[e], __fmul_rn(0.2f, __fsub_rn(p[e], target)));
  }
  float sp = 0.f;
  for (int e = 0; e < E; ++e) sp += p[e] * gg[e];
  for (int e = 0; e < E; ++e) dzg[(size_t)b * E + e] = p[e] * (gg[e] - sp);
}

hipError_t launch_moe_route(const float *logits, float *prob, int32_t *act, const MoeRoute &rt,
                            hipStream_t s) {
  if (rt.E > MOE_MAX_E || rt.K < 1 || rt.K > rt.E) return hipErrorInvalidValue;
  hipLaunchKernelGGL(moe_route_kernel, dim3((rt.B + 255) / 256), dim3(256), 0, s, logits, prob, act, rt);
  return hipGetLastError();
}

static unsigned grid_of(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (unsigned)(b > 8192 ? 8192 : (b < 1 ? 1 : b));
}

hipError_t launch_moe_combine(const float *eout, const float *prob, const int32_t *act, float *y,
                              int B, int O, int E, int K, hipStream_t s) {
  hipLaunchKernelGGL(moe_combine_kernel, dim3(grid_of((int64_t)B * O)), dim3(256), 0, s, eout, prob,
                     act, y, B, O, E, K);
  return hipGetLastError();
}

hipError_t launch_moe_backward_deltas(const float *g, const float *eout, const float *prob,
                                      const int32_t *act, float *edz, float *dzg, int B, int O,
                                      int E, int K, int training, hipStream_t s) {
  hipLaunchKernelGGL(moe_expert_dz_kernel, dim3(grid_of((int64_t)E * B * O)), dim3(256), 0, s, g, eout,
                     prob, act, edz, B, O, E, K);
  hipLaunchKernelGGL(moe_gate_grad_kernel, dim3((B + 255) / 256), dim3(256), 0, s, g, eout, prob, act,
                     dzg, B, O, E, K, training);
  return hipGetLastError();
}

}  // namespace gn
