// SequenceUnroller(GRU) training kernels (unroller.go:57-213, gru.go).
//
// Reference semantics kept (the quirks are the oracle's, see gru.go):
//  - gates (update u, reset r, candidate c); pre = b + Wx x, plus Wh_u h and
//    Wh_r h for u and r; the candidate adds Wh_r (r * h) with the *reset*
//    gate's recurrent block (gru.go:246-253); h' = h + u (c - h);
//  - backward per step (gru.go:347-510): dU = dh (c - h_prev) u (1 - u),
//    dC = dh (1 - u) (1 - c^2); the reset delta is never computed (0);
//    dh_prev = Wh_u^T dU + Wh_r^T (dC r) + dh u is added to the running dh
//    (unroller.go:189-206);
//  - input-weight gradients use the last step's input for every step.
//
// GPU formulation.  x W_x^T + b for every (sample, step) is one GEMM before
// the recurrence.  The recurrence runs one workgroup per sample, thread i
// owning hidden unit i: the forward reads W_h transposed ([H][2H], so that
// the threads of one row read consecutive floats), the backward reads W_h
// as stored (column i of W_h^T is row-contiguous across threads).  The
// backward stores dG = [dU | 0 | dC] per step; the weight gradients are then
// GEMMs over (sample, step): dW_h,u = dU^T h_prev, dW_h,r = dC^T (r * h_prev),
// dW_x = (sum_t dG)^T x_last, db = sum dG.
#include "gn_common.h"

namespace gn {

__device__ __forceinline__ float gru_sig(float x) { return 1.0f / (1.0f + (float)exp((double)(-x))); }
__device__ __forceinline__ float gru_tanh(float x) { return (float)tanh((double)x); }

// xw [B*T][3H] = b + Wx x_t (from the GEMM); WhT [H][2H]; writes pre
// [B*T][3H] (with the recurrent parts), hprev [B*T][H] (h before each step),
// rh [B*T][H] (r * h_prev) and out [B][H] (h_T).
__global__ __launch_bounds__(1024) void gru_fwd_kernel(const float *__restrict__ xw,
                                                       const float *__restrict__ WhT,
                                                       float *__restrict__ pre,
                                                       float *__restrict__ hprev,
                                                       float *__restrict__ rh,
                                                       float *__restrict__ out, int T, int H,
                                                       int seq) {
  extern __shared__ float sm[];
  float *h = sm, *srh = sm + H;
  const int b = blockIdx.x, i = threadIdx.x;
  const bool act = i < H;
  if (act) h[i] = 0.0f;  // GRU.Reset (gru.go:171-180)
  __syncthreads();
  for (int t = 0; t < T; ++t) {
    const size_t row = (size_t)b * T + t;
    float u = 0.f, hi = 0.f, pu = 0.f, pr = 0.f;
    if (act) {
      hi = h[i];
      float su = 0.f, sr = 0.f;
      for (int j = 0; j < H; ++j) {
        const float hj = h[j];
        su += WhT[(size_t)j * 2 * H + i] * hj;
        sr += WhT[(size_t)j * 2 * H + H + i] * hj;
      }
      pu = xw[row * 3 * H + i] + su;
      pr = xw[row * 3 * H + H + i] + sr;
      u = gru_sig(pu);
      const float r = gru_sig(pr);
      srh[i] = r * hi;
      hprev[row * H + i] = hi;
    }
    __syncthreads();
    if (act) {
      float sc = 0.f;
      for (int j = 0; j < H; ++j) sc += WhT[(size_t)j * 2 * H + H + i] * srh[j];
      const float pc = xw[row * 3 * H + 2 * H + i] + sc;
      const float c = gru_tanh(pc);
      pre[row * 3 * H + i] = pu;
      pre[row * 3 * H + H + i] = pr;
      pre[row * 3 * H + 2 * H + i] = pc;
      rh[row * H + i] = srh[i];
      h[i] = hi + u * (c - hi);  // every read of h[] this step happened before the barrier
      if (seq) out[row * H + i] = h[i];  // returnSequences: every state, [B][T][H]
    }
    __syncthreads();
  }
  if (act && !seq) out[(size_t)b * H + i] = h[i];
}

// g [B][H] = dL/dh_T; Wh [2H][H] as stored; writes dG [B*T][3H].
__global__ __launch_bounds__(1024) void gru_bwd_kernel(const float *__restrict__ g,
                                                       const float *__restrict__ pre,
                                                       const float *__restrict__ hprev,
                                                       const float *__restrict__ Wh,
                                                       float *__restrict__ dG, int T, int H,
                                                       int seq) {
  extern __shared__ float sm[];
  float *sdu = sm, *sdcr = sm + H;
  const int b = blockIdx.x, i = threadIdx.x;
  const bool act = i < H;
  // g: dL/dh_T [B][H], or with seq dL/dh_t [B][T][H] added to the carried
  // gradient at every step (unroller.go:192-198)
  float dh = act ? (seq ? g[((size_t)b * T + T - 1) * H + i] : g[(size_t)b * H + i]) : 0.f;
  for (int t = T - 1; t >= 0; --t) {
    const size_t row = (size_t)b * T + t;
    float u = 0.f;
    if (act && seq && t < T - 1) dh += g[row * H + i];
    if (act) {
      u = gru_sig(pre[row * 3 * H + i]);
      const float r = gru_sig(pre[row * 3 * H + H + i]);
      const float c = gru_tanh(pre[row * 3 * H + 2 * H + i]);
      const float hp = hprev[row * H + i];
      const float du = dh * (c - hp) * u * (1 - u);
      const float dc = dh * (1 - u) * (1 - c * c);
      dG[row * 3 * H + i] = du;
      dG[row * 3 * H + H + i] = 0.0f;
      dG[row * 3 * H + 2 * H + i] = dc;
      sdu[i] = du;
      sdcr[i] = dc * r;
    }
    __syncthreads();
    if (act) {
      float s = 0.f;
      for (int j = 0; j < H; ++j) s += Wh[(size_t)j * H + i] * sdu[j];
      for (int j = 0; j < H; ++j) s += Wh[(size_t)(H + j) * H + i] * sdcr[j];
      s += dh * u;
      dh += s;
    }
    __syncthreads();  // sdu / sdcr are rewritten next step
  }
}

bool gru_supported(int H) { return H >= 1 && H <= 1024; }

hipError_t launch_gru_fwd(const float *xw, const float *WhT, float *pre, float *hprev, float *rh,
                          float *out, int B, int T, int H, hipStream_t s, int seq) {
  if (!gru_supported(H)) return hipErrorInvalidValue;
  const int threads = (H + 63) / 64 * 64;
  hipLaunchKernelGGL(gru_fwd_kernel, dim3(B), dim3(threads), 2 * H * sizeof(float), s, xw, WhT, pre,
                     hprev, rh, out, T, H, seq);
  return hipGetLastError();
}

hipError_t launch_gru_bwd(const float *g, const float *pre, const float *hprev, const float *Wh,
                          float *dG, int B, int T, int H, hipStream_t s, int seq) {
  if (!gru_supported(H)) return hipErrorInvalidValue;
  const int threads = (H + 63) / 64 * 64;
  hipLaunchKernelGGL(gru_bwd_kernel, dim3(B), dim3(threads), 2 * H * sizeof(float), s, g, pre, hprev,
                     Wh, dG, T, H, seq);
  return hipGetLastError();
}

}  // namespace gn
