// Transformer-path kernels: Embedding gather / last-sample scatter,
// PositionalEncoding add, causal multi-head attention forward / backward,
// LayerNorm forward / backward, CLSPooling, per-sample token sums.
//
// Semantics follow the reference per sample (transformer.go, layernorm.go,
// embedding.go):
//  - scores s_ij = (q_i . k_j) / sqrt(hd), -1e9 where j > i under the causal
//    mask, row softmax with exp in float64 (activations.go:161-183),
//    o_i = sum_j p_ij v_j (transformer.go:466-503);
//  - backward dP_ij = gO_i . v_j, dS_ij = p_ij (dP_ij - sum_k dP_ik p_ik),
//    gradScore = dS / sqrt(hd), gQ += gradScore k, gK += gradScore q,
//    gV += p gO (transformer.go:583-648);
//  - LayerNorm y = gamma (x - mu)/std + beta, std = sqrt(var + eps) in float64;
//    backward dx = (gp - sum(gp)/N)/std - (x-mu) sum(gp (x-mu)) / (N std^2)
//    with gp = g gamma (layernorm.go:405-424; the exact gradient would have
//    std^3 in the last term);
//  - Embedding.Backward zeroes the whole gradient before scattering, so only
//    the last sample of each worker chunk contributes (embedding.go:152-154).
#include "gn_common.h"

namespace gn {

constexpr int AT_T = 128;   // max sequence length held in LDS
constexpr int AT_HD = 32;   // max head dim held in LDS
constexpr int AT_HP = AT_HD + 1;

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wmax(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ---------------------------------------------------------------------------
// Embedding / PositionalEncoding / CLS
// ---------------------------------------------------------------------------
// out[r, :] = E[floor(x[r]), :] + (pe ? pe[r % T, :] : 0); ids[r] = index.
// Out-of-range ids (an error in the reference, embedding.go:126-128) raise
// *err and read row 0.
__global__ __launch_bounds__(256) void embed_kernel(const float *__restrict__ x,
                                                    const float *__restrict__ E,
                                                    int32_t *__restrict__ ids,
                                                    float *__restrict__ out, int rows, int V,
                                                    int D, int *__restrict__ err) {
  const int64_t n = (int64_t)rows * D;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int r = (int)(e / D), d = (int)(e % D);
    int idx = (int)floor((double)x[r]);
    if (idx < 0 || idx >= V) {
      if (d == 0) atomicOr(err, 1);
      idx = 0;
    }
    if (d == 0) ids[r] = idx;
    out[e] = E[(int64_t)idx * D + d];
  }
}

__global__ __launch_bounds__(256) void pe_add_kernel(const float *__restrict__ x,
                                                     const float *__restrict__ pe,
                                                     float *__restrict__ out, int64_t n, int TD) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256)
    out[e] = x[e] + pe[e % TD];
}

// grad[E] = 0, then for each worker chunk's last sample, in order: rows of its
// tokens scatter-added in token order (one block: a deterministic sequence).
__global__ __launch_bounds__(256) void embed_grad_kernel(const float *__restrict__ g,
                                                         const int32_t *__restrict__ ids,
                                                         float *__restrict__ gradE, int B, int T,
                                                         int D, int W, float scale) {
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  const int chunk = (B + Wc - 1) / Wc;
  for (int s = chunk - 1; s < B + chunk - 1; s += chunk) {
    const int b = min(s, B - 1);
    for (int t = 0; t < T; ++t) {
      const int idx = ids[(int64_t)b * T + t];
      for (int d = threadIdx.x; d < D; d += 256)  // thread d owns column d: ordered adds
        gradE[(int64_t)idx * D + d] += g[((int64_t)b * T + t) * D + d] * scale;
    }
    if (s >= B - 1) break;
  }
}

__global__ __launch_bounds__(256) void cls_fwd_kernel(const float *__restrict__ x,
                                                      float *__restrict__ out, int B, int TD, int D) {
  const int64_t n = (int64_t)B * D;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256)
    out[e] = x[(e / D) * TD + e % D];
}

__global__ __launch_bounds__(256) void cls_bwd_kernel(const float *__restrict__ g,
                                                      float *__restrict__ gin, int B, int TD,
                                                      int D) {
  const int64_t n = (int64_t)B * TD;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t b = e / TD;
    const int r = (int)(e % TD);
    gin[e] = r < D ? g[b * D + r] : 0.0f;
  }
}

// S[b, :] = sum_t X[b, t, :]   (per-sample token sums for the Q10 dW outer products)
__global__ __launch_bounds__(256) void token_sum_kernel(const float *__restrict__ X,
                                                        float *__restrict__ S, int B, int T, int N) {
  const int64_t n = (int64_t)B * N;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t b = e / N;
    const int c = (int)(e % N);
    const float *p = X + b * T * N + c;
    float s = 0.f;
    for (int t = 0; t < T; ++t) s += p[(int64_t)t * N];
    S[e] = s;
  }
}

// ---------------------------------------------------------------------------
// LayerNorm over rows of N (one wave64 per row)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ln_fwd_kernel(const float *__restrict__ x,
                                                     const float *__restrict__ gam,
                                                     const float *__restrict__ bet,
                                                     float *__restrict__ y,
                                                     float *__restrict__ stats, int rows, int N,
                                                     float eps) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float *xr = x + (int64_t)r * N;
  float s = 0.f;
  for (int i = lane; i < N; i += 64) s += xr[i];
  const float mean = wsum(s) / (float)N;
  float ss = 0.f;
  for (int i = lane; i < N; i += 64) {
    const float d = xr[i] - mean;
    ss += d * d;
  }
  const float var = wsum(ss) / (float)N;
  const float std = (float)sqrt((double)(var + eps));
  for (int i = lane; i < N; i += 64) y[(int64_t)r * N + i] = gam[i] * ((xr[i] - mean) / std) + bet[i];
  if (lane == 0) {
    stats[2 * r] = mean;
    stats[2 * r + 1] = std;
  }
}

// dx by the reference formula; gx[r, i] = g * xhat (for the dgamma column sums)
__global__ __launch_bounds__(256) void ln_bwd_kernel(const float *__restrict__ g,
                                                     const float *__restrict__ x,
                                                     const float *__restrict__ gam,
                                                     const float *__restrict__ stats,
                                                     float *__restrict__ dx,
                                                     float *__restrict__ gx, int rows, int N) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float *gr = g + (int64_t)r * N, *xr = x + (int64_t)r * N;
  const float mean = stats[2 * r], std = stats[2 * r + 1];
  float sg = 0.f, sgx = 0.f;
  for (int i = lane; i < N; i += 64) {
    const float gp = gr[i] * gam[i];
    sg += gp;
    sgx += gp * (xr[i] - mean);
  }
  sg = wsum(sg);
  sgx = wsum(sgx);
  const float nf = (float)N;
  for (int i = lane; i < N; i += 64) {
    const float diff = xr[i] - mean;
    const float gp = gr[i] * gam[i];
    float v = (gp - sg / nf) / std;
    v -= (diff * sgx) / (nf * std * std);
    dx[(int64_t)r * N + i] = v;
    gx[(int64_t)r * N + i] = gr[i] * (diff / std);
  }
}

// ---------------------------------------------------------------------------
// Causal multi-head attention, one workgroup per (sample, head)
// Q/K/V/O are [B*T, D] with head h in columns [h*hd, (h+1)*hd).
// P [B, NH, T, T] keeps the probabilities for the backward pass.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_fwd_kernel(const float *__restrict__ Q,
                                                       const float *__restrict__ K,
                                                       const float *__restrict__ V,
                                                       float *__restrict__ P,
                                                       float *__restrict__ O, int T, int D,
                                                       int NH, int causal) {
  __shared__ float sq[AT_T * AT_HP], sk[AT_T * AT_HP], sv[AT_T * AT_HP];
  __shared__ float prow[4][AT_T];
  const int b = blockIdx.x / NH, h = blockIdx.x % NH;
  const int hd = D / NH;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int e = threadIdx.x; e < T * hd; e += 256) {
    const int t = e / hd, d = e % hd;
    const int64_t gi = ((int64_t)b * T + t) * D + h * hd + d;
    sq[t * AT_HP + d] = Q[gi];
    sk[t * AT_HP + d] = K[gi];
    sv[t * AT_HP + d] = V[gi];
  }
  __syncthreads();
  const float scale = (float)sqrt((double)hd);
  float *Pb = P + ((int64_t)b * NH + h) * T * T;
  for (int i0 = 0; i0 < T; i0 += 4) {  // uniform trip count: barriers below are legal
    const int i = i0 + w;
    const bool ok = i < T;
    if (ok) {
      // scores (lanes over j), masked entries -1e9 as in the reference
      float mx = -__builtin_inff();
      for (int j = lane; j < T; j += 64) {
        float sc;
        if (causal && j > i) {
          sc = -1e9f;
        } else {
          float dot = 0.f;
          for (int d = 0; d < hd; ++d) dot += sq[i * AT_HP + d] * sk[j * AT_HP + d];
          sc = dot / scale;
        }
        prow[w][j] = sc;
        mx = fmaxf(mx, sc);
      }
      mx = wmax(mx);
      float s = 0.f;
      for (int j = lane; j < T; j += 64) {
        const float e = (float)exp((double)(prow[w][j] - mx));
        prow[w][j] = e;
        s += e;
      }
      s = wsum(s);
      for (int j = lane; j < T; j += 64) {
        const float p = prow[w][j] / s;
        prow[w][j] = p;
        Pb[(int64_t)i * T + j] = p;
      }
    }
    __syncthreads();
    if (ok) {
      for (int d = lane; d < hd; d += 64) {
        float acc = 0.f;
        for (int j = 0; j < T; ++j) acc += prow[w][j] * sv[j * AT_HP + d];
        O[((int64_t)b * T + i) * D + h * hd + d] = acc;
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void attn_bwd_kernel(const float *__restrict__ Q,
                                                       const float *__restrict__ K,
                                                       const float *__restrict__ V,
                                                       const float *__restrict__ P,
                                                       const float *__restrict__ GO,
                                                       float *__restrict__ GQ,
                                                       float *__restrict__ GK,
                                                       float *__restrict__ GV, int T, int D,
                                                       int NH, int causal) {
  __shared__ float sq[AT_T * AT_HP], sk[AT_T * AT_HP], sv[AT_T * AT_HP], sg[AT_T * AT_HP];
  __shared__ float ds[AT_T * (AT_T + 1)];
  const int b = blockIdx.x / NH, h = blockIdx.x % NH;
  const int hd = D / NH;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int TP = AT_T + 1;
  for (int e = threadIdx.x; e < T * hd; e += 256) {
    const int t = e / hd, d = e % hd;
    const int64_t gi = ((int64_t)b * T + t) * D + h * hd + d;
    sq[t * AT_HP + d] = Q[gi];
    sk[t * AT_HP + d] = K[gi];
    sv[t * AT_HP + d] = V[gi];
    sg[t * AT_HP + d] = GO[gi];
  }
  __syncthreads();
  const float scale = (float)sqrt((double)hd);
  const float *Pb = P + ((int64_t)b * NH + h) * T * T;
  // dS rows (one wave per row)
  for (int i = w; i < T; i += 4) {
    float r = 0.f;
    for (int j = lane; j < T; j += 64) {
      float dp = 0.f;
      if (!(causal && j > i))
        for (int d = 0; d < hd; ++d) dp += sg[i * AT_HP + d] * sv[j * AT_HP + d];
      ds[i * TP + j] = dp;
      r += dp * Pb[(int64_t)i * T + j];
    }
    r = wsum(r);
    for (int j = lane; j < T; j += 64) {
      const float p = Pb[(int64_t)i * T + j];
      ds[i * TP + j] = (causal && j > i) ? 0.f : (ds[i * TP + j] * p - p * r) / scale;
    }
  }
  __syncthreads();
  // gQ_i = sum_j dS_ij k_j ; gK_j = sum_i dS_ij q_i ; gV_j = sum_i p_ij gO_i
  for (int e = threadIdx.x; e < T * hd; e += 256) {
    const int t = e / hd, d = e % hd;
    float gq = 0.f, gk = 0.f, gv = 0.f;
    for (int j = 0; j < T; ++j) gq += ds[t * TP + j] * sk[j * AT_HP + d];
    for (int i = 0; i < T; ++i) {
      gk += ds[i * TP + t] * sq[i * AT_HP + d];
      gv += Pb[(int64_t)i * T + t] * sg[i * AT_HP + d];
    }
    const int64_t gi = ((int64_t)b * T + t) * D + h * hd + d;
    GQ[gi] = gq;
    GK[gi] = gk;
    GV[gi] = gv;
  }
}

static unsigned blocks_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 16384) b = 16384;
  return (unsigned)(b < 1 ? 1 : b);
}

hipError_t launch_embed(const float *x, const float *E, int32_t *ids, float *out, int rows, int V,
                        int D, int *err, hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(blocks_for((int64_t)rows * D)), dim3(256), 0, s, x, E, ids,
                     out, rows, V, D, err);
  return hipGetLastError();
}

hipError_t launch_pe_add(const float *x, const float *pe, float *out, int B, int TD, hipStream_t s) {
  const int64_t n = (int64_t)B * TD;
  hipLaunchKernelGGL(pe_add_kernel, dim3(blocks_for(n)), dim3(256), 0, s, x, pe, out, n, TD);
  return hipGetLastError();
}

hipError_t launch_embed_grad(const float *g, const int32_t *ids, float *gradE, int V, int B, int T,
                             int D, int W, float scale, hipStream_t s) {
  hipError_t e = hipMemsetAsync(gradE, 0, (size_t)V * D * sizeof(float), s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(embed_grad_kernel, dim3(1), dim3(256), 0, s, g, ids, gradE, B, T, D, W, scale);
  return hipGetLastError();
}

hipError_t launch_cls_fwd(const float *x, float *out, int B, int TD, int D, hipStream_t s) {
  hipLaunchKernelGGL(cls_fwd_kernel, dim3(blocks_for((int64_t)B * D)), dim3(256), 0, s, x, out, B,
                     TD, D);
  return hipGetLastError();
}

hipError_t launch_cls_bwd(const float *g, float *gin, int B, int TD, int D, hipStream_t s) {
  hipLaunchKernelGGL(cls_bwd_kernel, dim3(blocks_for((int64_t)B * TD)), dim3(256), 0, s, g, gin, B,
                     TD, D);
  return hipGetLastError();
}

hipError_t launch_token_sum(const float *X, float *S, int B, int T, int N, hipStream_t s) {
  hipLaunchKernelGGL(token_sum_kernel, dim3(blocks_for((int64_t)B * N)), dim3(256), 0, s, X, S, B, T,
                     N);
  return hipGetLastError();
}

hipError_t launch_ln_fwd(const float *x, const float *gam, const float *bet, float *y, float *stats,
                         int rows, int N, hipStream_t s) {
  hipLaunchKernelGGL(ln_fwd_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, gam, bet, y, stats,
                     rows, N, 1e-5f);
  return hipGetLastError();
}

hipError_t launch_ln_bwd(const float *g, const float *x, const float *gam, const float *stats,
                         float *dx, float *gx, int rows, int N, hipStream_t s) {
  hipLaunchKernelGGL(ln_bwd_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, g, x, gam, stats, dx, gx,
                     rows, N);
  return hipGetLastError();
}

bool attn_supported(int T, int D, int NH) {
  return NH > 0 && D % NH == 0 && T >= 1 && T <= AT_T && D / NH <= AT_HD;
}

hipError_t launch_attn_fwd(const float *Q, const float *K, const float *V, float *P, float *O, int B,
                           int T, int D, int NH, int causal, hipStream_t s) {
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(B * NH), dim3(256), 0, s, Q, K, V, P, O, T, D, NH, causal);
  return hipGetLastError();
}

hipError_t launch_attn_bwd(const float *Q, const float *K, const float *V, const float *P,
                           const float *GO, float *GQ, float *GK, float *GV, int B, int T, int D,
                           int NH, int causal, hipStream_t s) {
  hipLaunchKernelGGL(attn_bwd_kernel, dim3(B * NH), dim3(256), 0, s, Q, K, V, P, GO, GQ, GK, GV, T, D,
                     NH, causal);
  return hipGetLastError();
}

}  // namespace gn
