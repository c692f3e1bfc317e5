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

// grad[E] = 0 (hipMemsetAsync before the launch), then the token rows of each
// worker chunk's last sample are scatter-added in (chunk, token) order.  Block
// l takes contributing row l: if l is the first row carrying its id it sums,
// in order, every row with that id and writes the row of gradE; rows whose id
// appeared earlier write nothing, so all writes are to distinct rows.
constexpr int EG_MAXL = 2048;  // contributing rows held in LDS

__device__ __forceinline__ int eg_sample(int l, int T, int chunk, int B) {
  return min((l / T + 1) * chunk - 1, B - 1);
}

__global__ __launch_bounds__(256) void embed_grad_kernel(const float *__restrict__ g,
                                                         const int32_t *__restrict__ ids,
                                                         float *__restrict__ gradE, int B, int T,
                                                         int D, int chunk, int L, float scale) {
  __shared__ int sid[EG_MAXL];
  __shared__ int first;
  const int l = blockIdx.x;
  for (int e = threadIdx.x; e < L; e += 256)
    sid[e] = ids[(int64_t)eg_sample(e, T, chunk, B) * T + e % T];
  if (threadIdx.x == 0) first = 1;
  __syncthreads();
  const int my = sid[l];
  for (int e = threadIdx.x; e < l; e += 256)
    if (sid[e] == my) first = 0;  // benign race: every writer stores 0
  __syncthreads();
  if (!first) return;
  for (int d = threadIdx.x; d < D; d += 256) {
    float acc = 0.f;
    for (int e = l; e < L; ++e)
      if (sid[e] == my) acc += g[((int64_t)eg_sample(e, T, chunk, B) * T + e % T) * D + d];
    gradE[(int64_t)my * D + d] = acc * scale;
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
// Block = 64 columns x 4 token groups of sample blockIdx.y; partials added in LDS.
__global__ __launch_bounds__(256) void token_sum_kernel(const float *__restrict__ X,
                                                        float *__restrict__ S, int B, int T, int N) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int64_t b = blockIdx.y;
  float s = 0.f;
  if (c < N) {
    const float *p = X + b * T * N + c;
    for (int t = grp; t < T; t += 4) s += p[(int64_t)t * N];
  }
  red[grp][lane] = s;
  __syncthreads();
  if (grp == 0 && c < N) S[b * N + c] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
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
// Causal multi-head attention on fp32 MFMA, one workgroup per (sample, head).
// Q/K/V/O are [B*T, D] with head h in columns [h*hd, (h+1)*hd); T <= 128 and
// hd <= 32 are held in LDS (zero-padded to 128 x 32).  P [B, NH, T, T] keeps
// the probabilities for the backward pass.  Wave w owns rows [32w, 32w+32) of
// every T x T matrix.  v_mfma_f32_32x32x2_f32 operands: A[m = l%32][k = l/32],
// B[k = l/32][n = l%32]; result register r of lane l is row
// 8*(r/4) + 4*(l/32) + r%4, column l%32.
// ---------------------------------------------------------------------------
typedef float fx16 __attribute__((ext_vector_type(16)));
constexpr int AT_SP = AT_T + 1;  // row pitch of the T x T LDS matrix

__device__ __forceinline__ int mrow(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// row-wise max / sum over the 32 lanes that share lane/32
__device__ __forceinline__ float hmax32(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float hsum32(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Stage rows [0, 128) x cols [0, 32) of head h into LDS (pitch AT_HP), zero padded.
__device__ __forceinline__ void stage_head(float *dst, const float *__restrict__ src, int b, int h,
                                           int T, int D, int hd) {
  for (int e = threadIdx.x; e < AT_T * AT_HD; e += 256) {
    const int t = e / AT_HD, d = e % AT_HD;
    dst[t * AT_HP + d] = (t < T && d < hd) ? src[((int64_t)b * T + t) * D + h * hd + d] : 0.f;
  }
}

// acc += A_rows[32 rows from r0] . B_rows[32 rows from c0]^T over k in [0, kn)
// with A and B both stored [row][k] at pitch AT_HP (S = Q K^T, dP = gO V^T).
__device__ __forceinline__ void mm_nt(fx16 &acc, const float *A, const float *Bm, int r0, int c0,
                                      int kn, int lane) {
  for (int k = 0; k < kn; k += 2) {
    const float a = A[(r0 + (lane & 31)) * AT_HP + k + (lane >> 5)];
    const float b = Bm[(c0 + (lane & 31)) * AT_HP + k + (lane >> 5)];
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
  }
}

__global__ __launch_bounds__(256) void attn_fwd_kernel(const float *__restrict__ Q,
                                                       const float *__restrict__ K,
                                                       const float *__restrict__ V,
                                                       float *__restrict__ P,
                                                       float *__restrict__ O, int T, int D,
                                                       int NH, int causal) {
  __shared__ float sq[AT_T * AT_HP], sk[AT_T * AT_HP], sv[AT_T * AT_HP];
  __shared__ float sp[AT_T * AT_SP];
  const int b = blockIdx.x / NH, h = blockIdx.x % NH;
  const int hd = D / NH;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  stage_head(sq, Q, b, h, T, D, hd);
  stage_head(sk, K, b, h, T, D, hd);
  stage_head(sv, V, b, h, T, D, hd);
  __syncthreads();
  const float scale = (float)sqrt((double)hd);
  const int r0 = 32 * w;
  // scores for the 4 column tiles; fully masked causal tiles are skipped
  fx16 acc[4];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    acc[jt] = fx16{};
    if (!(causal && jt > w)) mm_nt(acc[jt], sq, sk, r0, 32 * jt, hd + (hd & 1), lane);
  }
  // row softmax: -1e9 on causal-masked entries (as the reference), columns
  // >= T do not exist; exp in float64 (activations.go:161-183)
  const int cl = lane & 31;
  float mx[16], sum[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) mx[r] = -__builtin_inff();
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = r0 + mrow(r, lane), j = 32 * jt + cl;
      float sc;
      if (j >= T) sc = -__builtin_inff();
      else if (causal && j > i) sc = -1e9f;
      else sc = acc[jt][r] / scale;
      acc[jt][r] = sc;
      mx[r] = fmaxf(mx[r], sc);
    }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    mx[r] = hmax32(mx[r]);
    sum[r] = 0.f;
  }
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = 32 * jt + cl;
      const float e = j < T ? (float)exp((double)(acc[jt][r] - mx[r])) : 0.f;
      acc[jt][r] = e;
      sum[r] += e;
    }
#pragma unroll
  for (int r = 0; r < 16; ++r) sum[r] = hsum32(sum[r]);
  float *Pb = P + ((int64_t)b * NH + h) * T * T;
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = r0 + mrow(r, lane), j = 32 * jt + cl;
      const float p = acc[jt][r] / sum[r];
      sp[i * AT_SP + j] = p;
      if (i < T && j < T) Pb[(int64_t)i * T + j] = p;
    }
  __syncthreads();
  // O = P V over j < min(T, rows of this wave + 1 under the causal mask)
  fx16 o = fx16{};
  const int kend = causal ? min(T, r0 + 32) : T;
  for (int j = 0; j < kend; j += 2) {
    const float a = sp[(r0 + (lane & 31)) * AT_SP + j + (lane >> 5)];
    const float bv = sv[(j + (lane >> 5)) * AT_HP + (lane & 31)];
    o = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bv, o, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = r0 + mrow(r, lane), d = cl;
    if (i < T && d < hd) O[((int64_t)b * T + i) * D + h * hd + d] = o[r];
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
  __shared__ float sp[AT_T * AT_SP];  // P, then dS
  const int b = blockIdx.x / NH, h = blockIdx.x % NH;
  const int hd = D / NH;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int cl = lane & 31;
  stage_head(sq, Q, b, h, T, D, hd);
  stage_head(sk, K, b, h, T, D, hd);
  stage_head(sv, V, b, h, T, D, hd);
  stage_head(sg, GO, b, h, T, D, hd);
  const float *Pb = P + ((int64_t)b * NH + h) * T * T;
  for (int e = threadIdx.x; e < AT_T * AT_T; e += 256) {
    const int i = e / AT_T, j = e % AT_T;
    sp[i * AT_SP + j] = (i < T && j < T) ? Pb[(int64_t)i * T + j] : 0.f;
  }
  __syncthreads();
  const float scale = (float)sqrt((double)hd);
  const int r0 = 32 * w;
  const int kpad = hd + (hd & 1);
  auto store = [&](float *G, const fx16 &v) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = r0 + mrow(r, lane), d = cl;
      if (t < T && d < hd) G[((int64_t)b * T + t) * D + h * hd + d] = v[r];
    }
  };
  // gV_j = sum_i p_ij gO_i  (rows j of this wave; p_ij = 0 for i < j when causal)
  {
    fx16 acc = fx16{};
    for (int i = causal ? r0 : 0; i < T; i += 2) {
      const float a = sp[(i + (lane >> 5)) * AT_SP + r0 + (lane & 31)];
      const float bv = sg[(i + (lane >> 5)) * AT_HP + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bv, acc, 0, 0, 0);
    }
    store(GV, acc);
  }
  // dP_ij = gO_i . v_j ; r_i = sum_j dP_ij p_ij ; dS = (dP p - p r) / sqrt(hd)
  fx16 dp[4];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    dp[jt] = fx16{};
    if (!(causal && jt > w)) mm_nt(dp[jt], sg, sv, r0, 32 * jt, kpad, lane);
  }
  float rs[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) rs[r] = 0.f;
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = r0 + mrow(r, lane), j = 32 * jt + cl;
      const bool live = j < T && !(causal && j > i);
      if (!live) dp[jt][r] = 0.f;
      rs[r] += dp[jt][r] * sp[i * AT_SP + j];
    }
#pragma unroll
  for (int r = 0; r < 16; ++r) rs[r] = hsum32(rs[r]);
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = r0 + mrow(r, lane), j = 32 * jt + cl;
      const bool live = j < T && !(causal && j > i);
      const float p = sp[i * AT_SP + j];
      dp[jt][r] = live ? (dp[jt][r] * p - p * rs[r]) / scale : 0.f;
    }
  __syncthreads();  // every wave has read P (gV and r): overwrite it with dS
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 16; ++r) sp[(r0 + mrow(r, lane)) * AT_SP + 32 * jt + cl] = dp[jt][r];
  __syncthreads();
  // gQ_i = sum_j dS_ij k_j  (j <= i when causal)
  {
    fx16 acc = fx16{};
    const int kend = causal ? min(T, r0 + 32) : T;
    for (int j = 0; j < kend; j += 2) {
      const float a = sp[(r0 + (lane & 31)) * AT_SP + j + (lane >> 5)];
      const float bv = sk[(j + (lane >> 5)) * AT_HP + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bv, acc, 0, 0, 0);
    }
    store(GQ, acc);
  }
  // gK_j = sum_i dS_ij q_i  (i >= j when causal)
  {
    fx16 acc = fx16{};
    for (int i = causal ? r0 : 0; i < T; i += 2) {
      const float a = sp[(i + (lane >> 5)) * AT_SP + r0 + (lane & 31)];
      const float bv = sq[(i + (lane >> 5)) * AT_HP + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bv, acc, 0, 0, 0);
    }
    store(GK, acc);
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
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  const int chunk = (B + Wc - 1) / Wc;
  const int nsamp = (B + chunk - 1) / chunk;  // one contributing sample per chunk
  const int L = nsamp * T;
  if (L > EG_MAXL) return hipErrorInvalidValue;
  hipError_t e = hipMemsetAsync(gradE, 0, (size_t)V * D * sizeof(float), s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(embed_grad_kernel, dim3(L), dim3(256), 0, s, g, ids, gradE, B, T, D, chunk, L,
                     scale);
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
  hipLaunchKernelGGL(token_sum_kernel, dim3((N + 63) / 64, B), dim3(256), 0, s, X, S, B, T, N);
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
