// SequenceUnroller(LSTM) training kernels (unroller.go:57-213, lstm.go).
//
// Reference semantics kept (the quirks are the oracle's, see lstm.go):
//  - only the input-gate rows get Wx x + Wh h; f, g, o pre-activations are
//    their biases (the gate helpers run over outSize rows, lstm.go:319-326,
//    1065-1101);
//  - backward per step: dc = dh*o*(1-tanh^2 c) + dcNext, gate deltas, dcNext =
//    dc*f, dhPrev = Wh^T dG added to the running dh (lstm.go:556-691,
//    unroller.go:190-209);
//  - dWx uses the last forward step's input for every step (lstm.go:594-618);
//  - after every backward step the worker's cumulative LSTM gradient is
//    clipped to L2 norm <= 1 (lstm.go:693-751).
//
// GPU formulation.  The BPTT recursion of the deltas does not depend on the
// accumulated gradient, so it runs first (one workgroup per sample), storing
// dG_t.  The clip sequence G <- clip(G + D_t) of a worker chain is then solved
// exactly through the Gram matrix of its contributions,
//   <D_u, D_v> = (dG_u . dG_v) * (x_u . x_v + h_u . h_v + 1)
// (each contribution is the outer product of dG with [x_last | hPrev | 1]),
// which yields scalar weights w_t with G_final = sum_t w_t D_t.  The weighted
// gradients are then three GEMMs / column sums: dWx = (sum_t w dG) x_last^T,
// dWh = (w dG)^T hPrev, db = sum w dG.
#include "gn_common.h"

namespace gn {

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + (float)exp((double)(-x))); }
__device__ __forceinline__ float tanh32(float x) { return (float)tanh((double)x); }

// out[c][r] = in[r][c] for r < rows, c < cols (tiled through LDS)
__global__ __launch_bounds__(256) void transpose_kernel(const float *__restrict__ in,
                                                        float *__restrict__ out, int rows,
                                                        int cols) {
  __shared__ float tile[32][33];
  const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int j = ty; j < 32; j += 8) {
    const int r = by + j, c = bx + tx;
    if (r < rows && c < cols) tile[j][tx] = in[(size_t)r * cols + c];
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    const int c = bx + j, r = by + tx;
    if (c < cols && r < rows) out[(size_t)c * rows + r] = tile[tx][j];
  }
}

// Forward over T steps, one workgroup per sample, thread i = hidden unit i.
// WxT [I][H] and WhT [H][H] are the transposed input-gate blocks.
// Saves pre_i [B][T][H], c [B][T][H], hbuf [B][T+1][H] (hbuf[b][0] = 0,
// hbuf[b][t+1] = h_t) and writes h_{T-1} to out [B][H].
__global__ void lstm_fwd_kernel(const float *__restrict__ x, const float *__restrict__ WxT,
                                const float *__restrict__ WhT, const float *__restrict__ bias,
                                float *__restrict__ pre_i, float *__restrict__ cbuf,
                                float *__restrict__ hbuf, float *__restrict__ out, int T, int I,
                                int H) {
  extern __shared__ float sm[];
  float *hs = sm, *xs = sm + H;
  const int b = blockIdx.x, i = threadIdx.x;
  const bool act = i < H;
  const float *xb = x + (size_t)b * T * I;
  float bi = 0.f, fg = 0.f, gg = 0.f, og = 0.f;
  if (act) {
    hs[i] = 0.f;
    hbuf[(size_t)b * (T + 1) * H + i] = 0.f;
    bi = bias[i];
    fg = sigm(bias[H + i]);       // Q13: f, g, o pre-activations are the biases
    gg = tanh32(bias[2 * H + i]);
    og = sigm(bias[3 * H + i]);
  }
  float c = 0.f, hnew = 0.f;
  for (int t = 0; t < T; ++t) {
    for (int j = i; j < I; j += blockDim.x) xs[j] = xb[(size_t)t * I + j];
    __syncthreads();
    if (act) {
      float a = bi;
      if (I >= 64) {  // lstmComputeInputGates: direct accumulation
        for (int j = 0; j < I; ++j) a += WxT[(size_t)j * H + i] * xs[j];
      } else {        // lstmComputeInputGatesUnrolled4x: sum, then add
        float s = 0.f;
        for (int j = 0; j < I; ++j) s += WxT[(size_t)j * H + i] * xs[j];
        a += s;
      }
      for (int j = 0; j < H; ++j) a += WhT[(size_t)j * H + i] * hs[j];
      const size_t o = ((size_t)b * T + t) * H + i;
      pre_i[o] = a;
      const float ig = sigm(a);
      c = fg * c + ig * gg;
      hnew = og * tanh32(c);
      cbuf[o] = c;
      hbuf[((size_t)b * (T + 1) + t + 1) * H + i] = hnew;
    }
    __syncthreads();
    if (act) hs[i] = hnew;
  }
  if (act) out[(size_t)b * H + i] = hnew;
}

// BPTT deltas, one workgroup per sample.  gh = dL/dh_{T-1} [B][H].
// D [B][T+1][4H]: row t = (dI, dF, dC, dO) of step t; row T = 0 (padding that
// lines D up with hbuf for the dWh GEMM).
__global__ void lstm_bwd_kernel(const float *__restrict__ gh, const float *__restrict__ pre_i,
                                const float *__restrict__ cbuf, const float *__restrict__ Wh,
                                const float *__restrict__ bias, float *__restrict__ D, int T,
                                int H) {
  extern __shared__ float dG[];  // 4H
  const int b = blockIdx.x, i = threadIdx.x;
  const bool act = i < H;
  const int G4 = 4 * H;
  float *Db = D + (size_t)b * (T + 1) * G4;
  for (int k = i; k < G4; k += blockDim.x) Db[(size_t)T * G4 + k] = 0.f;
  float cur = act ? gh[(size_t)b * H + i] : 0.f, dcn = 0.f;
  float fg = 0.f, gg = 0.f, og = 0.f, dfd = 0.f, dgd = 0.f, dod = 0.f;
  if (act) {
    fg = sigm(bias[H + i]);
    gg = tanh32(bias[2 * H + i]);
    og = sigm(bias[3 * H + i]);
    dfd = fg * (1.0f - fg);   // Sigmoid.Derivative(pre_f) recomputes sigmoid(pre_f)
    dgd = 1.0f - gg * gg;     // Tanh.Derivative
    dod = og * (1.0f - og);
  }
  for (int t = T - 1; t >= 0; --t) {
    if (act) {
      const size_t o = ((size_t)b * T + t) * H + i;
      const float ig = sigm(pre_i[o]);
      const float did = ig * (1.0f - ig);
      const float ct = cbuf[o];
      const float cp = t > 0 ? cbuf[o - H] : 0.f;
      const float tc = tanh32(ct);
      const float dc = cur * og * (1 - tc * tc) + dcn;
      const float dI = dc * gg * did;
      const float dF = dc * cp * dfd;
      const float dC = dc * ig * dgd;
      const float dO = cur * tc * dod;
      dcn = dc * fg;
      dG[i] = dI;
      dG[H + i] = dF;
      dG[2 * H + i] = dC;
      dG[3 * H + i] = dO;
      float *row = Db + (size_t)t * G4;
      row[i] = dI;
      row[H + i] = dF;
      row[2 * H + i] = dC;
      row[3 * H + i] = dO;
    }
    __syncthreads();
    if (act) {
      float s = 0.f;  // dhPrev = Wh^T dG, gates then units in order
      for (int k = 0; k < G4; ++k) s += Wh[(size_t)k * H + i] * dG[k];
      cur += s;
    }
    __syncthreads();
  }
}

// Contribution u of chain ch: sample b = b0 + u / T, backward step t = T-1 - u % T.
struct ChainMap {
  int T, chunk, B;
  __device__ __forceinline__ void at(int ch, int u, int &b, int &t) const {
    b = ch * chunk + u / T;
    t = T - 1 - u % T;
  }
  __device__ __forceinline__ int len(int ch) const {
    const int s0 = ch * chunk, s1 = min(B, s0 + chunk);
    return s1 > s0 ? (s1 - s0) * T : 0;
  }
};

// Lower-triangular Gram of one chain, Gm[ch][v][u] (u <= v), in double:
// <D_u, D_v> = (dG_u . dG_v) * (x_u . x_v + h_u . h_v + 1).
// Block = 16x16 entries, LDS tiles of 32 k.
__global__ __launch_bounds__(256) void lstm_gram_kernel(const float *__restrict__ D,
                                                        const float *__restrict__ hbuf,
                                                        const float *__restrict__ x,
                                                        double *__restrict__ Gm, ChainMap cm,
                                                        int I, int H, int nmax) {
  __shared__ float su[16][33], sv[16][33];
  const int ch = blockIdx.y;
  const int n = cm.len(ch);
  // tile (tv, tu) with tu <= tv from the linear block index
  int lin = blockIdx.x, tv = 0;
  while (lin > tv) {
    lin -= tv + 1;
    ++tv;
  }
  const int tu = lin;
  const int ntile = (n + 15) / 16;
  if (tv >= ntile) return;
  const int r = threadIdx.x >> 4, s = threadIdx.x & 15;
  const int v = tv * 16 + r, u = tu * 16 + s;
  const int G4 = 4 * H;
  double acc[3] = {0.0, 0.0, 0.0};
  // segments: 0 = dG (4H), 1 = hPrev (H), 2 = x_last (I)
  for (int seg = 0; seg < 3; ++seg) {
    const int K = seg == 0 ? G4 : (seg == 1 ? H : I);
    for (int k0 = 0; k0 < K; k0 += 32) {
      // load 16 rows x 32 k for the v-rows and the u-rows
      for (int e = threadIdx.x; e < 2 * 16 * 32; e += 256) {
        const int which = e / 512, rr = (e / 32) % 16, kk = e % 32;
        const int idx = (which ? tv : tu) * 16 + rr;
        float val = 0.f;
        if (idx < n && k0 + kk < K) {
          int bb, tt;
          cm.at(ch, idx, bb, tt);
          if (seg == 0)
            val = D[((size_t)bb * (cm.T + 1) + tt) * G4 + k0 + kk];
          else if (seg == 1)
            val = hbuf[((size_t)bb * (cm.T + 1) + tt) * H + k0 + kk];
          else
            val = x[((size_t)bb * cm.T + cm.T - 1) * I + k0 + kk];
        }
        if (which) sv[rr][kk] = val;
        else su[rr][kk] = val;
      }
      __syncthreads();
      double a = 0.0;
#pragma unroll 8
      for (int kk = 0; kk < 32; ++kk) a += (double)sv[r][kk] * (double)su[s][kk];
      acc[seg] += a;
      __syncthreads();
    }
  }
  if (v < n && u <= v && u < n)
    Gm[(size_t)ch * nmax * nmax + (size_t)v * nmax + u] = acc[0] * (acc[2] + acc[1] + 1.0);
}

// Sequential clip of one chain from its Gram matrix; one workgroup per chain.
// w_u = P * a_u; at step v: N^2 = |G|^2 + 2 P sum_{u<v} a_u <D_u,D_v> + <D_v,D_v>,
// c = N > 1 ? 1/N : 1 (clipGradients), P *= c, a_v = c / P, |G|^2 = c^2 N^2.
__global__ __launch_bounds__(256) void lstm_clip_kernel(const double *__restrict__ Gm,
                                                        double *__restrict__ a,
                                                        float *__restrict__ w, ChainMap cm,
                                                        int nmax) {
  __shared__ double red[4];
  const int ch = blockIdx.x;
  const int n = cm.len(ch);
  const double *G = Gm + (size_t)ch * nmax * nmax;
  double *ac = a + (size_t)ch * nmax;
  double P = 1.0, nrm2 = 0.0;
  for (int v = 0; v < n; ++v) {
    const double *row = G + (size_t)v * nmax;
    double s = 0.0;
    for (int u = threadIdx.x; u < v; u += 256) s += ac[u] * row[u];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    const double N2 = nrm2 + 2.0 * P * s + row[v];
    const double N = sqrt(N2 > 0.0 ? N2 : 0.0);
    const double c = N > 1.0 ? 1.0 / N : 1.0;
    P *= c;
    if (threadIdx.x == 0) ac[v] = c / P;
    nrm2 = c * c * N2;
    if (P < 1e-200) {  // fold P into the coefficients before it underflows
      __syncthreads();
      for (int u = threadIdx.x; u <= v; u += 256) ac[u] *= P;
      P = 1.0;
    }
    __syncthreads();
  }
  for (int u = threadIdx.x; u < n; u += 256) {
    int b, t;
    cm.at(ch, u, b, t);
    w[(size_t)b * (cm.T + 1) + t] = (float)(P * ac[u]);
  }
}

// D[b][t][:] *= w[b][t];  S[b][k] = sum_t D[b][t][k]  (t < T)
__global__ __launch_bounds__(256) void lstm_weight_kernel(float *__restrict__ D,
                                                          const float *__restrict__ w,
                                                          float *__restrict__ S, int B, int T,
                                                          int G4) {
  const int64_t n = (int64_t)B * G4;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int b = (int)(e / G4), k = (int)(e % G4);
    float s = 0.f;
    for (int t = T - 1; t >= 0; --t) {
      float *p = D + ((size_t)b * (T + 1) + t) * G4 + k;
      const float d = *p * w[(size_t)b * (T + 1) + t];
      *p = d;
      s += d;
    }
    S[(size_t)b * G4 + k] = s;
  }
}

hipError_t launch_transpose(const float *in, float *out, int rows, int cols, hipStream_t s) {
  dim3 g((cols + 31) / 32, (rows + 31) / 32);
  hipLaunchKernelGGL(transpose_kernel, g, dim3(256), 0, s, in, out, rows, cols);
  return hipGetLastError();
}

static int lstm_block(int H) { return ((H + 63) / 64) * 64; }

hipError_t launch_lstm_fwd(const float *x, const float *WxT, const float *WhT, const float *bias,
                           float *pre_i, float *cbuf, float *hbuf, float *out, int B, int T, int I,
                           int H, hipStream_t s) {
  const size_t shm = (size_t)(H + I) * sizeof(float);
  hipLaunchKernelGGL(lstm_fwd_kernel, dim3(B), dim3(lstm_block(H)), shm, s, x, WxT, WhT, bias, pre_i,
                     cbuf, hbuf, out, T, I, H);
  return hipGetLastError();
}

hipError_t launch_lstm_bwd(const float *gh, const float *pre_i, const float *cbuf, const float *Wh,
                           const float *bias, float *D, int B, int T, int H, hipStream_t s) {
  const size_t shm = (size_t)4 * H * sizeof(float);
  hipLaunchKernelGGL(lstm_bwd_kernel, dim3(B), dim3(lstm_block(H)), shm, s, gh, pre_i, cbuf, Wh,
                     bias, D, T, H);
  return hipGetLastError();
}

hipError_t launch_lstm_clip_weights(const float *D, const float *hbuf, const float *x, double *gram,
                                    double *coef, float *w, int B, int T, int I, int H, int W,
                                    hipStream_t s) {
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  ChainMap cm{T, (B + Wc - 1) / Wc, B};
  const int nchains = (B + cm.chunk - 1) / cm.chunk;
  const int nmax = cm.chunk * T;
  const int ntile = (nmax + 15) / 16;
  dim3 g(ntile * (ntile + 1) / 2, nchains);
  hipLaunchKernelGGL(lstm_gram_kernel, g, dim3(256), 0, s, D, hbuf, x, gram, cm, I, H, nmax);
  hipLaunchKernelGGL(lstm_clip_kernel, dim3(nchains), dim3(256), 0, s, gram, coef, w, cm, nmax);
  return hipGetLastError();
}

hipError_t launch_lstm_weight(float *D, const float *w, float *S, int B, int T, int H,
                              hipStream_t s) {
  const int64_t n = (int64_t)B * 4 * H;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(lstm_weight_kernel, dim3((unsigned)blocks), dim3(256), 0, s, D, w, S, B, T,
                     4 * H);
  return hipGetLastError();
}

}  // namespace gn
