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

#include <atomic>

namespace gn {

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) holds per device and per
// kernel.  set[d] is the largest size already set on device d for one kernel:
// a later launch that needs more LDS (a larger H) sets it again.
static constexpr int kAttrDevices = 64;
static hipError_t ensure_lds_attr(const void *fn, int bytes, std::atomic<int> (&set)[kAttrDevices]) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kAttrDevices) return hipErrorInvalidDevice;
  if (set[dev].load(std::memory_order_relaxed) >= bytes) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return e;
  int cur = set[dev].load(std::memory_order_relaxed);
  while (cur < bytes && !set[dev].compare_exchange_weak(cur, bytes)) {
  }
  return hipSuccess;
}

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

// s = sum_{j0 <= j < j1} W[j * stride] * v[j], with U loads issued together
// (the weights come from L2 every step; batching them hides its latency).
template <int U>
__device__ __forceinline__ float dot_strided(const float *__restrict__ W, int stride,
                                             const float *v, int j0, int j1) {
  float s = 0.f;
  int j = j0;
  for (; j + U <= j1; j += U) {
    float w[U];
#pragma unroll
    for (int e = 0; e < U; ++e) w[e] = W[(size_t)(j + e) * stride];
#pragma unroll
    for (int e = 0; e < U; ++e) s += w[e] * v[j + e];
  }
  for (; j < j1; ++j) s += W[(size_t)j * stride] * v[j];
  return s;
}

// The same for four consecutive columns at once (16-byte loads: a CU streams
// L2-resident weights about twice as fast with dwordx4 as with dword loads).
template <int U>
__device__ __forceinline__ float4 dot4_strided(const float4 *__restrict__ W, int stride4,
                                               const float *v, int j0, int j1) {
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  int j = j0;
  for (; j + U <= j1; j += U) {
    float4 w[U];
#pragma unroll
    for (int e = 0; e < U; ++e) w[e] = W[(size_t)(j + e) * stride4];
#pragma unroll
    for (int e = 0; e < U; ++e) {
      const float x = v[j + e];
      s.x += w[e].x * x;
      s.y += w[e].y * x;
      s.z += w[e].z * x;
      s.w += w[e].w * x;
    }
  }
  for (; j < j1; ++j) {
    const float4 w = W[(size_t)j * stride4];
    const float x = v[j];
    s.x += w.x * x;
    s.y += w.y * x;
    s.z += w.z * x;
    s.w += w.w * x;
  }
  return s;
}

// Recurrent mat-vec of one step: part[q][c] = sum over the q-th share of k of
// W[k][c] * v[k] (W is K x H row-major).  V4: thread (g, q) owns columns
// 4g..4g+3 (H % 4 == 0, W 16-byte aligned); otherwise thread (i, q) owns
// column i.  GB = threads per share (a multiple of 64), NQ shares.  Shares
// q < QL read their rows from Wl, a copy of W's leading rows in LDS (the rest
// stream from L2 every step).
template <bool V4>
__device__ __forceinline__ void step_matvec(const float *__restrict__ W, const float *Wl, int QL,
                                            const float *v, int K, int H, int GB, int NQ,
                                            float *part) {
  const int c = threadIdx.x % GB, q = threadIdx.x / GB;
  if (q >= NQ) return;
  const int k0 = (K * q) / NQ, k1 = (K * (q + 1)) / NQ;
  if (V4) {
    if (4 * c < H) {
      const float4 s = q < QL ? dot4_strided<16>(reinterpret_cast<const float4 *>(Wl) + c, H / 4, v, k0, k1)
                              : dot4_strided<16>(reinterpret_cast<const float4 *>(W) + c, H / 4, v, k0, k1);
      *reinterpret_cast<float4 *>(part + q * H + 4 * c) = s;
    }
  } else if (c < H) {
    part[q * H + c] = q < QL ? dot_strided<32>(Wl + c, H, v, k0, k1) : dot_strided<32>(W + c, H, v, k0, k1);
  }
}

// Forward over T steps, one workgroup per sample.  xw [B][T][H] holds the
// input-gate x projections x_t . Wx_i (one GEMM before the recurrence), so a
// step only needs Wh_i h_{t-1}, split over NQ shares of j and summed in LDS.
// WhT [H][H] is the transposed input-gate block of Wh.  Thread i < H owns
// hidden unit i's state.
// Saves ig = sigmoid(pre_i), tc = tanh(c), c [B][T][H] and hbuf [B][T+1][H]
// (hbuf[b][0] = 0, hbuf[b][t+1] = h_t), and writes h_{T-1} to out [B][H].
template <bool V4>
__global__ __launch_bounds__(1024) void lstm_fwd_kernel(const float *__restrict__ xw,
                                                        const float *__restrict__ WhT,
                                                        const float *__restrict__ bias,
                                                        float *__restrict__ igb,
                                                        float *__restrict__ tcb,
                                                        float *__restrict__ cbuf,
                                                        float *__restrict__ hbuf,
                                                        float *__restrict__ out, int T, int H,
                                                        int GB, int NQ, int QL, int seq) {
  extern __shared__ float sm[];
  float *hs = sm, *part = sm + ((H + 3) & ~3);  // part[NQ][H], 16-byte aligned
  float *Wl = part + NQ * H;                    // WhT rows [0, H*QL/NQ), 16-byte aligned
  {
    const int nl = (H * QL / NQ) * H;
    for (int e = threadIdx.x * 4; e < nl; e += blockDim.x * 4)
      *reinterpret_cast<float4 *>(Wl + e) = *reinterpret_cast<const float4 *>(WhT + e);
  }
  const int b = blockIdx.x;
  const int i = threadIdx.x;
  const bool own = i < H;
  const float *xwb = xw + (size_t)b * T * H;
  float bi = 0.f, fg = 0.f, gg = 0.f, og = 0.f, xwn = 0.f;
  if (own) {
    hs[i] = 0.f;
    hbuf[(size_t)b * (T + 1) * H + i] = 0.f;
    bi = bias[i];
    fg = sigm(bias[H + i]);       // Q13: f, g, o pre-activations are the biases
    gg = tanh32(bias[2 * H + i]);
    og = sigm(bias[3 * H + i]);
    xwn = xwb[i];
  }
  __syncthreads();
  float c = 0.f, hnew = 0.f;
  for (int t = 0; t < T; ++t) {
    const float xwc = xwn;
    if (own && t + 1 < T) xwn = xwb[(size_t)(t + 1) * H + i];  // next step's, in flight
    step_matvec<V4>(WhT, Wl, QL, hs, H, H, GB, NQ, part);
    __syncthreads();
    if (own) {
      float sh = 0.f;
      for (int r = 0; r < NQ; ++r) sh += part[r * H + i];
      const float a = (bi + xwc) + sh;  // bias, then Wx x, then Wh h (lstm.go:1065-1101)
      const size_t o = ((size_t)b * T + t) * H + i;
      const float ig = sigm(a);
      c = fg * c + ig * gg;
      const float tc = tanh32(c);
      hnew = og * tc;
      igb[o] = ig;
      tcb[o] = tc;
      cbuf[o] = c;
      hbuf[((size_t)b * (T + 1) + t + 1) * H + i] = hnew;
      hs[i] = hnew;
      if (seq) out[((size_t)b * T + t) * H + i] = hnew;  // returnSequences: every state
    }
    __syncthreads();
  }
  if (own && !seq) out[(size_t)b * H + i] = hnew;
}

// The same recurrence with each thread's share of WhT in registers for the
// whole sequence (at most LF_R rows x 4 columns per thread: H <= 256), so a
// step reads no weights at all; the products are summed in the order
// lstm_fwd_kernel uses, so the results are the same bit for bit.
constexpr int LF_R = 16;
__global__ __launch_bounds__(1024) void lstm_fwd_reg_kernel(const float *__restrict__ xw,
                                                            const float *__restrict__ WhT,
                                                            const float *__restrict__ bias,
                                                            float *__restrict__ igb,
                                                            float *__restrict__ tcb,
                                                            float *__restrict__ cbuf,
                                                            float *__restrict__ hbuf,
                                                            float *__restrict__ out, int T, int H,
                                                            int GB, int NQ, int seq) {
  extern __shared__ float sm[];
  float *hs = sm, *part = sm + ((H + 3) & ~3);  // part[NQ][H], 16-byte aligned
  const int b = blockIdx.x;
  const int i = threadIdx.x;
  const int c = i % GB, q = i / GB;
  const bool mv = q < NQ && 4 * c < H;
  const int k0 = mv ? (H * q) / NQ : 0;
  const int nk = mv ? (H * (q + 1)) / NQ - k0 : 0;  // <= LF_R (checked by the launcher)
  float4 wr[LF_R];
#pragma unroll
  for (int e = 0; e < LF_R; ++e)
    wr[e] = e < nk ? reinterpret_cast<const float4 *>(WhT)[(size_t)(k0 + e) * (H / 4) + c]
                   : make_float4(0.f, 0.f, 0.f, 0.f);
  const bool own = i < H;
  const float *xwb = xw + (size_t)b * T * H;
  float bi = 0.f, fg = 0.f, gg = 0.f, og = 0.f, xwn = 0.f;
  if (own) {
    hs[i] = 0.f;
    hbuf[(size_t)b * (T + 1) * H + i] = 0.f;
    bi = bias[i];
    fg = sigm(bias[H + i]);       // Q13: f, g, o pre-activations are the biases
    gg = tanh32(bias[2 * H + i]);
    og = sigm(bias[3 * H + i]);
    xwn = xwb[i];
  }
  __syncthreads();
  float cc = 0.f, hnew = 0.f;
  for (int t = 0; t < T; ++t) {
    const float xwc = xwn;
    if (own && t + 1 < T) xwn = xwb[(size_t)(t + 1) * H + i];  // next step's, in flight
    if (mv) {
      float4 sacc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int e = 0; e < LF_R; ++e)
        if (e < nk) {
          const float x = hs[k0 + e];
          sacc.x += wr[e].x * x;
          sacc.y += wr[e].y * x;
          sacc.z += wr[e].z * x;
          sacc.w += wr[e].w * x;
        }
      *reinterpret_cast<float4 *>(part + q * H + 4 * c) = sacc;
    }
    __syncthreads();
    if (own) {
      float sh = 0.f;
      for (int r = 0; r < NQ; ++r) sh += part[r * H + i];
      const float a = (bi + xwc) + sh;  // bias, then Wx x, then Wh h (lstm.go:1065-1101)
      const size_t o = ((size_t)b * T + t) * H + i;
      const float ig = sigm(a);
      cc = fg * cc + ig * gg;
      const float tc = tanh32(cc);
      hnew = og * tc;
      igb[o] = ig;
      tcb[o] = tc;
      cbuf[o] = cc;
      hbuf[((size_t)b * (T + 1) + t + 1) * H + i] = hnew;
      hs[i] = hnew;
      if (seq) out[((size_t)b * T + t) * H + i] = hnew;  // returnSequences: every state
    }
    __syncthreads();
  }
  if (own && !seq) out[(size_t)b * H + i] = hnew;
}

// BPTT deltas, one workgroup per sample.  gh = dL/dh_{T-1} [B][H].
// D [B][T+1][4H]: row t = (dI, dF, dC, dO) of step t; row T = 0 (padding that
// lines D up with hbuf for the dWh GEMM).  dhPrev = Wh^T dG is split over NQ
// shares of the 4H rows and summed in LDS; the saved gate values of step t-1
// are fetched while step t runs.  Thread i < H owns hidden unit i.
template <bool V4>
__global__ __launch_bounds__(1024) void lstm_bwd_kernel(const float *__restrict__ gh,
                                                        const float *__restrict__ igb,
                                                        const float *__restrict__ tcb,
                                                        const float *__restrict__ cbuf,
                                                        const float *__restrict__ Wh,
                                                        const float *__restrict__ bias,
                                                        float *__restrict__ D, int T, int H,
                                                        int GB, int NQ, int seq) {
  extern __shared__ float dG[];  // 4H, then part[NQ][H]
  float *part = dG + 4 * H;
  const int b = blockIdx.x;
  const int i = threadIdx.x;
  const bool own = i < H;
  const int G4 = 4 * H;
  float *Db = D + (size_t)b * (T + 1) * G4;
  for (int k = threadIdx.x; k < G4; k += blockDim.x) Db[(size_t)T * G4 + k] = 0.f;
  // gh: dL/dh_{T-1} [B][H], or with seq (returnSequences) dL/dh_t [B][T][H],
  // added to the carried gradient at every step (unroller.go:192-198)
  const size_t ob = (size_t)b * T * H + i;
  float cur = own ? (seq ? gh[ob + (size_t)(T - 1) * H] : gh[(size_t)b * H + i]) : 0.f, dcn = 0.f;
  float fg = 0.f, gg = 0.f, og = 0.f, dfd = 0.f, dgd = 0.f, dod = 0.f;
  float ign = 0.f, tcn = 0.f, cpn = 0.f, gsn = 0.f;  // step t's saved values, fetched one step early
  if (own) {
    fg = sigm(bias[H + i]);
    gg = tanh32(bias[2 * H + i]);
    og = sigm(bias[3 * H + i]);
    dfd = fg * (1.0f - fg);   // Sigmoid.Derivative(pre_f) recomputes sigmoid(pre_f)
    dgd = 1.0f - gg * gg;     // Tanh.Derivative
    dod = og * (1.0f - og);
    ign = igb[ob + (size_t)(T - 1) * H];
    tcn = tcb[ob + (size_t)(T - 1) * H];
    cpn = T > 1 ? cbuf[ob + (size_t)(T - 2) * H] : 0.f;
  }
  for (int t = T - 1; t >= 0; --t) {
    if (own) {
      const float ig = ign, tc = tcn, cp = cpn;
      if (seq && t < T - 1) cur += gsn;
      if (t > 0) {
        ign = igb[ob + (size_t)(t - 1) * H];
        tcn = tcb[ob + (size_t)(t - 1) * H];
        cpn = t > 1 ? cbuf[ob + (size_t)(t - 2) * H] : 0.f;
        if (seq) gsn = gh[ob + (size_t)(t - 1) * H];
      }
      const float did = ig * (1.0f - ig);
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
    step_matvec<V4>(Wh, nullptr, 0, dG, G4, H, GB, NQ, part);
    __syncthreads();
    if (own) {
      float s = 0.f;
      for (int r = 0; r < NQ; ++r) s += part[r * H + i];
      cur += s;
    }
  }
}

// Cooperative BPTT (H = 32, 64, 128 or 256, B <= 64): the per-sample
// recurrence of lstm_bwd_kernel is bound by every step re-reading the 4H x H
// recurrent weights from L2 into one CU (1 MB per step at H = 256).  Here a
// group of LC_KM workgroups shares LC_SPG samples; member m keeps columns
// [m*U, (m+1)*U) of Wh (U = H / LC_KM) in LDS for the whole sequence, owns
// those hidden units' state and gate deltas, and computes their dhPrev from
// the group's full dG.  Per step each member publishes its units' dG through
// an exchange buffer (double-buffered by step parity) whose 64-bit words hold
// a value and the step's tag together; a reader polls the words it needs
// until each carries the step's tag.  Value and tag are one single-copy
// atomic (agent-scope, relaxed) word, so a word with the right tag holds that
// step's value: no separate flag, no wait for store completion, one memory
// round trip per step.  Two buffers suffice: a member writes step s + 2 into
// step s's buffer only after reading every member's step s + 1 words, which
// each member wrote after it had read all of step s.  Every poll is bounded
// by spin_limit; a timeout sets *err and the kernel runs to its end without
// further waits (results are then invalid and the caller reports the error).
// All workgroups must be resident together: launched cooperatively, one per
// CU.  Workgroup ids map to XCDs round-robin, so a group's members are given
// ids of one residue mod 8 (one XCD).
constexpr int LC_KM = 8;
constexpr int LC_SPG = 2;
constexpr int LC_NT = 1024;

__host__ __device__ inline int lstm_coop_groups(int B) { return (B + LC_SPG - 1) / LC_SPG; }
__host__ __device__ inline int lstm_coop_grid(int B) {
  return (lstm_coop_groups(B) + 7) / 8 * 8 * LC_KM;
}
static inline size_t lstm_coop_lds(int H) {
  const int U = H / LC_KM;
  return ((size_t)4 * H * (U + 4) + (size_t)LC_SPG * 4 * H + (size_t)(LC_NT / 64) * LC_SPG * U +
          (size_t)2 * 4 * LC_SPG * U) *
         sizeof(float);
}

__device__ __forceinline__ unsigned long long lc_word(float v, unsigned tag) {
  return ((unsigned long long)tag << 32) | (unsigned long long)__float_as_uint(v);
}

__global__ __launch_bounds__(LC_NT) void lstm_bwd_coop_kernel(
    const float *__restrict__ gh, const float *__restrict__ igb, const float *__restrict__ tcb,
    const float *__restrict__ cbuf, const float *__restrict__ Wh, const float *__restrict__ bias,
    float *__restrict__ D, unsigned long long *X, int *err, int B, int T, int H, unsigned base,
    int spin_limit, int seq) {
  extern __shared__ float sm[];
  const int U = H / LC_KM, UP = U + 4, G4 = 4 * H;
  float *Wsl = sm;                          // [4H][UP]: Wh[r][u0 + u]
  float *dGs = Wsl + (size_t)G4 * UP;       // [SPG][4H]: the group's dG of this step
  float *part = dGs + LC_SPG * G4;          // [waves][SPG][U]
  float *gpre = part + (LC_NT / 64) * LC_SPG * U;  // [2][4][SPG * U]: owners' next ig, tc, c, dL/dh
  const int wg = blockIdx.x, xcd = wg & 7, rest = wg >> 3;
  const int m = rest % LC_KM, g = (rest / LC_KM) * 8 + xcd;
  const int ngroups = lstm_coop_groups(B);
  if (g >= ngroups) return;  // every member of a group computes the same g
  const int Bp = ngroups * LC_SPG;
  const int u0 = m * U;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int idx = tid; idx < G4 * U; idx += LC_NT) {
    const int r = idx / U, u = idx - r * U;
    Wsl[r * UP + u] = Wh[(size_t)r * H + u0 + u];
  }
  // owner lanes: thread s * U + u (wave 0) holds unit u0 + u of sample g*SPG + s
  const bool own = tid < LC_SPG * U;
  const int so = tid / U, uo = tid - so * U;
  const int bo = g * LC_SPG + so, io = u0 + uo;
  const bool valid = own && bo < B;
  float cur = 0.f, dcn = 0.f, fg = 0.f, gg = 0.f, og = 0.f, dfd = 0.f, dgd = 0.f, dod = 0.f;
  float ign = 0.f, tcn = 0.f, cpn = 0.f;
  const size_t ob = (size_t)bo * T * H + io;
  if (valid) {
    cur = seq ? gh[ob + (size_t)(T - 1) * H] : gh[(size_t)bo * H + io];
    fg = sigm(bias[H + io]);
    gg = tanh32(bias[2 * H + io]);
    og = sigm(bias[3 * H + io]);
    dfd = fg * (1.0f - fg);
    dgd = 1.0f - gg * gg;
    dod = og * (1.0f - og);
    ign = igb[ob + (size_t)(T - 1) * H];
    tcn = tcb[ob + (size_t)(T - 1) * H];
    cpn = T > 1 ? cbuf[ob + (size_t)(T - 2) * H] : 0.f;
    float *padrow = D + ((size_t)bo * (T + 1) + T) * G4;
#pragma unroll
    for (int q = 0; q < 4; ++q) padrow[q * H + io] = 0.f;
  }
  bool bad = spin_limit < 0;  // forced timeout (test hook): give up without polling
  if (bad && tid == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Two roles with two barriers per step each, in separate loops (no
  // control-flow merge inside a step, where the compiler would make wave 0
  // wait for its stores): wave 0 holds the owner lanes; waves 1.. fetch the
  // exchange and compute Wh^T dG.  A wait for a load also waits for every
  // vector store issued before it, so the owners load nothing after their
  // exchange stores within a step.
  const int NO = LC_SPG * U;  // owner slots
  if (wave == 0) {
    for (int step = 0; step < T; ++step) {
      const int t = T - 1 - step, par = t & 1;
      const unsigned tag = base + (unsigned)step + 1u;
      unsigned long long *xb = X + (size_t)par * Bp * G4 + (size_t)g * LC_SPG * G4;
      if (own) {
        // step 0's saved gates from the prologue, later ones prefetched into
        // LDS by the other waves during the previous step
        const float *gp = gpre + (size_t)par * 4 * NO;
        const float ig = step ? gp[tid] : ign, tc = step ? gp[NO + tid] : tcn,
                    cp = step ? gp[2 * NO + tid] : cpn;
        if (seq && step) cur += gp[3 * NO + tid];  // this step's own gradient (unroller.go:192-198)
        const float did = ig * (1.0f - ig);
        const float dc = cur * og * (1 - tc * tc) + dcn;
        const float dv[4] = {dc * gg * did, dc * cp * dfd, dc * ig * dgd, cur * tc * dod};
        dcn = dc * fg;
        if (valid) {
          float *row = D + ((size_t)bo * (T + 1) + t) * G4;
#pragma unroll
          for (int q = 0; q < 4; ++q) row[q * H + io] = dv[q];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
          __hip_atomic_store(xb + (size_t)so * G4 + q * H + io, lc_word(valid ? dv[q] : 0.f, tag),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();  // dGs filled
      __syncthreads();  // partial sums written
      if (own) {
        float sum = 0.f;
        for (int w = 1; w < LC_NT / 64; ++w) sum += part[(size_t)w * LC_SPG * U + so * U + uo];
        cur += sum;
      }
    }
    return;
  }
  // waves 1..: thread rt = tid - 64 = (share, c4) sums the rows of its share
  // for units 4*c4 .. 4*c4+3 of both samples
  const int rt = tid - 64;
  constexpr int NRT = LC_NT - 64;
  const int C4 = U / 4;                     // 1, 2, 4 or 8: divides 64 and NRT
  const int c4 = rt % C4, share = rt / C4;
  const int nshare = NRT / C4;
  const int rps = (G4 + nshare - 1) / nshare;
  const int r0 = min(share * rps, G4), r1 = min(r0 + rps, G4);
  constexpr int MAXW = (LC_SPG * 4 * 256 + NRT - 1) / NRT;  // exchange words per thread, H <= 256
  const int nw = LC_SPG * G4;
  // prefetch role: thread rt < NK * NO loads value (rt / NO) of owner slot rt % NO
  const int NK = seq ? 4 : 3;
  const int pk = rt / NO, ps = rt - pk * NO;
  const int pb = g * LC_SPG + ps / U, pu = u0 + ps % U;
  const bool pv = rt < NK * NO && pb < B;
  const float *psrc = pk == 0 ? igb : (pk == 1 ? tcb : (pk == 2 ? cbuf : gh));
  const size_t pbase = (size_t)pb * T * H + pu;
  for (int step = 0; step < T; ++step) {
    const int t = T - 1 - step, par = t & 1;
    const unsigned tag = base + (unsigned)step + 1u;
    const unsigned long long *xb = X + (size_t)par * Bp * G4 + (size_t)g * LC_SPG * G4;
    // the next step's saved gate (step t - 1: ig, tc of t - 1, c of t - 2)
    const int tl = pk == 2 ? t - 2 : t - 1;
    const float pre = pv && t > 0 && tl >= 0 ? psrc[pbase + (size_t)tl * H] : 0.f;
    // all of this thread's words at once, then re-poll those without this step's tag
    unsigned long long wv[MAXW];
#pragma unroll
    for (int k = 0; k < MAXW; ++k) {
      const int idx = rt + k * NRT;
      wv[k] = idx < nw ? __hip_atomic_load(xb + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : 0ull;
    }
    if (rt < NK * NO) gpre[(size_t)(par ^ 1) * 4 * NO + rt] = pre;
#pragma unroll
    for (int k = 0; k < MAXW; ++k) {
      const int idx = rt + k * NRT;
      if (idx < nw) {
        int spins = 0;
        while (!bad && (unsigned)(wv[k] >> 32) != tag) {
          if (++spins > spin_limit) {
            bad = true;
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          wv[k] = __hip_atomic_load(xb + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        dGs[idx] = __uint_as_float((unsigned)wv[k]);
      }
    }
    __syncthreads();  // dGs filled
    float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0;
    for (int r = r0; r < r1; ++r) {
      const float4 w = *reinterpret_cast<const float4 *>(Wsl + r * UP + 4 * c4);
      const float g0 = dGs[r], g1 = dGs[G4 + r];
      a0.x += w.x * g0; a0.y += w.y * g0; a0.z += w.z * g0; a0.w += w.w * g0;
      a1.x += w.x * g1; a1.y += w.y * g1; a1.z += w.z * g1; a1.w += w.w * g1;
    }
    for (int o = C4; o < 64; o <<= 1) {
      a0.x += __shfl_xor(a0.x, o, 64); a0.y += __shfl_xor(a0.y, o, 64);
      a0.z += __shfl_xor(a0.z, o, 64); a0.w += __shfl_xor(a0.w, o, 64);
      a1.x += __shfl_xor(a1.x, o, 64); a1.y += __shfl_xor(a1.y, o, 64);
      a1.z += __shfl_xor(a1.z, o, 64); a1.w += __shfl_xor(a1.w, o, 64);
    }
    if (lane < C4) {
      float *p0 = part + (size_t)wave * LC_SPG * U + 4 * lane;
      *reinterpret_cast<float4 *>(p0) = a0;
      *reinterpret_cast<float4 *>(p0 + U) = a1;
    }
    __syncthreads();  // partial sums written
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

// Gram of one chain in double, stored by columns: GT[ch][u][v] = <D_u, D_v>
// for u <= v (so the clip's per-block products read consecutive v),
// <D_u, D_v> = (dG_u . dG_v) * (x_u . x_v + h_u . h_v + 1).
// One block = a 64x64 tile pair (tv >= tu); 4 waves of 32x32, each 2x2
// v_mfma_f64_16x16x4_f64 tiles with one accumulator set for the dG segment and
// one for the [x | hPrev] segments; the MFMA rows are u and its columns v, so
// the stores run along v.  K is staged 16 at a time through LDS as doubles
// ([k][row], so a lane's operand read is one 8-byte word).
// f64 16x16x4 operand layout: A[m = l%16][k = l/16], B[k = l/16][n = l%16];
// result element i of lane l is row 4*i + l/16, column l%16.
typedef double d4v __attribute__((ext_vector_type(4)));

// A finished Gram tile is published by a count per (chain, 64-column tile):
// every thread's stores are released at agent scope before the barrier, then
// one release increment.  The counts only grow (launch e leaves column tv of
// each chain at e * (tv + 1)), so they are never reset.
__device__ __forceinline__ void gram_publish(unsigned *cnt, int ch, int tv, int nmax) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(cnt + (size_t)ch * ((nmax + 63) / 64) + tv, 1u, __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Waits (bounded) until column tile tv of chain ch holds `want` tiles: relaxed
// polls, then one acquire fence; on a timeout sets *err and returns (the
// results are then invalid).
__device__ __forceinline__ void gram_wait(const unsigned *cnt, int ch, int tv, int nmax,
                                          unsigned want, int *err, int spin_limit) {
  const unsigned *c = cnt + (size_t)ch * ((nmax + 63) / 64) + tv;
  int spins = 0;
  while ((int)(__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - want) < 0) {
    if (++spins > spin_limit) {
      __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

__global__ __launch_bounds__(256) void lstm_gram_kernel(const float *__restrict__ D,
                                                        const float *__restrict__ hbuf,
                                                        const float *__restrict__ x,
                                                        double *__restrict__ Gm, ChainMap cm,
                                                        int I, int H, int nmax, unsigned *cnt) {
  __shared__ double sv[16][64], su[16][64];
  const int ch = blockIdx.x;  // chains vary fastest in dispatch order
  const int n = cm.len(ch);
  // tile (tv, tu) with tu <= tv from the linear block index
  int lin = blockIdx.y, tv = 0;
  while (lin > tv) {
    lin -= tv + 1;
    ++tv;
  }
  const int tu = lin;
  const int ntile = (n + 63) / 64;
  if (tv >= ntile) return;  // whole block leaves before any barrier
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int G4 = 4 * H;
  // staging: thread -> row rr (0..63) and a quarter kq of the 16 k
  const int rr = tid >> 2, kq = (tid & 3) * 4;
  const int iv = tv * 64 + rr, iu = tu * 64 + rr;
  int bv = 0, tvv = 0, bu = 0, tuu = 0;
  if (iv < n) cm.at(ch, iv, bv, tvv);
  if (iu < n) cm.at(ch, iu, bu, tuu);
  d4v acc[2][2][2];
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[q][i][j] = d4v{0.0, 0.0, 0.0, 0.0};
  for (int seg = 0; seg < 3; ++seg) {
    const int K = seg == 0 ? G4 : (seg == 1 ? H : I);
    const float *pv, *pu;
    if (seg == 0) {
      pv = D + ((size_t)bv * (cm.T + 1) + tvv) * G4;
      pu = D + ((size_t)bu * (cm.T + 1) + tuu) * G4;
    } else if (seg == 1) {
      pv = hbuf + ((size_t)bv * (cm.T + 1) + tvv) * H;
      pu = hbuf + ((size_t)bu * (cm.T + 1) + tuu) * H;
    } else {
      pv = x + ((size_t)bv * cm.T + cm.T - 1) * I;
      pu = x + ((size_t)bu * cm.T + cm.T - 1) * I;
    }
    const int q = seg == 0 ? 0 : 1;
    for (int k0 = 0; k0 < K; k0 += 16) {
      float fv[4], fu[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = k0 + kq + e;
        fv[e] = (iv < n && k < K) ? pv[k] : 0.f;
        fu[e] = (iu < n && k < K) ? pu[k] : 0.f;
      }
      __syncthreads();
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sv[kq + e][rr] = (double)fv[e];
        su[kq + e][rr] = (double)fu[e];
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int k = kk * 4 + (lane >> 4);
        double a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = su[k][wm * 32 + i * 16 + (lane & 15)];
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = sv[k][wn * 32 + j * 16 + (lane & 15)];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[q][i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[q][i][j], 0, 0, 0);
      }
    }
  }
  double *Gc = Gm + (size_t)ch * nmax * nmax;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int u = tu * 64 + wm * 32 + i * 16 + 4 * r + (lane >> 4);
        const int v = tv * 64 + wn * 32 + j * 16 + (lane & 15);
        if (v < n && u <= v) Gc[(size_t)u * nmax + v] = acc[0][i][j][r] * (acc[1][i][j][r] + 1.0);
      }
  if (cnt) gram_publish(cnt, ch, tv, nmax);
}

// One 16-byte group of a Gram row: K runs over [dG | hPrev | x_last]; the first
// 4H go to the dG accumulators, the rest (zero padded to a multiple of 32) to
// the [x | hPrev] ones.
__device__ __forceinline__ float4 gram_row4(const float *__restrict__ D,
                                            const float *__restrict__ hbuf,
                                            const float *__restrict__ x, int b, int t, int T,
                                            int I, int H, int k) {
  const int G4 = 4 * H;
  if (k < G4) return *reinterpret_cast<const float4 *>(D + ((size_t)b * (T + 1) + t) * G4 + k);
  k -= G4;
  if (k < H) return *reinterpret_cast<const float4 *>(hbuf + ((size_t)b * (T + 1) + t) * H + k);
  k -= H;
  if (k < I) return *reinterpret_cast<const float4 *>(x + ((size_t)b * T + T - 1) * I + k);
  return make_float4(0.f, 0.f, 0.f, 0.f);
}


// The same Gram with 16-byte staging (H % 8 == 0, I % 4 == 0 and 16-byte aligned
// rows), staged as float32: each K stage (32 wide) of the 64 u-rows and
// 64 v-rows goes to LDS with 16-byte stores ([row][32 + 4], the pad keeps the
// b128 reads of 16 consecutive rows on distinct banks), and lane l of a wave
// takes k = 8*(l/16) + s at MFMA step s of a stage, so its 8 operand values of
// a row are two b128 reads, widened to double as they are used (the products
// and sums stay in float64).  The next stage is prefetched into registers
// during the MFMAs; one barrier per stage.
__global__ __launch_bounds__(256) void lstm_gram_v5_kernel(const float *__restrict__ D,
                                                           const float *__restrict__ hbuf,
                                                           const float *__restrict__ x,
                                                           double *__restrict__ Gm, ChainMap cm,
                                                           int I, int H, int nmax, unsigned *cnt) {
  constexpr int KS = 32, GP = KS + 4;
  __shared__ __attribute__((aligned(16))) float su[2][64 * GP], sv[2][64 * GP];
  const int ch = blockIdx.x;  // chains vary fastest in dispatch order
  const int n = cm.len(ch);
  int lin = blockIdx.y, tv = 0;
  while (lin > tv) {
    lin -= tv + 1;
    ++tv;
  }
  const int tu = lin;
  if (tv >= (n + 63) / 64) return;  // whole block leaves before any barrier
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int G4 = 4 * H;
  const int Kz = G4 + ((H + I + KS - 1) / KS) * KS;  // padded K; G4 % KS == 0
  const int nst = Kz / KS;
  // staging: float4 slot f = tid + 256 j of a stage is row f >> 3, k 4 (f & 7)
  int bu[2], tuu[2], bv[2], tvv[2];
  bool oku[2], okv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = (tid + 256 * j) >> 3;
    const int iu = tu * 64 + r, iv = tv * 64 + r;
    oku[j] = iu < n;
    okv[j] = iv < n;
    bu[j] = tuu[j] = bv[j] = tvv[j] = 0;
    if (oku[j]) cm.at(ch, iu, bu[j], tuu[j]);
    if (okv[j]) cm.at(ch, iv, bv[j], tvv[j]);
  }
  float4 ru[2], rv[2];
  auto load = [&](int k0) {
    // explicit branches: a select between the row and a zero vector became a
    // flat load through a pointer into private memory
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int k = k0 + 4 * ((tid + 256 * j) & 7);
      if (oku[j])
        ru[j] = gram_row4(D, hbuf, x, bu[j], tuu[j], cm.T, I, H, k);
      else
        ru[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (okv[j])
        rv[j] = gram_row4(D, hbuf, x, bv[j], tvv[j], cm.T, I, H, k);
      else
        rv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int f = tid + 256 * j, o = (f >> 3) * GP + 4 * (f & 7);
      *reinterpret_cast<float4 *>(&su[buf][o]) = ru[j];
      *reinterpret_cast<float4 *>(&sv[buf][o]) = rv[j];
    }
  };
  d4v acc[2][2][2];
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[q][i][j] = d4v{0.0, 0.0, 0.0, 0.0};
  load(0);
  store(0);
  __syncthreads();
  const int kl = 8 * (lane >> 4), m16 = lane & 15;
  for (int st = 0; st < nst; ++st) {
    const int cur = st & 1;
    const bool more = st + 1 < nst;
    if (more) load((st + 1) * KS);  // in flight during the MFMAs
    float fa[2][8], fb[2][8];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float *pa = &su[cur][(wm * 32 + i * 16 + m16) * GP + kl];
      const float *pb = &sv[cur][(wn * 32 + i * 16 + m16) * GP + kl];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 a4 = *reinterpret_cast<const float4 *>(pa + 4 * h);
        const float4 b4 = *reinterpret_cast<const float4 *>(pb + 4 * h);
        fa[i][4 * h] = a4.x; fa[i][4 * h + 1] = a4.y; fa[i][4 * h + 2] = a4.z; fa[i][4 * h + 3] = a4.w;
        fb[i][4 * h] = b4.x; fb[i][4 * h + 1] = b4.y; fb[i][4 * h + 2] = b4.z; fb[i][4 * h + 3] = b4.w;
      }
    }
    const int q = st * KS < G4 ? 0 : 1;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (q == 0) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[0][i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)fa[i][s], (double)fb[j][s],
                                                                acc[0][i][j], 0, 0, 0);
      } else {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[1][i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)fa[i][s], (double)fb[j][s],
                                                                acc[1][i][j], 0, 0, 0);
      }
    }
    if (more) store(cur ^ 1);  // that buffer was last read before the previous barrier
    __syncthreads();
  }
  double *Gc = Gm + (size_t)ch * nmax * nmax;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int u = tu * 64 + wm * 32 + i * 16 + 4 * r + (lane >> 4);
        const int v = tv * 64 + wn * 32 + j * 16 + (lane & 15);
        if (v < n && u <= v) Gc[(size_t)u * nmax + v] = acc[0][i][j][r] * (acc[1][i][j][r] + 1.0);
      }
  if (cnt) gram_publish(cnt, ch, tv, nmax);
}

// Sequential clip of one chain from its Gram matrix; one workgroup per chain.
// With a_u = 1/P_{u-1} (P_v = c_0 ... c_v) the clipped sum is G_v = P_v sum_{u<=v} a_u D_u,
// and step v needs s_v = sum_{u<v} a_u <D_u,D_v>:
//   N^2 = |G|^2 + 2 P s_v + <D_v,D_v>,  c = N > 1 ? 1/N : 1 (clipGradients),
//   P *= c,  a_v = c / P,  |G|^2 = c^2 N^2.
// Blocked by CLIP_BLK steps: the in-block recursion runs in wave 0 with lane r
// holding row r's running s and the block's Gram tile in LDS, so a step costs a
// few lane reads and one fused update instead of a block-wide reduction; while
// it runs, waves 1-15 compute the next block's share of s from all earlier
// blocks (a matrix-vector product over the Gram columns) and stage its tiles,
// and the current block's own share is added from a 64x64 cross tile after.
// Whenever P falls below 1e-150 the coefficients are rescaled by P (exact:
// everything is linear in the a's), in-block at once and for earlier blocks
// (and the next block's partial s) at the end of the block.
constexpr int CLIP_BLK = 64;
constexpr int CLIP_UNR = 16;
constexpr int CLIP_NT = 1024;               // wave 0: recursion; waves 1..15: next block
constexpr int CLIP_NS = (CLIP_NT - 64) / 32;  // shares of the next block's matrix-vector product

__device__ __forceinline__ double readlane_d(double x, int l) {
  const int lo = __builtin_amdgcn_readlane(__double2loint(x), l);
  const int hi = __builtin_amdgcn_readlane(__double2hiint(x), l);
  return __hiloint2double(hi, lo);
}

// Beside the Gram kernel (cnt set) nothing guarantees that the two kernels
// run at the same time (a profiler or a busy device may run them one after
// the other), so the wait for the first Gram column is short (bail_limit
// polls, 2048 by default): without it the chain's workgroup records bailed[ch] = epoch and
// ends; the launch queued after the Gram kernel and after this one (cnt
// null, bailed set) then runs the chains that bailed and no others.
__global__ __launch_bounds__(CLIP_NT) void lstm_clip_kernel(const double *__restrict__ Gm,
                                                        double *__restrict__ a,
                                                        float *__restrict__ w, ChainMap cm,
                                                        int nmax, const unsigned *cnt,
                                                        unsigned epoch, unsigned *started,
                                                        unsigned *bailed, int *err, int spin_limit,
                                                        int bail_limit) {
  // tile[buf][u][r] = <D_{v0+u}, D_{v0+r}> (u <= r) of the current / next block;
  // cross[u][r] = <D_{v0+u}, D_{v1+r}>: current block rows x next block columns
  __shared__ double tile[2][CLIP_BLK][CLIP_BLK + 1];
  __shared__ double cross[CLIP_BLK][CLIP_BLK + 1];
  __shared__ double sold[CLIP_BLK], partq[CLIP_NS][CLIP_BLK], ablk[CLIP_BLK];
  __shared__ double bcast[2];  // P after the block, rescale applied during the block
  const int ch = blockIdx.x;
  const int n = cm.len(ch);
  const double *G = Gm + (size_t)ch * nmax * nmax;  // GT[u][v]
  double *ac = a + (size_t)ch * nmax;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nblk = (n + CLIP_BLK - 1) / CLIP_BLK;
  // run beside the Gram kernel: announce residency, then read each Gram
  // column tile only once its count says this launch's tiles are stored
  if (cnt) {
    __shared__ int go;
    if (tid == 0) {
      __hip_atomic_store(started + ch, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned *c0 = cnt + (size_t)ch * ((nmax + 63) / 64);
      const int limit = spin_limit < bail_limit ? spin_limit : bail_limit;
      int spins = 0, ok = 1;
      if (nblk > 0)
        while ((int)(__hip_atomic_load(c0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - epoch) < 0) {
          if (++spins > limit) {
            ok = 0;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
        }
      if (!ok) __hip_atomic_store(bailed + ch, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      go = ok;
    }
    __syncthreads();
    if (!go) return;  // the launch after the Gram kernel does this chain
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  } else if (bailed) {
    if (__hip_atomic_load(bailed + ch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch) return;
  }
  {
    const int nb0 = min(CLIP_BLK, n);
    for (int e = tid; e < CLIP_BLK * CLIP_BLK; e += CLIP_NT) {
      const int u = e / CLIP_BLK, r = e % CLIP_BLK;
      tile[0][u][r] = (r < nb0 && u <= r) ? G[(size_t)u * nmax + r] : 0.0;
    }
    if (tid < CLIP_BLK) sold[tid] = 0.0;
    if (tid == 0) bcast[0] = 1.0;
  }
  __syncthreads();
  double P = 1.0, Q = 1.0, nrm2 = 0.0;  // wave 0 only; Q = 1/P
  for (int k = 0; k < nblk; ++k) {
    const int v0 = k * CLIP_BLK, nb = min(CLIP_BLK, n - v0);
    const int v1 = v0 + CLIP_BLK, nb1 = k + 1 < nblk ? min(CLIP_BLK, n - v1) : 0;
    if (wv == 0) {
      // Per step only the norm recursion is serial: a_j = 1/P_{j-1} = Q is
      // known when the step starts, so the running-s update of the later rows
      // overlaps it, and 1/N comes from a refined reciprocal square root.
      double(*T)[CLIP_BLK + 1] = tile[k & 1];
      double sl = lane < nb ? sold[lane] : 0.0;  // running s of row v0 + lane
      double al = 0.0;                            // a_{v0 + lane} once known
      double blkscale = 1.0;
      // the lane's tile column and the diagonal, read two steps ahead
      double t0 = T[0][lane], d0 = T[0][0];
      double t1 = nb > 1 ? T[1][lane] : 0.0, d1 = nb > 1 ? T[1][1] : 0.0;
      for (int j = 0; j < nb; ++j) {
        double t2 = 0.0, d2 = 0.0;
        if (j + 2 < nb) {
          t2 = T[j + 2][lane];
          d2 = T[j + 2][j + 2];
        }
        const double aj = Q;
        const double sj = readlane_d(sl, j);
        al = lane == j ? aj : al;
        sl = lane > j ? fma(aj, t0, sl) : sl;
        const double N2 = fma(2.0 * P, sj, nrm2) + d0;
        // clipGradients: scale by 1/N when N > 1 (rsq + one Newton step);
        // both outcomes are computed and selected, no branch on the chain
        double y = __builtin_amdgcn_rsq(N2);
        y = y * (1.5 - 0.5 * N2 * (y * y));
        const bool clip = N2 > 1.0;
        P = clip ? P * y : P;
        Q = clip ? Q * (N2 * y) : Q;
        nrm2 = clip ? (y * y) * N2 : (N2 > 0.0 ? N2 : 0.0);
        if (P < 1e-150) {  // fold P into every coefficient so far
          sl *= P;
          al *= P;
          blkscale *= P;
          Q *= P;
          P = 1.0;
        }
        t0 = t1;
        t1 = t2;
        d0 = d1;
        d1 = d2;
      }
      ablk[lane] = lane < nb ? al : 0.0;
      if (lane < nb) ac[v0 + lane] = al;
      if (lane == 0) {
        bcast[0] = P;
        bcast[1] = blkscale;
      }
    } else if (nb1 > 0) {
      if (cnt) gram_wait(cnt, ch, k + 1, nmax, epoch * (unsigned)(k + 2), err, spin_limit);
      // meanwhile the other three waves prepare the next block: the part of
      // its s from blocks before this one (a's final up to this block's
      // rescale, applied below), its diagonal tile and the cross tile
      // thread (pair of rows 2p, 2p+1; share q of CLIP_NS) reads 16-byte pairs
      const int t = tid - 64, pr = t & 31, q = t >> 5;
      double s0 = 0.0, s1 = 0.0;
      if (2 * pr < nb1) {
        const double2 *col = reinterpret_cast<const double2 *>(G + v1 + 2 * pr);
        const int ld2 = nmax / 2;  // nmax is even (the Gram's pitch)
        constexpr int S = CLIP_NS;
        int u = q;
        for (; u + S * (CLIP_UNR - 1) < v0; u += S * CLIP_UNR) {
          double2 gv[CLIP_UNR];
          double av[CLIP_UNR];
#pragma unroll
          for (int e = 0; e < CLIP_UNR; ++e) {
            gv[e] = col[(size_t)(u + S * e) * ld2];
            av[e] = ac[u + S * e];
          }
#pragma unroll
          for (int e = 0; e < CLIP_UNR; ++e) {
            s0 += av[e] * gv[e].x;
            s1 += av[e] * gv[e].y;
          }
        }
        for (; u < v0; u += S) {
          const double2 g2 = col[(size_t)u * ld2];
          s0 += ac[u] * g2.x;
          s1 += ac[u] * g2.y;
        }
      }
      partq[q][2 * pr] = s0;
      partq[q][2 * pr + 1] = s1;
      double(*Tn)[CLIP_BLK + 1] = tile[(k + 1) & 1];
      for (int e = t; e < CLIP_BLK * CLIP_BLK; e += CLIP_NT - 64) {
        const int u = e / CLIP_BLK, rr = e % CLIP_BLK;
        Tn[u][rr] = (rr < nb1 && u <= rr) ? G[(size_t)(v1 + u) * nmax + v1 + rr] : 0.0;
        cross[u][rr] = (u < nb && rr < nb1) ? G[(size_t)(v0 + u) * nmax + v1 + rr] : 0.0;
      }
    }
    __syncthreads();
    const double bs = bcast[1];
    if (nb1 > 0 && tid < CLIP_BLK) {
      double sn = 0.0;
      for (int r = 0; r < CLIP_NS; ++r) sn += partq[r][tid];
      sn *= bs;
      for (int u = 0; u < nb; ++u) sn += ablk[u] * cross[u][tid];
      sold[tid] = sn;
    }
    if (bs != 1.0)  // rescale owed by the earlier blocks' coefficients
      for (int u = tid; u < v0; u += CLIP_NT) ac[u] *= bs;
    __syncthreads();
  }
  const double Pf = bcast[0];
  for (int u = tid; u < n; u += CLIP_NT) {
    int b, t;
    cm.at(ch, u, b, t);
    w[(size_t)b * (cm.T + 1) + t] = (float)(Pf * ac[u]);
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
    float *col = D + (size_t)b * (T + 1) * G4 + k;
    const float *wb = w + (size_t)b * (T + 1);
    int t = T - 1;
    for (; t >= 7; t -= 8) {  // eight steps' loads in flight, then the same order as below
      float dv[8], wv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        dv[u] = col[(size_t)(t - u) * G4];
        wv[u] = wb[t - u];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float d = dv[u] * wv[u];
        col[(size_t)(t - u) * G4] = d;
        s += d;
      }
    }
    for (; t >= 0; --t) {
      const float d = col[(size_t)t * G4] * wb[t];
      col[(size_t)t * G4] = d;
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

// Thread layout of the recurrent mat-vec: GB threads per share of K (one per
// column, or per 4 columns with 16-byte loads), as many shares as fit 1024.
// Pitch of one chain's Gram matrix (rows of doubles): even, so the clip can
// read 16-byte pairs.
int lstm_gram_pitch(int n) { return (n + 1) & ~1; }

struct LstmLayout {
  bool v4;
  int GB, NQ;
};
static LstmLayout lstm_layout(int H, const float *W) {
  LstmLayout L;
  L.v4 = (H % 4 == 0) && ((reinterpret_cast<uintptr_t>(W) & 15) == 0);
  const int cols = L.v4 ? H / 4 : H;
  L.GB = ((cols + 63) / 64) * 64;
  L.NQ = std::max(1, std::min(16, 1024 / L.GB));
  return L;
}
static bool lstm_fits(int H) { return H >= 1 && H <= 1024; }

hipError_t launch_lstm_fwd(const float *xw, const float *WhT, const float *bias, float *igb,
                           float *tcb, float *cbuf, float *hbuf, float *out, int B, int T, int H,
                           hipStream_t s, int seq) {
  if (!lstm_fits(H)) return hipErrorInvalidValue;
  const LstmLayout L = lstm_layout(H, WhT);
  const size_t base = (size_t)(((H + 3) & ~3) + L.NQ * H) * sizeof(float);
  if (L.v4 && (H + L.NQ - 1) / L.NQ <= LF_R) {  // every thread's WhT share fits its registers
    hipLaunchKernelGGL(lstm_fwd_reg_kernel, dim3(B), dim3(1024), base, s, xw, WhT, bias, igb, tcb,
                       cbuf, hbuf, out, T, H, L.GB, L.NQ, seq);
    return hipGetLastError();
  }
  // as many leading shares of WhT in LDS as fit 128 KB (whole float4 rows:
  // the V4 layout only; the copy needs 16-byte aligned WhT)
  int QL = 0;
  if (L.v4 && H % 4 == 0)
    while (QL < L.NQ && (size_t)(H * (QL + 1) / L.NQ) * H * sizeof(float) <= (128u << 10)) ++QL;
  const size_t shm = base + (size_t)(H * QL / L.NQ) * H * sizeof(float);
  static std::atomic<int> attr_v4[kAttrDevices], attr_v1[kAttrDevices];
  {
    const hipError_t e =
        L.v4 ? ensure_lds_attr(reinterpret_cast<const void *>(lstm_fwd_kernel<true>), (int)shm, attr_v4)
             : ensure_lds_attr(reinterpret_cast<const void *>(lstm_fwd_kernel<false>), (int)shm, attr_v1);
    if (e != hipSuccess) return e;
  }
  if (L.v4)
    hipLaunchKernelGGL(lstm_fwd_kernel<true>, dim3(B), dim3(1024), shm, s, xw, WhT, bias, igb, tcb,
                       cbuf, hbuf, out, T, H, L.GB, L.NQ, QL, seq);
  else
    hipLaunchKernelGGL(lstm_fwd_kernel<false>, dim3(B), dim3(1024), shm, s, xw, WhT, bias, igb, tcb,
                       cbuf, hbuf, out, T, H, L.GB, L.NQ, 0, seq);
  return hipGetLastError();
}

hipError_t launch_lstm_bwd(const float *gh, const float *igb, const float *tcb, const float *cbuf,
                           const float *Wh, const float *bias, float *D, int B, int T, int H,
                           hipStream_t s, int seq) {
  if (!lstm_fits(H)) return hipErrorInvalidValue;
  const LstmLayout L = lstm_layout(H, Wh);
  const size_t shm = (size_t)(4 * H + L.NQ * H) * sizeof(float);
  if (L.v4)
    hipLaunchKernelGGL(lstm_bwd_kernel<true>, dim3(B), dim3(1024), shm, s, gh, igb, tcb, cbuf, Wh,
                       bias, D, T, H, L.GB, L.NQ, seq);
  else
    hipLaunchKernelGGL(lstm_bwd_kernel<false>, dim3(B), dim3(1024), shm, s, gh, igb, tcb, cbuf, Wh,
                       bias, D, T, H, L.GB, L.NQ, seq);
  return hipGetLastError();
}

bool lstm_coop_eligible(int B, int H) {
  // U = H / 8 units per member, handled 4 at a time by U / 4 lanes whose
  // shuffle reduction needs a power of two
  return B >= 1 && B <= 64 && (H == 32 || H == 64 || H == 128 || H == 256);
}

size_t lstm_coop_sync_bytes(int B, int H) {
  const int Bp = lstm_coop_groups(B) * LC_SPG;
  return (size_t)2 * Bp * 4 * H * sizeof(unsigned long long);
}

// sync: lstm_coop_sync_bytes(B, H) bytes, zeroed once at allocation: the
// tagged exchange words (tags only ever grow: each launch passes base = the
// previous launch's last tag, so no word of an earlier launch matches).
// err: device int, 0 on success.
hipError_t launch_lstm_bwd_coop(const float *gh, const float *igb, const float *tcb,
                                const float *cbuf, const float *Wh, const float *bias, float *D,
                                void *sync, int *err, unsigned *epoch, int B, int T, int H,
                                int spin_limit, hipStream_t s, int seq) {
  if (!lstm_coop_eligible(B, H)) return hipErrorInvalidValue;
  unsigned long long *X = reinterpret_cast<unsigned long long *>(sync);
  const size_t shm = lstm_coop_lds(H);
  static std::atomic<int> attr_set[kAttrDevices];
  {
    const hipError_t e =
        ensure_lds_attr(reinterpret_cast<const void *>(lstm_bwd_coop_kernel), (int)shm, attr_set);
    if (e != hipSuccess) return e;
  }
  unsigned base = *epoch;
  void *args[] = {(void *)&gh, (void *)&igb, (void *)&tcb, (void *)&cbuf, (void *)&Wh,
                  (void *)&bias, (void *)&D, (void *)&X, (void *)&err,
                  (void *)&B, (void *)&T, (void *)&H, (void *)&base, (void *)&spin_limit,
                  (void *)&seq};
  hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void *>(lstm_bwd_coop_kernel),
                                            dim3(lstm_coop_grid(B)), dim3(LC_NT), args, shm, s);
  if (e == hipSuccess) *epoch = base + (unsigned)T;
  return e;
}

hipError_t launch_lstm_gram(const float *D, const float *hbuf, const float *x, double *gram, int B,
                            int T, int I, int H, int W, hipStream_t s, unsigned *cnt) {
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  ChainMap cm{T, (B + Wc - 1) / Wc, B};
  const int nchains = (B + cm.chunk - 1) / cm.chunk;
  const int nmax = lstm_gram_pitch(cm.chunk * T);
  const int ntile = (nmax + 63) / 64;
  dim3 g(nchains, ntile * (ntile + 1) / 2);  // column tiles complete in order, all chains together
  const bool vec = H % 8 == 0 && I % 4 == 0 &&
                  (((reinterpret_cast<uintptr_t>(D) | reinterpret_cast<uintptr_t>(hbuf) |
                     reinterpret_cast<uintptr_t>(x)) & 15) == 0);
  if (vec)
    hipLaunchKernelGGL(lstm_gram_v5_kernel, g, dim3(256), 0, s, D, hbuf, x, gram, cm, I, H, nmax, cnt);
  else
    hipLaunchKernelGGL(lstm_gram_kernel, g, dim3(256), 0, s, D, hbuf, x, gram, cm, I, H, nmax, cnt);
  return hipGetLastError();
}

// One thread: waits (bounded) until every chain's clip workgroup has started,
// so the Gram kernel queued after it cannot fill the CUs first.  Only the
// overlap depends on it: after spin_limit polls it lets the Gram kernel go.
__global__ void lstm_clip_gate_kernel(const unsigned *started, int nchains, unsigned epoch,
                                      int spin_limit) {
  if (threadIdx.x != 0) return;
  int spins = 0;
  for (int ch = 0; ch < nchains; ++ch)
    while (__hip_atomic_load(started + ch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch) {
      if (++spins > spin_limit) return;
      __builtin_amdgcn_s_sleep(2);
    }
}

int lstm_gram_counters(int B, int T, int W) {
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  const int chunk = (B + Wc - 1) / Wc, nchains = (B + chunk - 1) / chunk;
  return nchains * ((lstm_gram_pitch(chunk * T) + 63) / 64);
}

hipError_t launch_lstm_clip_gate(const unsigned *started, int B, int W, unsigned epoch, int *err,
                                 int spin_limit, hipStream_t s) {
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  const int chunk = (B + Wc - 1) / Wc, nchains = (B + chunk - 1) / chunk;
  (void)err;
  hipLaunchKernelGGL(lstm_clip_gate_kernel, dim3(1), dim3(64), 0, s, started, nchains, epoch,
                     spin_limit < 0 ? 0 : spin_limit);
  return hipGetLastError();
}

hipError_t launch_lstm_clip(const double *gram, double *coef, float *w, int B, int T, int W,
                            hipStream_t s, const unsigned *cnt, unsigned epoch, unsigned *started,
                            int *err, int spin_limit, unsigned *bailed, int bail_limit) {
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  ChainMap cm{T, (B + Wc - 1) / Wc, B};
  const int nchains = (B + cm.chunk - 1) / cm.chunk;
  const int nmax = lstm_gram_pitch(cm.chunk * T);
  if (cnt && (!started || !err || !bailed)) return hipErrorInvalidValue;
  // beside the Gram kernel, unused dynamic LDS keeps its workgroups off the
  // clip's CUs (their waves would take issue slots from the serial recursion)
  const size_t pad = cnt ? (size_t)24 << 10 : 0;
  static std::atomic<int> attr_set[kAttrDevices];
  if (cnt) {
    const hipError_t e =
        ensure_lds_attr(reinterpret_cast<const void *>(lstm_clip_kernel), (int)pad, attr_set);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(lstm_clip_kernel, dim3(nchains), dim3(CLIP_NT), pad, s, gram, coef, w, cm, nmax,
                     cnt, epoch, started, bailed, err, spin_limit, bail_limit);
  return hipGetLastError();
}

hipError_t launch_lstm_clip_weights(const float *D, const float *hbuf, const float *x, double *gram,
                                    double *coef, float *w, int B, int T, int I, int H, int W,
                                    hipStream_t s) {
  const hipError_t e = launch_lstm_gram(D, hbuf, x, gram, B, T, I, H, W, s);
  if (e != hipSuccess) return e;
  return launch_lstm_clip(gram, coef, w, B, T, W, s);
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
