// Internal declarations shared by the runtime and the kernel files of
// libgoneuron_hip.so.  Kernels are gfx950-only (64-wide wavefronts, fp32 MFMA).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/goneuron_hip.h"

namespace gn {

// Activation derivative kinds used by kernels.  Computed from the saved
// *output* of the layer: out = act(pre) is deterministic, so relu'(pre) ==
// (out > 0), sigmoid'(pre) == out*(1-out), tanh'(pre) == 1-out*out exactly as
// the reference recomputes them from the pre-activation.
enum DerivKind : int32_t {
  D_ONE = 0,      // Linear: derivative 1
  D_RELU = 1,
  D_SIGMOID = 2,
  D_TANH = 3,
  D_NAN = 4,      // Softmax/LogSoftmax *values*: Derivative returns NaN (Q3)
  D_GELU = 5,     // GELU'(x) in float64 of the saved value, which must be the
                  // pre-activation (GELU *values* run as identity forward)
};

// GELU'(x) as activations.go:258-272 computes it, in float64.
__host__ __device__ __forceinline__ float gelu_deriv(float x) {
  const double xd = (double)x, x2 = xd * xd, x3 = xd * x2;
  const double arg = 0.7978845608028654 * (xd + 0.044715 * x3);
  const double tv = tanh(arg);
  const double t1 = 0.5 * (1.0 + tv);
  const double t2 = 0.5 * xd * (1.0 - tv * tv) * 0.7978845608028654 * (1.0 + 0.134145 * x2);
  return (float)(t1 + t2);
}

// Forward activation kinds applied elementwise in GEMM epilogues.
enum FwdKind : int32_t {
  F_IDENTITY = 0,
  F_RELU = 1,
  F_SIGMOID = 2,
  F_TANH = 3,
  F_NAN = 4,      // scalar Activate of Softmax/LogSoftmax values (Conv2D only)
  F_LEAKY = 5,    // *LeakyReLU with alpha 0.1 (the MoE experts)
};

struct GemmArgs {
  int M, N, K;
  const float *A;
  int lda;
  const float *B;
  int ldb;
  float *C;
  int ldc;
  float alpha;
  const float *bias;  // EPI_BIAS_ACT: per-column bias (may be null)
  const float *aux;   // EPI_DACT: saved output used for act'
  int ldaux;
  int act;            // FwdKind or DerivKind
  float *ws;          // split-K workspace (may be null: no split)
  size_t ws_cap;      // floats
  int aux_div;        // EPI_DACT: > 1 reads aux row (row/aux_div)*aux_div + aux_div-1
  const float *colscale;  // EPI_DACT: per-column factor applied before act' (may be null)
  // nbatch > 1: that many GEMMs, the z-th with A, B, bias and C advanced by
  // z times these strides (floats; 0 shares the operand)
  int nbatch;
  int64_t bstride_A, bstride_B, bstride_bias, bstride_C;
  // nbatch_in > 1: members form [nbatch / nbatch_in][nbatch_in]; member
  // z = zo * nbatch_in + zi is advanced by zo times the strides above plus zi
  // times these (attention's (sample, head) pairs inside [B*T, D] matrices)
  int nbatch_in;
  int64_t istride_A, istride_B, istride_C;
  // EPI_BIAS_ACT with a Dropout above (training): also drop_out[row, col] =
  // drop_mask[col] > 0 ? C[row, col] * drop_scale : 0 (the dropout kernel's
  // expression), at pitch ldc; in the split-K reduction when K splits, else by
  // a dropout launch after the GEMM.  nbatch <= 1.
  float *drop_out;
  const float *drop_mask;
  float drop_scale;
  // non-null: when K splits, only the partial sums are written to ws (the
  // reduce and epilogue are left to the caller) and *defer_splits receives
  // the split count; it receives 1 when the GEMM ran whole (with epilogue)
  int *defer_splits;
  // kseg > 0 (a multiple of 64, nbatch <= 1, 64-wide tiles): the K range is
  // cut into segments of kseg, segment s of op(A) / op(B) starting seg_A /
  // seg_B floats after segment 0 (a sum of products A_s B_s over operands
  // that are not adjacent in memory, in one launch); launch_gemm returns
  // hipErrorNotSupported where its plan cannot take them.  kseg_dA / kseg_dB
  // are filled by launch_gemm.
  int kseg;
  int64_t seg_A, seg_B, kseg_dA, kseg_dB;
  // cs_src set: when K splits, the split-K reduction launch also writes the
  // column sums cs_dst[c] = cs_scale * sum_r cs_src[r][c] (cs_rows x cs_cols,
  // dense) and sets *cs_done to 1 (else 0: the caller sums them itself)
  const float *cs_src;
  float *cs_dst;
  int cs_rows, cs_cols;
  float cs_scale;
  int *cs_done;
};
bool gemm_segments_ok(const GemmArgs &a);  // launch_gemm can take a's K segments

// EPI_SCALE    C = alpha*acc
// EPI_BIAS_ACT C = act(acc + bias[col])
// EPI_DACT     C = (acc * colscale[col]) * act'(aux[r', col])  (r' = row, or the last row of
//              its group; no colscale: acc * act')
// EPI_BIAS_ADD C = alpha*acc + bias[col] + aux[row, col]  (aux may alias C)
enum GemmEpi : int { EPI_SCALE = 0, EPI_BIAS_ACT = 1, EPI_DACT = 2, EPI_BIAS_ADD = 4 };

// op(A) layout: 'N' = A[m*lda+k] (K contiguous), 'T' = A[k*lda+m].
// op(B) layout: 'N' = B[k*ldb+n] (N contiguous), 'T' = B[n*ldb+k].
hipError_t launch_gemm(char ta, char tb, int epi, const GemmArgs &a, hipStream_t s);

hipError_t launch_adam(float *p, const float *g, float *m, float *v, int64_t n, float efflr,
                       float b1, float b2, float omb1, float omb2, float eps, hipStream_t s,
                       int max_blocks = 16384);

// Adam.StepInPlace for one parameter, opt.go:244-251:
//   m = b1*m + (1-b1)*g ; v = b2*v + (1-b2)*g*g ; p -= effLR*m/(sqrt(v)+eps)
// The library is built with -ffp-contract=off, so every product and sum is
// rounded on its own; '/' and sqrtf are IEEE correctly rounded under
// -fhip-fp32-correctly-rounded-divide-sqrt (== float32(math.Sqrt(float64(v)))).
__device__ __forceinline__ void adam1(float &p, float g, float &m, float &v, float efflr, float b1,
                                      float b2, float omb1, float omb2, float eps) {
  const float mi = b1 * m + omb1 * g;
  const float vi = b2 * v + omb2 * g * g;
  m = mi;
  v = vi;
  p = p - efflr * mi / (__builtin_sqrtf(vi) + eps);
}

// Network.Step's update carried by the kernel that writes a step's last
// gradients (no Adam launch of its own).  A gradient at gp in the arena's
// gradient region has its parameter, first and second moment at gp - stride,
// gp + stride and gp + 2 stride (the arena is [params | grads | m | v]).
struct AdamStep {
  float efflr, b1, b2, omb1, omb2, eps;
  int64_t stride;  // 0: no update
  // launch_conv_wgrad_reduce: extra blocks update the gradients
  // [rest + r0[i], rest + r1[i]) (final, their parameters read by no later
  // kernel of the step)
  float *rest;
  int64_t r0[2], r1[2];
};

// the update of the parameter whose gradient g was just stored at gp
__device__ __forceinline__ void adam_at(float *gp, float g, const AdamStep &a) {
  float *pp = gp - a.stride, *mp = gp + a.stride, *vp = gp + 2 * a.stride;
  float p = *pp, m = *mp, v = *vp;
  adam1(p, g, m, v, a.efflr, a.b1, a.b2, a.omb1, a.omb2, a.eps);
  *pp = p;
  *mp = m;
  *vp = v;
}

// db[o] = scale * sum_b dz[b*ld + o]
hipError_t launch_colsum(const float *dz, int rows, int cols, int ld, float scale, float *out,
                         float *scratch, size_t scratch_cap, hipStream_t s);
// up to 3 column sums of equal shape (dz[i] -> out[i]) in one launch pair
hipError_t launch_colsum_multi(const float *const *dz, float *const *out, int n, int rows, int cols,
                               int ld, float scale, float *scratch, size_t scratch_cap,
                               hipStream_t s);

// SwiGLU gating on Z = [gate | up] rows (2*out wide) and its backward into dZ
hipError_t launch_swiglu_fwd(const float *Z, float *y, int B, int out, hipStream_t s);
hipError_t launch_swiglu_bwd(const float *dy, const float *Z, int ldz, float *dZ, int B, int out,
                             hipStream_t s);

// dz = g * act'(out) elementwise (optionally with dropout mask/scale fused)
hipError_t launch_dact(const float *g, const float *out, float *dz, int64_t n, int deriv,
                       hipStream_t s);

// Output-layer row kernel: forward row activation (softmax/logsoftmax/none),
// per-sample loss, loss gradient, and dz through the activation's Jacobian
// (Q4).  z holds pre-activations [B,C]; out receives the activation output.
// bad (may be null): samples the batch loop skips (an Embedding index error).
// workers == 1: a bad sample adds no loss and no gradient (net.go:738-741);
// workers > 1: a worker stops at its chunk's first bad sample and its chunk
// loss is lost (net.go:641-644, 653-655).
hipError_t launch_out_rows(const float *z, const float *y, float *out, float *dz, float *loss_rows,
                           int B, int C, int row_act, int deriv, int loss_kind, const int32_t *bad,
                           int workers, hipStream_t s);
// launch_out_rows with each row in registers (rows of up to 16384 classes;
// hipErrorNotSupported for longer ones)
hipError_t launch_out_rows_reg(float *out, const float *y, float *dz, float *loss_rows, int B, int C,
                               int row_act, int deriv, int loss_kind, const int32_t *bad, int workers,
                               hipStream_t s);
enum RowAct : int { ROW_NONE = 0, ROW_SOFTMAX = 1, ROW_LOGSOFTMAX = 2, ROW_ELEMWISE = 3 };
// The output Dense layer of a training pass with few outputs as two kernels:
// tail_fwd = the forward GEMM (bias included) + launch_out_rows_reg's rows;
// tail_bwd = dW (scale dz^T x), db (scale colsum dz), dX (dz W with the dX
// GEMM's epilogue: cfac, then act' of aux) and, when gB_below is given, the
// bias gradient of the Dense whose dz that dX is (scale colsum gin).
// Supported: 1 <= C <= 32 outputs, in % 4 == 0, x and W 16-byte aligned
// (hipErrorInvalidValue otherwise).
bool tail_supported(int C, int in);
// The rows of x may come from a GEMM whose K split was not reduced
// (GemmArgs::defer_splits): x[r][c] = act(sum_s ws[s][r][c] + bias[c]) in
// split order (gemm_splitk_reduce's sum and epilogue), written to xo, and
// when a Dropout follows in training, dout = mask[c] > 0 ? x * scale : 0 is
// written too and is the layer's input.
struct TailSplitIn {
  const float *ws = nullptr;  // null: x is read as given
  int splits = 0;
  const float *bias = nullptr;
  int act = 0;
  float *xo = nullptr;
  float *dout = nullptr;
  const float *mask = nullptr;
  float scale = 0.f;
};
hipError_t launch_tail_fwd(const float *x, const float *W, const float *bias, const float *y, float *out,
                           float *dz, float *loss_rows, int B, int in, int C, int row_act, int deriv,
                           int loss_kind, const int32_t *bad, int workers, hipStream_t s,
                           const TailSplitIn &sp = TailSplitIn());
// xb / gWb / inb: gin is the dz of a Dense with input xb (B x inb); its
// weight gradient gWb = scale gin^T xb is summed here too (rows in order).
// pool_arg / pool_gin: gin is the gradient of a Flatten over a 2x2 stride-2
// MaxPool2D with pH x pW input planes (even); the values go through the
// pool's switches straight into pool_gin, its input gradient (gin unused).
hipError_t launch_tail_bwd(const float *x, const float *W, const float *dz, float *gW, float *gB, float *gin,
                           const float *aux, int deriv, const float *cfac, float *gB_below, int B, int in,
                           int C, float scale, hipStream_t s, const int32_t *pool_arg = nullptr,
                           float *pool_gin = nullptr, int pH = 0, int pW = 0, const float *xb = nullptr,
                           float *gWb = nullptr, int inb = 0);

// dst[0, n) = v by a kernel (no memset node, so it can sit in a captured graph)
hipError_t launch_fill(float *dst, float v, int64_t n, hipStream_t s);
// out = ((r + p0) + p1) + p2 with p_j = p + j * pstride
hipError_t launch_add3(const float *r, const float *p, int64_t pstride, float *out, int64_t n, hipStream_t s);

// Row activation only (forward/predict)
hipError_t launch_row_act(float *out, int B, int C, int row_act, hipStream_t s);
// dz of a hidden Softmax / LogSoftmax row activation from its output gradient
hipError_t launch_row_jac(const float *g, const float *out, float *dz, int B, int C, int row_act,
                          hipStream_t s);


// dropout: out = x*scale where mask else 0 (mask is per-feature, Q9)
hipError_t launch_dropout(const float *x, const float *mask, float scale, float *out, int B, int n,
                          hipStream_t s);

// Elementwise forward activation in place.
hipError_t launch_act_inplace(float *x, int64_t n, int fwd, hipStream_t s);

// ---- Conv2D / MaxPool2D (per-sample NCHW, samples contiguous) ----
struct ConvShape {
  int inC, outC, k, stride, pad, H, W, oH, oW;
};
struct PoolShape {
  int C, k, stride, pad, H, W, oH, oW;
};
// pool_out / pool_arg: a 2x2 stride-2 MaxPool2D over the conv output computed
// in the same pass (conv_fwd_pool_fusable shapes only)
hipError_t launch_conv_fwd(const float *x, const float *w, const float *bias, float *out,
                           const ConvShape &s, int B, int fwd, hipStream_t st, float *pool_out = nullptr,
                           int32_t *pool_arg = nullptr);
bool conv_fwd_pool_fusable(const ConvShape &s, const PoolShape &p, int B);
// grad = [dW | db] (scaled), dz = gout * act'(out) formed on the fly
// red: only the partial sums are launched; red receives the reduction's
// arguments for launch_conv_wgrad_reduce
struct ConvWgradReduce {
  const float *ws;
  int nblocks, nslots;
  float scale;
  float *grad;
};
hipError_t launch_conv_wgrad(const float *x, const float *gout, const float *out, float *grad,
                             const ConvShape &s, int B, int deriv, float scale, float *ws,
                             size_t ws_cap, hipStream_t st, ConvWgradReduce *red = nullptr);
// the deferred reduction, with the step's update of every gradient it writes
// and of upd.rest's ranges (extra blocks); upd null: the reduction alone
hipError_t launch_conv_wgrad_reduce(const ConvWgradReduce &red, const AdamStep *upd, hipStream_t st);
hipError_t launch_conv_dgrad(const float *gout, const float *out, const float *w, float *gin,
                             const ConvShape &s, int B, int deriv, hipStream_t st);
hipError_t launch_maxpool_fwd(const float *x, float *out, int32_t *argmax, const PoolShape &s,
                              int B, hipStream_t st);
hipError_t launch_maxpool_bwd(const float *gout, const int32_t *argmax, float *gin,
                              const PoolShape &s, int B, hipStream_t st);
// BatchNorm2D: training forward (per-plane stats st = mean, var, std; running
// stats updated in sample order) or inference forward; training backward with
// per-plane gamma / beta partial sums part [2][B*C] (part may be null).
hipError_t launch_bn_fwd(const float *x, const float *gb, float *y, float *st, float *rm, float *rv,
                         int B, int C, int HW, float eps, float mom, int training, hipStream_t s);
hipError_t launch_bn_bwd(const float *g, const float *x, const float *gb, const float *st, float *dx,
                         float *part, int B, int C, int HW, hipStream_t s);
// inference-mode backward: dx = g * gamma / std(running var); no parameter gradient
hipError_t launch_bn_bwd_eval(const float *g, const float *gb, const float *rv, float *dx, int B,
                              int C, int HW, float eps, hipStream_t s);
hipError_t launch_avgpool_fwd(const float *x, float *out, const PoolShape &s, int B, hipStream_t st);
hipError_t launch_avgpool_bwd(const float *gout, float *gin, const PoolShape &s, int B, hipStream_t st);

// ---- the reference's LCG (layer.go:61-81) on the device ----
constexpr uint64_t LCG_A = 6364136223846793005ull, LCG_C = 1ull;
// state after n steps of s -> a s + c (binary powers of the affine map)
__device__ __forceinline__ uint64_t lcg_jump(uint64_t s, uint64_t n) {
  uint64_t A = 1, C = 0, a = LCG_A, c = LCG_C;
  while (n) {
    if (n & 1) {
      A *= a;
      C = C * a + c;
    }
    c = c * (a + 1);
    a *= a;
    n >>= 1;
  }
  return A * s + C;
}
// Dropout's Q9 mask: element i is 0 when the (i+1)-th draw of RNG(42) is < p
// (the stream is reset before every sample, dropout.go:138-150, 399-401)
hipError_t launch_dropout_mask(float *mask, int n, float p, hipStream_t s);

// ---- MoE ----
constexpr int MOE_MAX_E = 64;  // experts routed by one thread's registers
struct MoeRoute {
  int B, E, K, training;
  int chunk;              // worker chunk (streams 1 + b / chunk), 0: one stream
  uint64_t base[65];      // noise stream states at the start of this forward
};
hipError_t launch_moe_route(const float *logits, float *prob, int32_t *act, const MoeRoute &rt,
                            hipStream_t s);
hipError_t launch_moe_combine(const float *eout, const float *prob, const int32_t *act, float *y,
                              int B, int O, int E, int K, hipStream_t s);
hipError_t launch_moe_backward_deltas(const float *g, const float *eout, const float *prob,
                                      const int32_t *act, float *edz, float *dzg, int B, int O,
                                      int E, int K, int training, hipStream_t s);

// ---- SequenceUnroller(GRU) ----
bool gru_supported(int H);
// seq (returnSequences): out [B][T][H]; g dL/dh_t [B][T][H] (else [B][H])
hipError_t launch_gru_fwd(const float *xw, const float *WhT, float *pre, float *hprev, float *rh,
                          float *out, int B, int T, int H, hipStream_t s, int seq = 0);
hipError_t launch_gru_bwd(const float *g, const float *pre, const float *hprev, const float *Wh,
                          float *dG, int B, int T, int H, hipStream_t s, int seq = 0);

// ---- SequenceUnroller(LSTM) ----
hipError_t launch_transpose(const float *in, float *out, int rows, int cols, hipStream_t s);
// seq (returnSequences): out is [B][T][H] (every state); in the backward gh is
// then dL/dh_t [B][T][H] instead of dL/dh_{T-1} [B][H]
hipError_t launch_lstm_fwd(const float *xw, const float *WhT, const float *bias, float *igb,
                           float *tcb, float *cbuf, float *hbuf, float *out, int B, int T, int H,
                           hipStream_t s, int seq = 0);
hipError_t launch_lstm_bwd(const float *gh, const float *igb, const float *tcb, const float *cbuf,
                           const float *Wh, const float *bias, float *D, int B, int T, int H,
                           hipStream_t s, int seq = 0);
// Cooperative BPTT (see k_lstm.hip): eligibility, the sync buffer it needs
// (flags + exchange, zeroed once at allocation), and the launch.  Returns an
// error without launching when not eligible or when the cooperative launch is
// refused (then lstm_bwd_kernel is the fallback).  *epoch carries the flag
// base across launches; spin_limit < 0 makes every wait time out at once.
bool lstm_coop_eligible(int B, int H);
size_t lstm_coop_sync_bytes(int B, int H);
hipError_t launch_lstm_bwd_coop(const float *gh, const float *igb, const float *tcb,
                                const float *cbuf, const float *Wh, const float *bias, float *D,
                                void *sync, int *err, unsigned *epoch, int B, int T, int H,
                                int spin_limit, hipStream_t s, int seq = 0);
int lstm_gram_pitch(int n);
// the two halves of launch_lstm_clip_weights: the chains' Gram matrices, then
// the clip recursion over them into the per-step weights.  They may also run
// side by side (clip on another stream): with `cnt` (lstm_gram_counters
// unsigned, zeroed once) the Gram kernel counts the finished tiles of each
// column and the clip of launch number `epoch` (1, 2, ...) waits for them;
// `started` (one unsigned per chain, zeroed once) receives `epoch` when a
// chain's clip workgroup is resident, and launch_lstm_clip_gate, queued
// before the Gram kernel, waits for that.  Waits are bounded by spin_limit
// polls and set *err on a timeout.
hipError_t launch_lstm_gram(const float *D, const float *hbuf, const float *x, double *gram, int B,
                            int T, int I, int H, int W, hipStream_t s, unsigned *cnt = nullptr);
// cnt set: beside the Gram kernel (may bail, see lstm_clip_kernel); cnt null
// and bailed set: only the chains whose bailed flag holds `epoch`
hipError_t launch_lstm_clip(const double *gram, double *coef, float *w, int B, int T, int W,
                            hipStream_t s, const unsigned *cnt = nullptr, unsigned epoch = 0,
                            unsigned *started = nullptr, int *err = nullptr, int spin_limit = 0,
                            unsigned *bailed = nullptr, int bail_limit = 2048);
int lstm_gram_counters(int B, int T, int W);
hipError_t launch_lstm_clip_gate(const unsigned *started, int B, int W, unsigned epoch, int *err,
                                 int spin_limit, hipStream_t s);
hipError_t launch_lstm_clip_weights(const float *D, const float *hbuf, const float *x, double *gram,
                                    double *coef, float *w, int B, int T, int I, int H, int W,
                                    hipStream_t s);
hipError_t launch_lstm_weight(float *D, const float *w, float *S, int B, int T, int H,
                              hipStream_t s);

// ---- Transformer path ----
// bad (may be null): per-sample flag, 1 when one of its ids lies outside [0, V)
// bad_or: only set flags (a later Embedding of the network adds its samples)
hipError_t launch_embed(const float *x, const float *E, int32_t *ids, float *out, int B, int T, int V,
                        int D, int32_t *bad, hipStream_t s, bool bad_or = false);
hipError_t launch_pe_add(const float *x, const float *pe, float *out, int B, int TD, hipStream_t s);
// Embedding then PositionalEncoding: out = the embedding rows, pe_out = out + pe[t]
hipError_t launch_embed_pe(const float *x, const float *E, const float *pe, int32_t *ids, float *out,
                           float *pe_out, int B, int T, int V, int D, int32_t *bad, hipStream_t s,
                           bool bad_or = false);
// ws (may be null below 2048 contributing rows): 2 x contributing rows ints.
// pe_grad (may be null; only where embed_grad_takes_pe): the gradient of a
// PositionalEncoding above the Embedding (the same gradient rows summed over
// the samples, times scale), written by the same launch.
bool embed_grad_takes_pe(int B, int T, int W);
// upd: the step's Adam update carried by the launch (its rows, the zeroed
// rows with g = 0, the PositionalEncoding's gradient, and upd->rest's float4
// ranges by extra blocks); only where embed_grad_upd_ok.
bool embed_grad_upd_ok(int B, int T, int D, int W, const float *gradE, const float *rest, int64_t stride);
hipError_t launch_embed_grad(const float *g, const int32_t *ids, float *gradE, int V, int B, int T,
                             int D, int W, float scale, const int32_t *bad, hipStream_t s,
                             float *ws = nullptr, size_t ws_floats = 0, float *pe_grad = nullptr,
                             const AdamStep *upd = nullptr);
hipError_t launch_cls_fwd(const float *x, float *out, int B, int TD, int D, hipStream_t s);
hipError_t launch_cls_bwd(const float *g, float *gin, int B, int TD, int D, hipStream_t s);
hipError_t launch_gap1d_fwd(const float *x, float *out, int B, int T, int D, hipStream_t s);
hipError_t launch_gap1d_bwd(const float *g, float *gin, int B, int T, int D, hipStream_t s);
hipError_t launch_token_sum(const float *X, float *S, int B, int T, int N, hipStream_t s);
// nmem token sums in one launch: member m reads X + m*xstride, writes S + m*sstride
hipError_t launch_token_sum_multi(const float *X, float *S, int B, int T, int N, int nmem,
                                  int64_t xstride, int64_t sstride, hipStream_t s);
// Up to three Linear layers' Q10 gradients from per-sample token sums:
// dW[o][i] = scale * sum_b S[b][o] X[b][i], db[o] = scale * sum_b S[b][o]
// (S pitch lds, X rows pitch ldx, dW M x N dense), b ascending.
struct TokDwSet {
  const float *S[3];
  const float *X[3];
  float *dW[3];
  float *db[3];
};
hipError_t launch_tok_dw(const TokDwSet &set, int nmem, int B, int M, int N, int lds, int ldx,
                         float scale, hipStream_t s);
// The parameter gradients of a transformer block's backward in one launch:
// up to six Linear layers' Q10 gradients (tok_dw's products; the token sums
// of sample b are S[b * np * ps + o] for np = 1, or the sum of np per-row-block
// partial rows S[(b * np + j) * ps + o], j ascending) and up to two
// LayerNorms' gamma / beta gradients from their backward's block partials
// (ln_param_final's sums).  launch_tb_params fills `start` (LayerNorm jobs'
// blocks first, then the Linear jobs').
struct TbParamJob {
  const float *S;
  int np;
  int64_t ps;
  const float *X;  // the last token's input row of sample 0; sample b at X + b * ldx
  int64_t ldx;
  float *dW, *db;
  int M, N;
};
struct TbLnJob {
  const float *part;  // nblk rows of [dgamma partial | dbeta partial], 2N each
  int nblk, N;
  float *dgam, *dbet;
};
constexpr int TBP_MAXLIN = 6, TBP_MAXLN = 2;
struct TbParamSet {
  TbParamJob lin[TBP_MAXLIN];
  TbLnJob ln[TBP_MAXLN];
  int nlin, nln;
  int start[TBP_MAXLIN + TBP_MAXLN + 1];
};
hipError_t launch_tb_params(TbParamSet &set, int B, float scale, hipStream_t s);
// cls (may be null): rows r with r % clsT == 0 are also written as row r / clsT of cls
hipError_t launch_ln_fwd(const float *x, const float *gam, const float *bet, float *y, float *stats,
                         int rows, int N, float eps, hipStream_t s, float *cls = nullptr, int clsT = 0);
hipError_t launch_ln_bwd_params(const float *g, const float *x, const float *gam, const float *stats,
                                float *dx, float *dgam, float *dbet, int rows, int N, float scale,
                                float *ws, size_t ws_cap, hipStream_t s);
// LayerNorm backward, dx and per-block partials only: part [ln_bwd_blocks(rows)][2N]
// (dgamma | dbeta, unscaled; a TbLnJob sums them), tsum (may be null) [blocks][N]
// the blocks' column sums of dx (ln_bwd_rows_per_block() rows each).  gpool (may
// be null, then g is read): a CLSPooling's gradient, row r / poolT for rows r
// with r % poolT == 0, zero elsewhere.  tsx (may be null): the same launch
// also writes tss[b][c] = sum_t tsx[b][t][c] (tsB samples of tsT x tsN), the
// per-sample token sums of another matrix.
int ln_bwd_blocks(int rows);
int ln_bwd_rows_per_block();
bool ln_bwd_part_supported(int N);
hipError_t launch_ln_bwd_part(const float *g, const float *gpool, int poolT, const float *x,
                              const float *gam, const float *stats, float *dx, float *part, float *tsum,
                              int rows, int N, hipStream_t s, const float *tsx = nullptr,
                              float *tss = nullptr, int tsB = 0, int tsT = 0, int tsN = 0);
hipError_t launch_ln_bwd(const float *g, const float *x, const float *gam, const float *stats,
                         float *dx, float *gx, int rows, int N, hipStream_t s);
// Rotary embedding of rows [rows, NH*hd] in place; position = row % T; cs/sn
// are [T][hd/2] tables; conj rotates the other way.
hipError_t launch_rope(float *x, const float *cs, const float *sn, int rows, int T, int NH, int hd,
                       int conj, hipStream_t s);
hipError_t launch_rms_fwd(const float *x, const float *gam, float *y, float *rms, int rows, int N,
                          float eps, hipStream_t s);
hipError_t launch_rms_bwd(const float *g, const float *x, const float *gam, const float *rms,
                          float *dx, float *gx, int rows, int N, hipStream_t s);
bool attn_supported(int T, int D, int NH);  // the fused kernels: T <= 128, D / NH <= 32
// Attention of any T and head size through batched GEMMs over the (sample,
// head) pairs and row kernels: the scores / probabilities and their
// gradients are materialised in `S` (attn_gemm_floats(B, T, NH) floats)
size_t attn_gemm_floats(int B, int T, int NH);
hipError_t launch_attn_fwd_gemm(const float *Q, const float *K, const float *V, float *O, int B, int T,
                                int D, int NH, int causal, float *S, hipStream_t s);
hipError_t launch_attn_bwd_gemm(const float *Q, const float *K, const float *V, const float *GO,
                                float *GQ, float *GK, float *GV, int B, int T, int D, int NH, int causal,
                                float *S, hipStream_t s);
hipError_t launch_attn_fwd(const float *Q, const float *K, const float *V, float *O, int B, int T,
                           int D, int NH, int causal, hipStream_t s);
// TS (may be null): the per-sample token sums of gQ, gK, gV ([B][D] each, member m at TS + m * tss)
hipError_t launch_attn_bwd(const float *Q, const float *K, const float *V, const float *GO,
                           float *GQ, float *GK, float *GV, int B, int T, int D, int NH, int causal,
                           hipStream_t s, float *TS = nullptr, int64_t tss = 0);


// ---- model views for the checkpoint writers (gn_runtime.hip) ----
int model_layer_count(gn_model *M);
const gn_layer_desc *model_layer_desc(gn_model *M, int i);
int model_loss_kind(gn_model *M);
std::vector<uint64_t> *model_noise_streams(gn_model *M, int i);  // MoE, else null
void model_set_timestep(gn_model *M, int t);
int model_timestep(gn_model *M);
const gn_adam_desc &model_adam(gn_model *M);
bool model_master_dims(gn_model *M);  // a forward pass ran on the network's own layers
void model_layer_geom(gn_model *M, int i, ConvShape *cs, PoolShape *ps, float *eps);
int model_error(gn_model *M, int code, const char *fmt, ...);    // records and returns code

}  // namespace gn
