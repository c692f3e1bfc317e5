// Per-layer operators on device pointers: batched stand-ins for the
// per-sample Layer.Forward / Backward calls of the reference
// (internal/layer/layer.go:84-132) and for the per-layer Metal entry points
// they replace (internal/layer/metal.go:6-50), built from the kernels the
// whole-model step uses.
//
// Conventions: B samples, each in the reference's flat per-sample layout,
// row-major; parameter gradients are written (not accumulated) and scaled by
// `scale` (1/B gives the batch average of Network.TrainBatch); an input
// gradient is written when its pointer is not null.  Calls queue work on the
// context's stream and return without synchronising.
#include <math.h>

#include <algorithm>
#include <vector>

#include "gn_ctx.h"

namespace {

int conv_shape(gn_ctx *c, ConvShape &cs, int B, int inC, int H, int W, int outC, int k, int stride,
               int pad) {
  if (B <= 0 || inC <= 0 || H <= 0 || W <= 0 || outC <= 0 || k <= 0 || stride <= 0 || pad < 0)
    return set_err(c, GN_ERR_INVALID, "bad Conv2D geometry");
  cs.inC = inC;
  cs.outC = outC;
  cs.k = k;
  cs.stride = stride;
  cs.pad = pad;
  cs.H = H;
  cs.W = W;
  cs.oH = (H + 2 * pad - k) / stride + 1;
  cs.oW = (W + 2 * pad - k) / stride + 1;
  if (cs.oH <= 0 || cs.oW <= 0) return set_err(c, GN_ERR_SHAPE, "Conv2D output would be empty");
  return GN_OK;
}

int pool_shape(gn_ctx *c, PoolShape &ps, int B, int C, int H, int W, int k, int stride, int pad) {
  if (B <= 0 || C <= 0 || H <= 0 || W <= 0 || k <= 0 || stride <= 0 || pad < 0)
    return set_err(c, GN_ERR_INVALID, "bad MaxPool2D geometry");
  ps.C = C;
  ps.k = k;
  ps.stride = stride;
  ps.pad = pad;
  ps.H = H;
  ps.W = W;
  ps.oH = (H + 2 * pad - k) / stride + 1;
  ps.oW = (W + 2 * pad - k) / stride + 1;
  if (ps.oH <= 0 || ps.oW <= 0) return set_err(c, GN_ERR_SHAPE, "MaxPool2D output would be empty");
  return GN_OK;
}

// regions of a caller workspace, each 64 floats (256 B) aligned
struct Carve {
  float *base;
  size_t off = 0;
  explicit Carve(float *b) : base(b) {}
  float *take(size_t n) {
    float *p = base ? base + off : nullptr;
    off += (n + 63) / 64 * 64;
    return p;
  }
};

}  // namespace

// ---------------------------------------------------------------------------
// Conv2D (conv2d.go:716-1174): out = act(conv(x, W) + b), per sample NCHW;
// params = [W (outC x inC x k x k) | b (outC)], the layer's Params() layout.
// The backward forms dz = gout * act'(out), writes [dW | db] = scale * sums
// over the batch and, when gin is set, the input gradient (col2im).
// ---------------------------------------------------------------------------
extern "C" int gn_conv2d_forward(gn_ctx *c, const float *x, const float *params, float *out,
                                 int32_t B, int32_t inC, int32_t H, int32_t W, int32_t outC,
                                 int32_t k, int32_t stride, int32_t pad, int32_t act) {
  ENTRY(c);
  ConvShape cs{};
  int rc = conv_shape(c, cs, B, inC, H, W, outC, k, stride, pad);
  if (rc) return rc;
  if (!x || !params || !out) return set_err(c, GN_ERR_INVALID, "null pointer");
  int fwd = 0, deriv = 0;
  if (plan_scalar_act(act, fwd, deriv)) return set_err(c, GN_ERR_INVALID, "unknown activation %d", act);
  KTimer kt(c, GN_KCLASS_OTHER, "conv_fwd", conv_flops(cs, B));
  HIP_OK(c, launch_conv_fwd(x, params, params + (int64_t)outC * inC * k * k, out, cs, B, fwd, c->stream));
  return GN_OK;
}

extern "C" int gn_conv2d_backward(gn_ctx *c, const float *x, const float *params, const float *out,
                                  const float *gout, float *grads, float *gin, int32_t B, int32_t inC,
                                  int32_t H, int32_t W, int32_t outC, int32_t k, int32_t stride,
                                  int32_t pad, int32_t act, float scale) {
  ENTRY(c);
  ConvShape cs{};
  int rc = conv_shape(c, cs, B, inC, H, W, outC, k, stride, pad);
  if (rc) return rc;
  if (!x || !params || !out || !gout || !grads) return set_err(c, GN_ERR_INVALID, "null pointer");
  int fwd = 0, deriv = 0;
  if (plan_scalar_act(act, fwd, deriv)) return set_err(c, GN_ERR_INVALID, "unknown activation %d", act);
  {
    KTimer kt(c, GN_KCLASS_OTHER, "conv_wgrad", conv_flops(cs, B) + 2.0 * B * outC * cs.oH * cs.oW);
    HIP_OK(c, launch_conv_wgrad(x, gout, out, grads, cs, B, deriv, scale, c->scratch, c->scratch_floats,
                                c->stream));
  }
  if (gin) {
    KTimer kt(c, GN_KCLASS_OTHER, "conv_dgrad", conv_flops(cs, B));
    HIP_OK(c, launch_conv_dgrad(gout, out, params, gin, cs, B, deriv, c->stream));
  }
  return GN_OK;
}

// ---------------------------------------------------------------------------
// MaxPool2D (maxpool2d.go:106-410): strict-greater first maximum of each
// window (padding never wins); argmax holds the flat input index (inside the
// sample) of every output, int32.  The backward sums gout into the winners.
// ---------------------------------------------------------------------------
extern "C" int gn_maxpool2d_forward(gn_ctx *c, const float *x, float *out, int32_t *argmax, int32_t B,
                                    int32_t C, int32_t H, int32_t W, int32_t k, int32_t stride,
                                    int32_t pad) {
  ENTRY(c);
  PoolShape ps{};
  int rc = pool_shape(c, ps, B, C, H, W, k, stride, pad);
  if (rc) return rc;
  if (!x || !out || !argmax) return set_err(c, GN_ERR_INVALID, "null pointer");
  KTimer kt(c, GN_KCLASS_OTHER, "maxpool_fwd", f4((double)B * C * H * W + 2.0 * B * C * ps.oH * ps.oW));
  HIP_OK(c, launch_maxpool_fwd(x, out, argmax, ps, B, c->stream));
  return GN_OK;
}

extern "C" int gn_maxpool2d_backward(gn_ctx *c, const float *gout, const int32_t *argmax, float *gin,
                                     int32_t B, int32_t C, int32_t H, int32_t W, int32_t k,
                                     int32_t stride, int32_t pad) {
  ENTRY(c);
  PoolShape ps{};
  int rc = pool_shape(c, ps, B, C, H, W, k, stride, pad);
  if (rc) return rc;
  if (!gout || !argmax || !gin) return set_err(c, GN_ERR_INVALID, "null pointer");
  KTimer kt(c, GN_KCLASS_OTHER, "maxpool_bwd", f4(2.0 * B * C * ps.oH * ps.oW + (double)B * C * H * W));
  HIP_OK(c, launch_maxpool_bwd(gout, argmax, gin, ps, B, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// Dropout (dropout.go:47-401).  Training: the mask is the first n draws of
// RNG(42) against p, the same for every sample because Reset reseeds the
// stream before each one (Q9), written to mask (n floats, 0 or 1);
// out = x * mask / (1 - p).  Inference: out = x, and the gradient passes
// unchanged.
// ---------------------------------------------------------------------------
extern "C" int gn_dropout_forward(gn_ctx *c, const float *x, float *out, float *mask, int32_t B,
                                  int32_t n, float p, int32_t training) {
  ENTRY(c);
  if (!x || !out || B <= 0 || n <= 0 || (training && !mask)) return set_err(c, GN_ERR_INVALID, "bad dropout args");
  if (!(p >= 0 && p <= 1)) return set_err(c, GN_ERR_INVALID, "dropout p %g outside [0, 1]", p);
  if (!training) {
    HIP_OK(c, hipMemcpyAsync(out, x, (size_t)B * n * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
    return GN_OK;
  }
  HIP_OK(c, launch_dropout_mask(mask, n, p, c->stream));
  const float keep = 1.0f - p;
  KTimer kt(c, GN_KCLASS_OTHER, "dropout", f4(2.0 * B * n + n));
  HIP_OK(c, launch_dropout(x, mask, 1.0f / keep, out, B, n, c->stream));
  return GN_OK;
}

extern "C" int gn_dropout_backward(gn_ctx *c, const float *gout, const float *mask, float *gin,
                                   int32_t B, int32_t n, float p, int32_t training) {
  ENTRY(c);
  if (!gout || !gin || B <= 0 || n <= 0 || (training && !mask))
    return set_err(c, GN_ERR_INVALID, "bad dropout args");
  if (!(p >= 0 && p <= 1)) return set_err(c, GN_ERR_INVALID, "dropout p %g outside [0, 1]", p);
  if (!training) {
    HIP_OK(c, hipMemcpyAsync(gin, gout, (size_t)B * n * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
    return GN_OK;
  }
  const float keep = 1.0f - p;
  KTimer kt(c, GN_KCLASS_OTHER, "dropout", f4(2.0 * B * n + n));
  HIP_OK(c, launch_dropout(gout, mask, 1.0f / keep, gin, B, n, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// Output layer: activation + loss + loss gradient through the activation
// (Dense's Softmax / LogSoftmax Jacobian, layer.go:504-567; loss.go:53-178).
// zo holds the pre-activations of B rows of C and receives the activation
// output; dz the gradient at the pre-activations; loss_rows the per-sample
// losses.
// ---------------------------------------------------------------------------
extern "C" int gn_softmax_ce_backward(gn_ctx *c, float *zo, const float *y, float *dz, float *loss_rows,
                                      int32_t B, int32_t C, int32_t act, int32_t act_is_ptr,
                                      int32_t loss_kind) {
  ENTRY(c);
  if (!zo || !y || !dz || !loss_rows || B <= 0 || C <= 0)
    return set_err(c, GN_ERR_INVALID, "bad softmax_ce args");
  if (loss_kind != GN_LOSS_MSE && loss_kind != GN_LOSS_CE)
    return set_err(c, GN_ERR_INVALID, "unknown loss %d", loss_kind);
  ActPlan ap;
  if (plan_act(act, act_is_ptr, ap)) return set_err(c, GN_ERR_INVALID, "unknown activation %d", act);
  KTimer kt(c, GN_KCLASS_OTHER, "out_rows", f4(4.0 * B * C + B));
  HIP_OK(c, launch_out_rows(zo, y, zo, dz, loss_rows, B, C, ap.row_act, ap.deriv, loss_kind, nullptr, 1,
                            c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// LayerNorm (layernorm.go:193-441) over rows of N: y = gamma (x - mean) / std
// + beta with std = sqrt(var + eps) (eps 0 selects 1e-5); stats keeps (mean,
// std) per row for the backward, whose dx follows the reference's formula
// (its last term uses N std^2; Q18).  work: rows x N floats of scratch for
// g * xhat.  dgamma / dbeta = scale * sums over the rows.
// ---------------------------------------------------------------------------
extern "C" int gn_layernorm_forward(gn_ctx *c, const float *x, const float *gamma, const float *beta,
                                    float *y, float *stats, int32_t rows, int32_t N, float eps) {
  ENTRY(c);
  if (!x || !gamma || !beta || !y || !stats || rows <= 0 || N <= 0 || !(eps >= 0))
    return set_err(c, GN_ERR_INVALID, "bad layernorm args");
  KTimer kt(c, GN_KCLASS_OTHER, "ln_fwd", f4(2.0 * rows * N + 2.0 * rows));
  HIP_OK(c, launch_ln_fwd(x, gamma, beta, y, stats, rows, N, eps > 0 ? eps : 1e-5f, c->stream));
  return GN_OK;
}

extern "C" int gn_layernorm_backward(gn_ctx *c, const float *g, const float *x, const float *gamma,
                                     const float *stats, float *dx, float *dgamma, float *dbeta,
                                     float *work, int32_t rows, int32_t N, float scale) {
  ENTRY(c);
  if (!g || !x || !gamma || !stats || !dx || !dgamma || !dbeta || !work || rows <= 0 || N <= 0)
    return set_err(c, GN_ERR_INVALID, "bad layernorm args");
  {
    KTimer kt(c, GN_KCLASS_OTHER, "ln_bwd", f4(4.0 * rows * N + 2.0 * rows));
    HIP_OK(c, launch_ln_bwd(g, x, gamma, stats, dx, work, rows, N, c->stream));
  }
  const float *src[2] = {work, g};
  float *dst[2] = {dgamma, dbeta};
  KTimer kt(c, GN_KCLASS_OTHER, "colsum", 2 * f4((double)rows * N + N));
  HIP_OK(c, launch_colsum_multi(src, dst, 2, rows, N, N, scale, c->scratch, c->scratch_floats, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// MultiHeadAttention (transformer.go:277-690): x is B x T x D; params =
// [wQ (W D x D, b D) | wK | wV | wOut].  Q, K, V are Linear Dense layers per
// token (RoPE on Q, K when use_rope), scaled dot-product attention per head
// (causal mask -1e9), out = wOut(attention).  The backward is the per-token
// Dense backward of the reference (the weight gradients use the last token's
// input, Q10), the attention backward, the conjugate rotation.  work holds
// what the forward saves for the backward (gn_mha_workspace floats); the
// forward and backward of one batch must share it and x.
// ---------------------------------------------------------------------------
namespace {
MhaBufs mha_carve(float *w, int B, int T, int D, int NH, int rope, size_t *floats) {
  Carve cv(w);
  MhaBufs m{};
  const size_t rows = (size_t)B * T;
  m.Q = cv.take(3 * rows * D);
  m.K = m.Q ? m.Q + rows * D : nullptr;
  m.V = m.K ? m.K + rows * D : nullptr;
  m.O = cv.take(rows * D);
  m.GO = cv.take(rows * D);
  m.GQ = cv.take(3 * rows * D);
  m.GK = m.GQ ? m.GQ + rows * D : nullptr;
  m.GV = m.GK ? m.GK + rows * D : nullptr;
  m.S = cv.take((size_t)B * D);
  m.S3 = cv.take(3 * (size_t)B * D);
  m.s3_stride = (int64_t)B * D;
  const size_t half = (size_t)std::max(D / std::max(NH, 1) / 2, 1);
  m.rcos = rope ? cv.take((size_t)T * half) : nullptr;
  m.rsin = rope ? cv.take((size_t)T * half) : nullptr;
  m.SC = attn_supported(T, D, NH) ? nullptr : cv.take(attn_gemm_floats(B, T, NH));
  if (floats) *floats = cv.off;
  return m;
}
int mha_check(gn_ctx *c, int B, int T, int D, int NH) {
  if (B <= 0 || T <= 0 || D <= 0 || NH <= 0 || D % NH) return set_err(c, GN_ERR_INVALID, "bad MHA sizes");
  return GN_OK;
}
}  // namespace

// applyRoPE's angles (transformer.go:215-221) in float32, as the reference
void rope_tables(int T, int hd, std::vector<float> &cs, std::vector<float> &sn) {
  const int half = hd / 2;
  cs.assign((size_t)T * std::max(half, 1), 0.f);
  sn.assign(cs.size(), 0.f);
  for (int t = 0; t < T; ++t)
    for (int k = 0; k < half; ++k) {
      const float theta = (float)pow(10000.0, -(double)(2 * k) / (double)hd);
      const float mt = (float)t * theta;
      cs[(size_t)t * half + k] = (float)cos((double)mt);
      sn[(size_t)t * half + k] = (float)sin((double)mt);
    }
}

// The MultiHeadAttention forward over B samples (transformer.go:405-527):
// Q, K, V projections in one batched GEMM (their weights, biases and output
// buffers equally spaced), RoPE, attention, out = wOut(attention).
int mha_forward_impl(gn_ctx *c, const float *x, const float *params, float *out, const MhaBufs &m,
                     int B, int T, int D, int NH, int causal, int rope) {
  const int rows = B * T, hd = D / NH;
  const int64_t nd = (int64_t)D * D + D;
  {
    GemmArgs a{};
    a.M = rows; a.N = D; a.K = D;
    a.A = x; a.lda = D; a.B = params; a.ldb = D;
    a.C = m.Q; a.ldc = D; a.alpha = 1.f; a.bias = params + (int64_t)D * D; a.act = F_IDENTITY;
    a.ws = c->scratch; a.ws_cap = c->scratch_floats;
    a.nbatch = 3;
    a.bstride_B = nd;
    a.bstride_bias = nd;
    a.bstride_C = m.K - m.Q;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(a));
    HIP_OK(c, launch_gemm('N', 'T', EPI_BIAS_ACT, a, c->stream));
  }
  if (rope) {
    KTimer kt(c, GN_KCLASS_OTHER, "rope", 2 * f4(2.0 * rows * D));
    HIP_OK(c, launch_rope(m.Q, m.rcos, m.rsin, rows, T, NH, hd, 0, c->stream));
    HIP_OK(c, launch_rope(m.K, m.rcos, m.rsin, rows, T, NH, hd, 0, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "attn_fwd", attn_flops(B, T, NH, hd, causal, false));
    if (m.SC)
      HIP_OK(c, launch_attn_fwd_gemm(m.Q, m.K, m.V, m.O, B, T, D, NH, causal, m.SC, c->stream));
    else
      HIP_OK(c, launch_attn_fwd(m.Q, m.K, m.V, m.O, B, T, D, NH, causal, c->stream));
  }
  GemmArgs o{};
  o.M = rows; o.N = D; o.K = D;
  o.A = m.O; o.lda = D; o.B = params + 3 * nd; o.ldb = D;
  o.C = out; o.ldc = D; o.alpha = 1.f; o.bias = params + 3 * nd + (int64_t)D * D; o.act = F_IDENTITY;
  o.ws = c->scratch; o.ws_cap = c->scratch_floats;
  KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(o));
  HIP_OK(c, launch_gemm('N', 'T', EPI_BIAS_ACT, o, c->stream));
  return GN_OK;
}

// The MultiHeadAttention backward (transformer.go:557-690): wOut, the
// attention, the conjugate rotation, then wQ, wK, wV, each a per-token Linear
// Dense whose weight gradient uses the last token's input (Q10) and whose
// bias gradient sums every token: both from the per-sample token sums, one
// launch per Linear (three for Q, K, V together).  gin (may be null) = gQ Wq
// + gK Wk + gV Wv.
int mha_backward_impl(gn_ctx *c, const float *x, const float *params, const float *gout, float *grads,
                      float *gin, const MhaBufs &m, int B, int T, int D, int NH, int causal, int rope,
                      float scale) {
  const int rows = B * T, hd = D / NH;
  const int64_t nd = (int64_t)D * D + D;
  float *G = grads;
  float *cs = c->scratch;
  const size_t cap = c->scratch_floats;
  {
    KTimer kt(c, GN_KCLASS_OTHER, "token_sum", token_sum_bytes(B, T, D));
    HIP_OK(c, launch_token_sum(gout, m.S, B, T, D, c->stream));
  }
  {
    TokDwSet set{};  // dWo = scale S^T O_last, dbo = scale colsum(S)
    set.S[0] = m.S;
    set.X[0] = m.O + (int64_t)(T - 1) * D;
    set.dW[0] = G + 3 * nd;
    set.db[0] = G + 3 * nd + (int64_t)D * D;
    KTimer kt(c, GN_KCLASS_OTHER, "tok_dw", f4(2.0 * B * D + (double)D * D + D));
    HIP_OK(c, launch_tok_dw(set, 1, B, D, D, D, T * D, scale, c->stream));
  }
  {
    GemmArgs a{};  // GO = gout Wo
    a.M = rows; a.N = D; a.K = D;
    a.A = gout; a.lda = D; a.B = params + 3 * nd; a.ldb = D;
    a.C = m.GO; a.ldc = D; a.alpha = 1.f;
    a.ws = cs; a.ws_cap = cap;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
    HIP_OK(c, launch_gemm('N', 'N', EPI_SCALE, a, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "attn_bwd", attn_flops(B, T, NH, hd, causal, true));
    if (m.SC)
      HIP_OK(c, launch_attn_bwd_gemm(m.Q, m.K, m.V, m.GO, m.GQ, m.GK, m.GV, B, T, D, NH, causal, m.SC,
                                     c->stream));
    else
      HIP_OK(c, launch_attn_bwd(m.Q, m.K, m.V, m.GO, m.GQ, m.GK, m.GV, B, T, D, NH, causal, c->stream));
  }
  if (rope) {  // transformer.go:660-664: the conjugate rotation before wQ / wK
    KTimer kt(c, GN_KCLASS_OTHER, "rope", 2 * f4(2.0 * rows * D));
    HIP_OK(c, launch_rope(m.GQ, m.rcos, m.rsin, rows, T, NH, hd, 1, c->stream));
    HIP_OK(c, launch_rope(m.GK, m.rcos, m.rsin, rows, T, NH, hd, 1, c->stream));
  }
  const int64_t sst = m.s3_stride;
  {
    KTimer kt(c, GN_KCLASS_OTHER, "token_sum", 3 * token_sum_bytes(B, T, D));
    HIP_OK(c, launch_token_sum_multi(m.GQ, m.S3, B, T, D, 3, m.GK - m.GQ, sst, c->stream));
  }
  {
    TokDwSet set{};
    for (int z = 0; z < 3; ++z) {
      set.S[z] = m.S3 + z * sst;
      set.X[z] = x + (int64_t)(T - 1) * D;
      set.dW[z] = G + z * nd;
      set.db[z] = G + z * nd + (int64_t)D * D;
    }
    KTimer kt(c, GN_KCLASS_OTHER, "tok_dw", 3 * f4(2.0 * B * D + (double)D * D + D));
    HIP_OK(c, launch_tok_dw(set, 3, B, D, D, D, T * D, scale, c->stream));
  }
  if (gin) {
    const float *gq[3] = {m.GQ, m.GK, m.GV};
    for (int i = 0; i < 3; ++i) {
      GemmArgs a{};
      a.M = rows; a.N = D; a.K = D;
      a.A = gq[i]; a.lda = D; a.B = params + i * nd; a.ldb = D;
      a.C = gin; a.ldc = D; a.alpha = 1.f;
      a.aux = gin; a.ldaux = D;
      a.ws = cs; a.ws_cap = cap;
      KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
      HIP_OK(c, launch_gemm('N', 'N', i == 0 ? EPI_SCALE : EPI_BIAS_ADD, a, c->stream));
    }
  }
  return GN_OK;
}

extern "C" int gn_mha_workspace(int32_t B, int32_t T, int32_t D, int32_t heads, int32_t use_rope,
                                int64_t *floats) {
  if (!floats || B <= 0 || T <= 0 || D <= 0 || heads <= 0) return GN_ERR_INVALID;
  size_t n = 0;
  mha_carve(nullptr, B, T, D, heads, use_rope, &n);
  *floats = (int64_t)n;
  return GN_OK;
}

extern "C" int gn_mha_forward(gn_ctx *c, const float *x, const float *params, float *out, float *work,
                              int32_t B, int32_t T, int32_t D, int32_t heads, int32_t causal,
                              int32_t use_rope) {
  ENTRY(c);
  int rc = mha_check(c, B, T, D, heads);
  if (rc) return rc;
  if (!x || !params || !out || !work) return set_err(c, GN_ERR_INVALID, "null pointer");
  MhaBufs m = mha_carve(work, B, T, D, heads, use_rope, nullptr);
  if (use_rope) {
    std::vector<float> cs, sn;
    rope_tables(T, D / heads, cs, sn);
    HIP_OK(c, hipMemcpyAsync(m.rcos, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice, c->stream));
    HIP_OK(c, hipMemcpyAsync(m.rsin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice, c->stream));
    HIP_OK(c, hipStreamSynchronize(c->stream));  // the host tables go out of scope
  }
  return mha_forward_impl(c, x, params, out, m, B, T, D, heads, causal, use_rope);
}

extern "C" int gn_mha_backward(gn_ctx *c, const float *x, const float *params, const float *gout,
                               float *grads, float *gin, float *work, int32_t B, int32_t T, int32_t D,
                               int32_t heads, int32_t causal, int32_t use_rope, float scale) {
  ENTRY(c);
  int rc = mha_check(c, B, T, D, heads);
  if (rc) return rc;
  if (!x || !params || !gout || !grads || !work) return set_err(c, GN_ERR_INVALID, "null pointer");
  MhaBufs m = mha_carve(work, B, T, D, heads, use_rope, nullptr);
  return mha_backward_impl(c, x, params, gout, grads, gin, m, B, T, D, heads, causal, use_rope, scale);
}

// ---------------------------------------------------------------------------
// SequenceUnroller(LSTM) (unroller.go:57-213, lstm.go:144-751) over a batch:
// x is B x T x I, params = [Wx (4H x I) | Wh (4H x H) | b (4H)], gates i, f,
// g, o; out = h_{T-1} (B x H).  The reference's quirks are kept: only the
// input gate adds Wx x + Wh h (Q13); dWx uses the last step's input (Q10);
// dh_{t-1} = dh_t + Wh^T dG (Q15); each worker chain's cumulative gradient is
// clipped to norm 1 after every step (Q14, `workers` chains of ceil(B /
// workers) samples, evaluated exactly through the chain's Gram matrix).  The
// input gradient (gin, B x T x I) uses the unclipped deltas, as the
// reference's dx does.  With return_sequences, out and gout are B x T x H,
// every step's h (unroller.go:85-127, 158-188).  work holds what the forward saves (gn_lstm_workspace
// floats for the same B, T, I, H, workers).
// ---------------------------------------------------------------------------
namespace {
struct LstmWork {
  float *WhT, *xw, *igb, *tcb, *cbuf, *hbuf, *Dg, *S, *wts;
  double *gram, *coef;
  size_t floats;
};
LstmWork lstm_carve(float *w, int B, int T, int I, int H, int workers) {
  Carve cv(w);
  LstmWork m{};
  const size_t Bm = B, TT = T, HH = H;
  m.WhT = cv.take(HH * HH);
  m.xw = cv.take(Bm * TT * HH);
  m.igb = cv.take(Bm * TT * HH);
  m.tcb = cv.take(Bm * TT * HH);
  m.cbuf = cv.take(Bm * TT * HH);
  m.hbuf = cv.take(Bm * (TT + 1) * HH);
  m.Dg = cv.take(Bm * (TT + 1) * 4 * HH);
  m.S = cv.take(Bm * 4 * HH);
  m.wts = cv.take(Bm * (TT + 1));
  const int Wc = std::min(std::max(workers, 1), B);
  const size_t chunk = (B + Wc - 1) / Wc;
  const size_t nmax = (size_t)lstm_gram_pitch((int)(chunk * T));
  const size_t nchains = (B + chunk - 1) / chunk;
  m.gram = reinterpret_cast<double *>(cv.take(2 * nchains * nmax * nmax));
  m.coef = reinterpret_cast<double *>(cv.take(2 * nchains * nmax));
  m.floats = cv.off;
  (void)I;
  return m;
}
}  // namespace

extern "C" int gn_lstm_workspace(int32_t B, int32_t T, int32_t I, int32_t H, int32_t workers,
                                 int64_t *floats) {
  if (!floats || B <= 0 || T <= 0 || I <= 0 || H <= 0) return GN_ERR_INVALID;
  *floats = (int64_t)lstm_carve(nullptr, B, T, I, H, workers).floats;
  return GN_OK;
}

extern "C" int gn_lstm_seq_forward(gn_ctx *c, const float *x, const float *params, float *out,
                                   float *work, int32_t B, int32_t T, int32_t I, int32_t H,
                                   int32_t return_sequences) {
  ENTRY(c);
  if (!x || !params || !out || !work || B <= 0 || T <= 0 || I <= 0 || H <= 0 || H > 1024)
    return set_err(c, GN_ERR_INVALID, "bad LSTM args (hidden <= 1024)");
  LstmWork m = lstm_carve(work, B, T, I, H, 1);
  const float *Wx = params, *Wh = Wx + (int64_t)4 * H * I, *bias = Wh + (int64_t)4 * H * H;
  {
    GemmArgs g{};  // xw[b*T + t] = x_t . Wx_i (the input-gate rows, Q13)
    g.M = B * T; g.N = H; g.K = I;
    g.A = x; g.lda = I; g.B = Wx; g.ldb = I;
    g.C = m.xw; g.ldc = H; g.alpha = 1.f;
    g.ws = c->scratch; g.ws_cap = c->scratch_floats;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(g));
    HIP_OK(c, launch_gemm('N', 'T', EPI_SCALE, g, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "transpose", f4(2.0 * H * H));
    HIP_OK(c, launch_transpose(Wh, m.WhT, H, H, c->stream));
  }
  KTimer kt(c, GN_KCLASS_OTHER, "lstm_fwd", 2.0 * H * H * B * T);
  HIP_OK(c, launch_lstm_fwd(m.xw, m.WhT, bias, m.igb, m.tcb, m.cbuf, m.hbuf, out, B, T, H, c->stream,
                            return_sequences ? 1 : 0));
  return GN_OK;
}

extern "C" int gn_lstm_seq_backward(gn_ctx *c, const float *x, const float *params, const float *gout,
                                    float *grads, float *gin, float *work, int32_t B, int32_t T,
                                    int32_t I, int32_t H, int32_t workers, float scale,
                                    int32_t return_sequences) {
  ENTRY(c);
  if (!x || !params || !gout || !grads || !work || B <= 0 || T <= 0 || I <= 0 || H <= 0 || H > 1024)
    return set_err(c, GN_ERR_INVALID, "bad LSTM args (hidden <= 1024)");
  // the forward's saved state sits where the carve of the same sizes puts it;
  // the Gram buffers (after it) are sized for `workers`
  LstmWork m = lstm_carve(work, B, T, I, H, workers);
  const int G4 = 4 * H;
  const float *Wx = params, *Wh = Wx + (int64_t)G4 * I, *bias = Wh + (int64_t)G4 * H;
  float *gWx = grads, *gWh = gWx + (int64_t)G4 * I, *gb = gWh + (int64_t)G4 * H;
  {
    KTimer kt(c, GN_KCLASS_OTHER, "lstm_bptt", 2.0 * G4 * H * B * T);
    HIP_OK(c, launch_lstm_bwd(gout, m.igb, m.tcb, m.cbuf, Wh, bias, m.Dg, B, T, H, c->stream,
                              return_sequences ? 1 : 0));
  }
  if (gin) {  // dx_t = Wx^T dG_t for every sample and step, before the clip weights touch dG
    GemmArgs a{};
    a.M = T; a.N = I; a.K = G4;
    a.A = m.Dg; a.lda = G4; a.B = Wx; a.ldb = I;
    a.C = gin; a.ldc = I; a.alpha = 1.f;
    a.ws = c->scratch; a.ws_cap = c->scratch_floats;
    a.nbatch = B;
    a.bstride_A = (int64_t)(T + 1) * G4;
    a.bstride_C = (int64_t)T * I;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
    HIP_OK(c, launch_gemm('N', 'N', EPI_SCALE, a, c->stream));
  }
  const int Wc = std::max(1, std::min(workers, B)), chunk = (B + Wc - 1) / Wc;
  const double nst = (double)chunk * T, nchain = (double)((B + chunk - 1) / chunk);
  {
    KTimer kt(c, GN_KCLASS_OTHER, "lstm_gram", nchain * nst * (nst + 1) * (5.0 * H + I));
    HIP_OK(c, launch_lstm_gram(m.Dg, m.hbuf, x, m.gram, B, T, I, H, workers, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "lstm_clip", nchain * 8.0 * nst * (nst + 1) / 2);
    HIP_OK(c, launch_lstm_clip(m.gram, m.coef, m.wts, B, T, workers, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "lstm_weight", f4(2.0 * B * (T + 1) * G4 + (double)B * G4));
    HIP_OK(c, launch_lstm_weight(m.Dg, m.wts, m.S, B, T, H, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "colsum", f4((double)B * G4 + G4));
    HIP_OK(c, launch_colsum(m.S, B, G4, G4, scale, gb, c->scratch, c->scratch_floats, c->stream));
  }
  GemmArgs a{};  // dWx = scale * S^T x_last
  a.M = G4; a.N = I; a.K = B;
  a.A = m.S; a.lda = G4;
  a.B = x + (int64_t)(T - 1) * I; a.ldb = T * I;
  a.C = gWx; a.ldc = I; a.alpha = scale;
  a.ws = c->scratch; a.ws_cap = c->scratch_floats;
  GemmArgs h{};  // dWh = scale * (w dG)^T hPrev, K over (sample, step)
  h.M = G4; h.N = H; h.K = B * (T + 1);
  h.A = m.Dg; h.lda = G4;
  h.B = m.hbuf; h.ldb = H;
  h.C = gWh; h.ldc = H; h.alpha = scale;
  h.ws = c->scratch; h.ws_cap = c->scratch_floats;
  KTimer kt(c, GN_KCLASS_GEMM, "gemm_dw", gemm_flops(a) + gemm_flops(h));
  HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, a, c->stream));
  HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, h, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// Embedding (embedding.go:79-183): x holds B x T token ids as floats
// (floor(x) is the index); out the rows of E (V x D); ids the int32 indices
// for the backward; bad (optional, B ints) flags the samples with an index
// outside [0, V) (the reference's Forward errors on them; their rows read
// row 0 here).  The backward zeroes gradE and adds the rows of each worker
// chunk's last sample (Embedding.Backward zeroes its gradient first, Q12;
// `workers` chunks of ceil(B / workers); with bad, the last sample of the
// chunk that the reference's loop would still run), times scale.
// ---------------------------------------------------------------------------
extern "C" int gn_embedding_forward(gn_ctx *c, const float *x, const float *E, float *out, int32_t *ids,
                                    int32_t *bad, int32_t B, int32_t T, int32_t V, int32_t D) {
  ENTRY(c);
  if (!x || !E || !out || !ids || B <= 0 || T <= 0 || V <= 0 || D <= 0)
    return set_err(c, GN_ERR_INVALID, "bad embedding args");
  KTimer kt(c, GN_KCLASS_OTHER, "embed_fwd", f4(2.0 * B * T + 2.0 * B * T * D));
  HIP_OK(c, launch_embed(x, E, ids, out, B, T, V, D, bad, c->stream));
  return GN_OK;
}

extern "C" int gn_embedding_backward(gn_ctx *c, const float *gout, const int32_t *ids,
                                     const int32_t *bad, float *gradE, int32_t B, int32_t T, int32_t V,
                                     int32_t D, int32_t workers, float scale) {
  ENTRY(c);
  if (!gout || !ids || !gradE || B <= 0 || T <= 0 || V <= 0 || D <= 0)
    return set_err(c, GN_ERR_INVALID, "bad embedding args");
  const int Wc = std::max(1, std::min(workers, B)), chunk = (B + Wc - 1) / Wc;
  const int nch = (B + chunk - 1) / chunk;
  KTimer kt(c, GN_KCLASS_OTHER, "embed_grad", f4((double)V * D + 2.0 * nch * T * D));
  if ((size_t)2 * nch * T > c->scratch_floats)
    return set_err(c, GN_ERR_UNSUPPORTED, "embedding backward: %d contributing rows exceed the scratch",
                   nch * T);
  HIP_OK(c, launch_embed_grad(gout, ids, gradE, V, B, T, D, workers, scale, bad, c->stream, c->scratch,
                              c->scratch_floats));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// AvgPool2D (avgpool2d.go:137-474): per sample C x H x W, windows k x k with
// stride and zero padding; the mean counts only the positions inside the
// input (count_include_pad false).  The backward spreads each output
// gradient over its window's positions.
// ---------------------------------------------------------------------------
extern "C" int gn_avgpool2d_forward(gn_ctx *c, const float *x, float *out, int32_t B, int32_t C, int32_t H,
                                    int32_t W, int32_t k, int32_t stride, int32_t pad) {
  ENTRY(c);
  PoolShape ps{};
  int rc = pool_shape(c, ps, B, C, H, W, k, stride, pad);
  if (rc) return rc;
  if (!x || !out) return set_err(c, GN_ERR_INVALID, "null pointer");
  KTimer kt(c, GN_KCLASS_OTHER, "avgpool_fwd", f4((double)B * C * H * W + (double)B * C * ps.oH * ps.oW));
  HIP_OK(c, launch_avgpool_fwd(x, out, ps, B, c->stream));
  return GN_OK;
}

extern "C" int gn_avgpool2d_backward(gn_ctx *c, const float *gout, float *gin, int32_t B, int32_t C,
                                     int32_t H, int32_t W, int32_t k, int32_t stride, int32_t pad) {
  ENTRY(c);
  PoolShape ps{};
  int rc = pool_shape(c, ps, B, C, H, W, k, stride, pad);
  if (rc) return rc;
  if (!gout || !gin) return set_err(c, GN_ERR_INVALID, "null pointer");
  KTimer kt(c, GN_KCLASS_OTHER, "avgpool_bwd", f4((double)B * C * ps.oH * ps.oW + (double)B * C * H * W));
  HIP_OK(c, launch_avgpool_bwd(gout, gin, ps, B, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// RMSNorm (rmsnorm.go:222-329) over rows of N: y = gamma x / rms, rms =
// sqrt(mean(x^2) + eps) (eps 0 selects 1e-5); the backward is the
// reference's formula (its projection term is scaled by gamma_j, Q19).
// work: rows x N floats (g x / rms for the gamma sums).
// ---------------------------------------------------------------------------
extern "C" int gn_rmsnorm_forward(gn_ctx *c, const float *x, const float *gamma, float *y, float *rms,
                                  int32_t rows, int32_t N, float eps) {
  ENTRY(c);
  if (!x || !gamma || !y || !rms || rows <= 0 || N <= 0 || !(eps >= 0))
    return set_err(c, GN_ERR_INVALID, "bad rmsnorm args");
  KTimer kt(c, GN_KCLASS_OTHER, "rms_fwd", f4(2.0 * rows * N + rows));
  HIP_OK(c, launch_rms_fwd(x, gamma, y, rms, rows, N, eps > 0 ? eps : 1e-5f, c->stream));
  return GN_OK;
}

extern "C" int gn_rmsnorm_backward(gn_ctx *c, const float *g, const float *x, const float *gamma,
                                   const float *rms, float *dx, float *dgamma, float *work, int32_t rows,
                                   int32_t N, float scale) {
  ENTRY(c);
  if (!g || !x || !gamma || !rms || !dgamma || !work || rows <= 0 || N <= 0)
    return set_err(c, GN_ERR_INVALID, "bad rmsnorm args");
  {
    KTimer kt(c, GN_KCLASS_OTHER, "rms_bwd", f4(4.0 * rows * N + rows));
    HIP_OK(c, launch_rms_bwd(g, x, gamma, rms, dx, work, rows, N, c->stream));
  }
  KTimer kt(c, GN_KCLASS_OTHER, "colsum", f4((double)rows * N + N));
  HIP_OK(c, launch_colsum(work, rows, N, N, scale, dgamma, c->scratch, c->scratch_floats, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// SwiGLU (swiglu.go:103-232): params = [W (out x in) | V (out x in)], no
// biases; y = swish(W x) * (V x).  work: gn_swiglu_workspace floats (the
// projections Z = [W x | V x] and their gradients); forward and backward of
// one batch share it.
// ---------------------------------------------------------------------------
extern "C" int gn_swiglu_workspace(int32_t B, int32_t out, int64_t *floats) {
  if (!floats || B <= 0 || out <= 0) return GN_ERR_INVALID;
  *floats = 4 * (int64_t)B * out;
  return GN_OK;
}

extern "C" int gn_swiglu_forward(gn_ctx *c, const float *x, const float *params, float *out, float *work,
                                 int32_t B, int32_t in, int32_t out_size) {
  ENTRY(c);
  if (!x || !params || !out || !work || B <= 0 || in <= 0 || out_size <= 0)
    return set_err(c, GN_ERR_INVALID, "bad swiglu args");
  const int out2 = 2 * out_size;
  {
    GemmArgs g{};  // Z[b] = [W x_b | V x_b]
    g.M = B; g.N = out2; g.K = in;
    g.A = x; g.lda = in;
    g.B = params; g.ldb = in;
    g.C = work; g.ldc = out2; g.alpha = 1.0f;
    g.ws = c->scratch; g.ws_cap = c->scratch_floats;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(g));
    HIP_OK(c, launch_gemm('N', 'T', EPI_SCALE, g, c->stream));
  }
  KTimer kt(c, GN_KCLASS_OTHER, "swiglu_fwd", f4(3.0 * B * out_size));
  HIP_OK(c, launch_swiglu_fwd(work, out, B, out_size, c->stream));
  return GN_OK;
}

extern "C" int gn_swiglu_backward(gn_ctx *c, const float *x, const float *params, const float *gout,
                                  float *grads, float *gin, float *work, int32_t B, int32_t in,
                                  int32_t out_size, float scale) {
  ENTRY(c);
  if (!x || !params || !gout || !grads || !work || B <= 0 || in <= 0 || out_size <= 0)
    return set_err(c, GN_ERR_INVALID, "bad swiglu args");
  float *Z = work, *dZ = work + 2 * (int64_t)B * out_size;
  {
    KTimer kt(c, GN_KCLASS_OTHER, "swiglu_bwd", f4(5.0 * B * out_size));
    HIP_OK(c, launch_swiglu_bwd(gout, Z, 2 * out_size, dZ, B, out_size, c->stream));
  }
  // [dW | dV] = scale dZ^T x, gin = dZ [W; V]
  HIP_OK(c, dense_bwd_core(c, x, params, dZ, grads, nullptr, gin, B, in, 2 * out_size, scale, nullptr, 0));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// BatchNorm2D (batchnorm2d.go:255-666): x is B x C x HW; params = [gamma |
// beta] or null (affine = false).  Training (Q22): each sample normalised by
// its own per-channel statistics (one sample per Forward in the reference's
// per-sample loop), the running mean / var advanced once per sample in sample
// order (biased variance, momentum as given); stats keeps (mean, var, std)
// per (sample, channel) for the backward.  Inference: the running
// statistics.  The backward writes [dgamma | dbeta] = scale * sums (zero in
// inference mode, where only dx flows, batchnorm2d.go:525-551); work: 2 B C
// floats.
// ---------------------------------------------------------------------------
extern "C" int gn_batchnorm2d_forward(gn_ctx *c, const float *x, const float *params, float *out,
                                      float *stats, float *running_mean, float *running_var, int32_t B,
                                      int32_t C, int32_t HW, float eps, float momentum, int32_t training) {
  ENTRY(c);
  if (!x || !out || !stats || !running_mean || !running_var || B <= 0 || C <= 0 || HW <= 0 || !(eps >= 0) ||
      !(momentum >= 0 && momentum <= 1))
    return set_err(c, GN_ERR_INVALID, "bad batchnorm2d args");
  KTimer kt(c, GN_KCLASS_OTHER, "bn_fwd", f4(2.0 * B * C * HW + 3.0 * B * C));
  HIP_OK(c, launch_bn_fwd(x, params, out, stats, running_mean, running_var, B, C, HW, eps > 0 ? eps : 1e-5f,
                          momentum, training ? 1 : 0, c->stream));
  return GN_OK;
}

extern "C" int gn_batchnorm2d_backward(gn_ctx *c, const float *gout, const float *x, const float *params,
                                       const float *stats, const float *running_var, float *grads, float *gin,
                                       float *work, int32_t B, int32_t C, int32_t HW, float eps,
                                       int32_t training, float scale) {
  ENTRY(c);
  if (!gout || !x || !stats || !running_var || !work || B <= 0 || C <= 0 || HW <= 0 || (params && !grads))
    return set_err(c, GN_ERR_INVALID, "bad batchnorm2d args");
  KTimer kt(c, GN_KCLASS_OTHER, "bn_bwd", f4(3.0 * B * C * HW + 2.0 * B * C));
  if (!training) {
    if (params) HIP_OK(c, launch_fill(grads, 0.0f, 2 * (int64_t)C, c->stream));
    if (gin)
      HIP_OK(c, launch_bn_bwd_eval(gout, params, running_var, gin, B, C, HW, eps > 0 ? eps : 1e-5f,
                                   c->stream));
    return GN_OK;
  }
  HIP_OK(c, launch_bn_bwd(gout, x, params, stats, gin, params ? work : nullptr, B, C, HW, c->stream));
  if (params) {
    HIP_OK(c, launch_colsum(work, B, C, C, scale, grads, c->scratch, c->scratch_floats, c->stream));
    HIP_OK(c, launch_colsum(work + (int64_t)B * C, B, C, C, scale, grads + C, c->scratch, c->scratch_floats,
                            c->stream));
  }
  return GN_OK;
}

// ---------------------------------------------------------------------------
// SequenceUnroller(GRU) (unroller.go:57-213, gru.go:192-703) over a batch: x
// is B x T x I, params = [Wx (3H x I) | Wh (2H x H) | b (3H)], gates u, r, c.
// The reference's quirks are kept: h' = h + u (c - h) forward but a backward
// that weights the candidate by (1 - u) and the direct path by u (Q23), no
// reset-gate delta (Q24), dWx from the last step's input, gradients carried
// as dh_{t-1} = dh_t + dh_prev.  return_sequences: out / gout hold every
// step's h.  work: gn_gru_workspace floats, shared by the forward and
// backward of one batch.
// ---------------------------------------------------------------------------
namespace {
struct GruWork {
  float *WhT, *xw, *pre, *hprev, *rh, *Dg, *S;
  size_t floats;
};
GruWork gru_carve(float *w, int B, int T, int H) {
  Carve cv(w);
  GruWork m{};
  const size_t rows = (size_t)B * T;
  m.WhT = cv.take(2 * (size_t)H * H);
  m.xw = cv.take(rows * 3 * H);
  m.pre = cv.take(rows * 3 * H);
  m.hprev = cv.take(rows * H);
  m.rh = cv.take(rows * H);
  m.Dg = cv.take(rows * 3 * H);
  m.S = cv.take((size_t)B * 3 * H);
  m.floats = cv.off;
  return m;
}
}  // namespace

extern "C" int gn_gru_workspace(int32_t B, int32_t T, int32_t I, int32_t H, int64_t *floats) {
  if (!floats || B <= 0 || T <= 0 || I <= 0 || H <= 0) return GN_ERR_INVALID;
  *floats = (int64_t)gru_carve(nullptr, B, T, H).floats;
  return GN_OK;
}

extern "C" int gn_gru_seq_forward(gn_ctx *c, const float *x, const float *params, float *out, float *work,
                                  int32_t B, int32_t T, int32_t I, int32_t H, int32_t return_sequences) {
  ENTRY(c);
  if (!x || !params || !out || !work || B <= 0 || T <= 0 || I <= 0 || !gru_supported(H))
    return set_err(c, GN_ERR_INVALID, "bad GRU args (hidden <= 1024)");
  GruWork m = gru_carve(work, B, T, H);
  const int G3 = 3 * H;
  const float *Wx = params, *Wh = Wx + (int64_t)G3 * I, *bias = Wh + (int64_t)2 * H * H;
  {
    GemmArgs g{};  // xw[b*T + t] = b + Wx x_t (gru.go:194-210)
    g.M = B * T; g.N = G3; g.K = I;
    g.A = x; g.lda = I; g.B = Wx; g.ldb = I;
    g.C = m.xw; g.ldc = G3; g.alpha = 1.0f;
    g.bias = bias; g.act = F_IDENTITY;
    g.ws = c->scratch; g.ws_cap = c->scratch_floats;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(g));
    HIP_OK(c, launch_gemm('N', 'T', EPI_BIAS_ACT, g, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "transpose", f4(4.0 * H * H));
    HIP_OK(c, launch_transpose(Wh, m.WhT, 2 * H, H, c->stream));
  }
  KTimer kt(c, GN_KCLASS_OTHER, "gru_fwd", 2.0 * 3 * H * H * B * T);
  HIP_OK(c, launch_gru_fwd(m.xw, m.WhT, m.pre, m.hprev, m.rh, out, B, T, H, c->stream,
                           return_sequences ? 1 : 0));
  return GN_OK;
}

extern "C" int gn_gru_seq_backward(gn_ctx *c, const float *x, const float *params, const float *gout,
                                   float *grads, float *gin, float *work, int32_t B, int32_t T, int32_t I,
                                   int32_t H, float scale, int32_t return_sequences) {
  ENTRY(c);
  if (!x || !params || !gout || !grads || !work || B <= 0 || T <= 0 || I <= 0 || !gru_supported(H))
    return set_err(c, GN_ERR_INVALID, "bad GRU args (hidden <= 1024)");
  GruWork m = gru_carve(work, B, T, H);
  const int G3 = 3 * H;
  const float *Wx = params, *Wh = Wx + (int64_t)G3 * I;
  float *gWx = grads, *gWh = gWx + (int64_t)G3 * I, *gb = gWh + (int64_t)2 * H * H;
  {
    KTimer kt(c, GN_KCLASS_OTHER, "gru_bwd", 2.0 * 2 * H * H * B * T);
    HIP_OK(c, launch_gru_bwd(gout, m.pre, m.hprev, Wh, m.Dg, B, T, H, c->stream, return_sequences ? 1 : 0));
  }
  if (gin) {  // dx_t = Wx^T [dU | dR (never set, 0) | dC] (gru.go:481-500)
    GemmArgs a{};
    a.M = B * T; a.N = I; a.K = G3;
    a.A = m.Dg; a.lda = G3; a.B = Wx; a.ldb = I;
    a.C = gin; a.ldc = I; a.alpha = 1.f;
    a.ws = c->scratch; a.ws_cap = c->scratch_floats;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
    HIP_OK(c, launch_gemm('N', 'N', EPI_SCALE, a, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "token_sum", token_sum_bytes(B, T, G3));
    HIP_OK(c, launch_token_sum(m.Dg, m.S, B, T, G3, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "colsum", f4((double)B * G3 + G3));
    HIP_OK(c, launch_colsum(m.S, B, G3, G3, scale, gb, c->scratch, c->scratch_floats, c->stream));
  }
  GemmArgs a{};  // dWx = scale * (sum_t dG)^T x_last
  a.M = G3; a.N = I; a.K = B;
  a.A = m.S; a.lda = G3;
  a.B = x + (int64_t)(T - 1) * I; a.ldb = T * I;
  a.C = gWx; a.ldc = I; a.alpha = scale;
  a.ws = c->scratch; a.ws_cap = c->scratch_floats;
  GemmArgs u{};  // dWh_u = scale * dU^T h_prev over (sample, step)
  u.M = H; u.N = H; u.K = B * T;
  u.A = m.Dg; u.lda = G3;
  u.B = m.hprev; u.ldb = H;
  u.C = gWh; u.ldc = H; u.alpha = scale;
  u.ws = c->scratch; u.ws_cap = c->scratch_floats;
  GemmArgs r{};  // dWh_r = scale * dC^T (r * h_prev): the candidate's use of the reset block
  r.M = H; r.N = H; r.K = B * T;
  r.A = m.Dg + 2 * H; r.lda = G3;
  r.B = m.rh; r.ldb = H;
  r.C = gWh + (int64_t)H * H; r.ldc = H; r.alpha = scale;
  r.ws = c->scratch; r.ws_cap = c->scratch_floats;
  KTimer kt(c, GN_KCLASS_GEMM, "gemm_dw", gemm_flops(a) + gemm_flops(u) + gemm_flops(r));
  HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, a, c->stream));
  HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, u, c->stream));
  HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, r, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// MoE (moe.go:140-313): params = [gating W (E x I), b (E) | per expert W (O x
// I), b (O)]; a Linear gating Dense, E Dense(LeakyReLU 0.1) experts, the top
// K by gate softmax combined with their probabilities (ties keep index
// order).  training adds the layer's RNG gate noise: *noise is that stream's
// state (NewRNG(42) at construction), advanced by E draws per sample, and
// the load-balancing gradient in the backward.  All experts run on every
// sample; the route picks K of them.  work: gn_moe_workspace floats, shared
// by the forward and backward of one batch.
// ---------------------------------------------------------------------------
namespace {
struct MoeWork {
  float *logits, *prob, *dzg, *eout, *edz;
  int32_t *act;
  size_t floats;
};
MoeWork moe_carve(float *w, int B, int I, int O, int E, int K) {
  Carve cv(w);
  MoeWork m{};
  m.logits = cv.take((size_t)B * E);
  m.prob = cv.take((size_t)B * E);
  m.dzg = cv.take((size_t)B * E);
  m.eout = cv.take((size_t)E * B * O);
  m.edz = cv.take((size_t)E * B * O);
  m.act = reinterpret_cast<int32_t *>(cv.take((size_t)B * K));
  m.floats = cv.off;
  (void)I;
  return m;
}
int moe_check(gn_ctx *c, int B, int I, int O, int E, int K) {
  if (B <= 0 || I <= 0 || O <= 0 || E <= 0 || E > MOE_MAX_E || K <= 0 || K > E)
    return set_err(c, GN_ERR_INVALID, "bad MoE sizes (experts <= %d, 0 < k <= experts)", MOE_MAX_E);
  return GN_OK;
}
}  // namespace

extern "C" int gn_moe_workspace(int32_t B, int32_t I, int32_t O, int32_t E, int32_t K, int64_t *floats) {
  if (!floats || B <= 0 || I <= 0 || O <= 0 || E <= 0 || K <= 0) return GN_ERR_INVALID;
  *floats = (int64_t)moe_carve(nullptr, B, I, O, E, K).floats;
  return GN_OK;
}

extern "C" int gn_moe_forward(gn_ctx *c, const float *x, const float *params, float *out, float *work,
                              int32_t B, int32_t I, int32_t O, int32_t E, int32_t K, int32_t training,
                              uint64_t *noise) {
  ENTRY(c);
  int rc = moe_check(c, B, I, O, E, K);
  if (rc) return rc;
  if (!x || !params || !out || !work || (training && !noise)) return set_err(c, GN_ERR_INVALID, "null pointer");
  MoeWork m = moe_carve(work, B, I, O, E, K);
  const int64_t e1 = (int64_t)O * I + O;
  {
    GemmArgs g{};  // gate logits = Wg x + bg
    g.M = B; g.N = E; g.K = I;
    g.A = x; g.lda = I; g.B = params; g.ldb = I;
    g.C = m.logits; g.ldc = E; g.alpha = 1.f; g.bias = params + (int64_t)E * I; g.act = F_IDENTITY;
    g.ws = c->scratch; g.ws_cap = c->scratch_floats;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(g));
    HIP_OK(c, launch_gemm('N', 'T', EPI_BIAS_ACT, g, c->stream));
  }
  MoeRoute rt{};
  rt.B = B; rt.E = E; rt.K = K; rt.training = training ? 1 : 0;
  rt.chunk = 0;
  rt.base[0] = training ? *noise : 42;
  {
    KTimer kt(c, GN_KCLASS_OTHER, "moe_route", f4(2.0 * B * E + (double)B * K));
    HIP_OK(c, launch_moe_route(m.logits, m.prob, m.act, rt, c->stream));
  }
  for (int e = 0; e < E; ++e) {
    const float *We = params + (int64_t)E * I + E + e * e1;
    GemmArgs g{};
    g.M = B; g.N = O; g.K = I;
    g.A = x; g.lda = I; g.B = We; g.ldb = I;
    g.C = m.eout + (int64_t)e * B * O; g.ldc = O; g.alpha = 1.f; g.bias = We + (int64_t)O * I;
    g.act = F_LEAKY;
    g.ws = c->scratch; g.ws_cap = c->scratch_floats;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(g));
    HIP_OK(c, launch_gemm('N', 'T', EPI_BIAS_ACT, g, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "moe_combine", f4((double)K * B * O + (double)B * O));
    HIP_OK(c, launch_moe_combine(m.eout, m.prob, m.act, out, B, O, E, K, c->stream));
  }
  if (training)  // E draws per sample on the layer's stream
    for (int64_t d = 0; d < (int64_t)B * E; ++d) *noise = *noise * 6364136223846793005ull + 1;
  return GN_OK;
}

extern "C" int gn_moe_backward(gn_ctx *c, const float *x, const float *params, const float *gout,
                               float *grads, float *gin, float *work, int32_t B, int32_t I, int32_t O,
                               int32_t E, int32_t K, int32_t training, float scale) {
  ENTRY(c);
  int rc = moe_check(c, B, I, O, E, K);
  if (rc) return rc;
  if (!x || !params || !gout || !grads || !work) return set_err(c, GN_ERR_INVALID, "null pointer");
  MoeWork m = moe_carve(work, B, I, O, E, K);
  const int64_t e1 = (int64_t)O * I + O;
  {
    KTimer kt(c, GN_KCLASS_OTHER, "moe_deltas", f4(2.0 * K * B * O + 3.0 * B * E));
    HIP_OK(c, launch_moe_backward_deltas(gout, m.eout, m.prob, m.act, m.edz, m.dzg, B, O, E, K,
                                         training ? 1 : 0, c->stream));
  }
  // gating and expert Dense backward: W grads = scale dz^T x, b grads = scale colsum(dz)
  HIP_OK(c, dense_bwd_core(c, x, params, m.dzg, grads, grads + (int64_t)E * I, nullptr, B, I, E, scale,
                           nullptr, 0));
  for (int e = 0; e < E; ++e) {
    float *gW = grads + (int64_t)E * I + E + e * e1;
    HIP_OK(c, dense_bwd_core(c, x, nullptr, m.edz + (int64_t)e * B * O, gW, gW + (int64_t)O * I, nullptr, B,
                             I, O, scale, nullptr, 0));
  }
  if (gin) {  // dx = dz_gate Wg + sum_e dz_e W_e
    GemmArgs a{};
    a.M = B; a.N = I; a.K = E;
    a.A = m.dzg; a.lda = E; a.B = params; a.ldb = I;
    a.C = gin; a.ldc = I; a.alpha = 1.f;
    a.ws = c->scratch; a.ws_cap = c->scratch_floats;
    {
      KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
      HIP_OK(c, launch_gemm('N', 'N', EPI_SCALE, a, c->stream));
    }
    for (int e = 0; e < E; ++e) {
      GemmArgs d{};
      d.M = B; d.N = I; d.K = O;
      d.A = m.edz + (int64_t)e * B * O; d.lda = O; d.B = params + (int64_t)E * I + E + e * e1; d.ldb = I;
      d.C = gin; d.ldc = I; d.alpha = 1.f;
      d.aux = gin; d.ldaux = I;
      d.ws = c->scratch; d.ws_cap = c->scratch_floats;
      KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(d));
      HIP_OK(c, launch_gemm('N', 'N', EPI_BIAS_ADD, d, c->stream));
    }
  }
  return GN_OK;
}
