// Library-private: the context, the per-launch timer, error reporting and the
// activation plans shared by the runtime (gn_runtime.hip) and the per-layer
// operator entry points (gn_ops.hip).  Not part of the C ABI.
#pragma once
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "gn_common.h"

// the definitions that follow sat in gn_runtime.hip's global scope, where the
// C ABI's gn_ctx lives (typedef struct gn_ctx gn_ctx, goneuron_hip.h)
using namespace gn;

struct gn_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipStream_t aux = nullptr;   // dW and bias sums next to the dX GEMMs (large models), LSTM clip
  std::string err;
  int fail_next = 0;
  hipDeviceProp_t props{};
  float *scratch = nullptr;  // colsum partials
  size_t scratch_floats = 0;
  float *scratch_aux = nullptr;  // the same for kernels queued on `aux` (scratch_floats long)
  float *noalloc = nullptr;      // this device's copy of `scratch` (gn_dense_backward_noalloc)
  // kernel timing (gn_timing_enable)
  bool timing = false;
  struct Rec {
    int cls;
    const char *name;  // kernel (or fused launch group) name, static storage
    double units;      // algorithmic bytes (memory-bound) or FLOPs (GEMM / MFMA) of the launch
    hipEvent_t a, b;
  };
  std::vector<Rec> recs;
  std::vector<hipEvent_t> pool;
  size_t pool_used = 0;
};

inline hipEvent_t ev_get(gn_ctx *c) {
  if (c->pool_used == c->pool.size()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    c->pool.push_back(e);
  }
  return c->pool[c->pool_used++];
}

// Brackets the kernels launched in its scope with events when timing is on
// (on the stream those kernels go to), under a name with the launch's
// algorithmic work: the bytes a memory-bound kernel must move (compulsory
// reads and writes, fp32) or the FLOPs of a matrix-core kernel.
struct KTimer {
  gn_ctx *c;
  int cls;
  const char *name;
  double units;
  hipStream_t st;
  hipEvent_t a = nullptr, b = nullptr;
  KTimer(gn_ctx *c_, int cls_, const char *name_, double units_, hipStream_t st_ = nullptr)
      : c(c_), cls(cls_), name(name_), units(units_), st(st_ ? st_ : c_->stream) {
    if (c->timing) {
      a = ev_get(c);
      b = ev_get(c);
      if (a && b) (void)hipEventRecord(a, st);
      else a = b = nullptr;
    }
  }
  ~KTimer() {
    if (a) {
      (void)hipEventRecord(b, st);
      c->recs.push_back({cls, name, units, a, b});
    }
  }
};

inline double gemm_flops(const GemmArgs &g) {
  return 2.0 * g.M * g.N * g.K * (g.nbatch > 1 ? g.nbatch : 1);
}
inline double f4(double n) { return 4.0 * n; }  // bytes of n floats
// attention FLOPs per launch: the score and value products over the (query,
// key) pairs the mask keeps, 2 products forward, 4 backward (dP, dQ, dK, dV)
inline double attn_flops(int B, int T, int NH, int hd, int causal, bool bwd) {
  const double pairs = causal ? 0.5 * T * (T + 1.0) : (double)T * T;
  return (bwd ? 8.0 : 4.0) * hd * pairs * B * NH;
}
// per-sample token sums: read B x T x N, write B x N
inline double token_sum_bytes(int B, int T, int N) { return f4((double)B * T * N + (double)B * N); }
// direct convolution work: 2 FLOPs per tap of every output
inline double conv_flops(const ConvShape &cs, int B) {
  return 2.0 * B * cs.outC * cs.oH * cs.oW * cs.inC * cs.k * cs.k;
}

inline int set_err(gn_ctx *c, int code, const char *fmt, ...) {
  if (c) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    c->err = buf;
  }
  return code;
}

#define HIP_OK(ctx, expr)                                                                  \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess)                                                                  \
      return set_err((ctx), GN_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                     __FILE__, __LINE__);                                                  \
  } while (0)

inline int check_fail(gn_ctx *c) {
  if (c && c->fail_next) {
    int code = c->fail_next;
    c->fail_next = 0;
    return set_err(c, code, "injected failure (gn_debug_fail_next)");
  }
  return GN_OK;
}

#define ENTRY(ctx)                              \
  do {                                          \
    if (!(ctx)) return GN_ERR_INVALID;          \
    int f_ = check_fail(ctx);                   \
    if (f_) return f_;                          \
    (void)hipSetDevice((ctx)->device);          \
  } while (0)

struct ActPlan {
  int row_act;  // RowAct (with fwd kind in bits 8.. for ROW_ELEMWISE)
  int fwd;      // FwdKind for elementwise forward
  int deriv;    // DerivKind
  bool jac;     // Softmax/LogSoftmax Jacobian backward
};

// cacheActivationType (layer.go:183-205) + the Activate/Derivative methods of
// activations.go: pointer Softmax/LogSoftmax get the row activation and the
// Jacobian; the values fall through to identity forward / NaN derivative.
inline int plan_act(int act, int is_ptr, ActPlan &p) {
  p = ActPlan{ROW_NONE, F_IDENTITY, D_ONE, false};
  switch (act) {
    case GN_ACT_RELU: p.fwd = F_RELU; p.deriv = D_RELU; break;
    case GN_ACT_SIGMOID: p.fwd = F_SIGMOID; p.deriv = D_SIGMOID; break;
    case GN_ACT_TANH: p.fwd = F_TANH; p.deriv = D_TANH; break;
    case GN_ACT_LINEAR: break;
    case GN_ACT_GELU:
      // only *activations.GELU is ActTypeGELU (layer.go:196-197); the value
      // runs as ActTypeNone: identity forward, Derivative(preAct) backward,
      // and the identity output is the pre-activation D_GELU needs
      if (is_ptr) return GN_ERR_UNSUPPORTED;
      p.deriv = D_GELU;
      break;
    case GN_ACT_SOFTMAX:
    case GN_ACT_LOGSOFTMAX:
      if (is_ptr) {
        p.row_act = act == GN_ACT_SOFTMAX ? ROW_SOFTMAX : ROW_LOGSOFTMAX;
        p.jac = true;
      } else {
        p.deriv = D_NAN;
      }
      break;
    default: return GN_ERR_INVALID;  // nil activation: the reference panics in Derivative
  }
  if (p.row_act == ROW_NONE && p.fwd != F_IDENTITY) p.row_act = ROW_ELEMWISE | (p.fwd << 8);
  return GN_OK;
}

// Conv2D calls the activation's scalar Activate / Derivative methods directly
// (conv2d.go:950, :1140): Softmax/LogSoftmax give NaN there.
inline int plan_scalar_act(int act, int &fwd, int &deriv) {
  switch (act) {
    case GN_ACT_RELU: fwd = F_RELU; deriv = D_RELU; return GN_OK;
    case GN_ACT_SIGMOID: fwd = F_SIGMOID; deriv = D_SIGMOID; return GN_OK;
    case GN_ACT_TANH: fwd = F_TANH; deriv = D_TANH; return GN_OK;
    case GN_ACT_LINEAR: fwd = F_IDENTITY; deriv = D_ONE; return GN_OK;
    case GN_ACT_SOFTMAX:
    case GN_ACT_LOGSOFTMAX: fwd = F_NAN; deriv = D_NAN; return GN_OK;
    default: return GN_ERR_INVALID;
  }
}



// MultiHeadAttention buffers of one batch (gn_ops.hip): Q, K, V (and GQ, GK,
// GV) equally spaced, token sums S [B][D] and S3 (three blocks s3_stride
// apart), RoPE tables [T][hd/2], materialised scores when the fused kernels
// do not hold the shape.
struct MhaBufs {
  float *Q, *K, *V, *O, *GO, *GQ, *GK, *GV, *S, *S3, *rcos, *rsin, *SC;
  int64_t s3_stride;
};
void rope_tables(int T, int hd, std::vector<float> &cs, std::vector<float> &sn);
int mha_forward_impl(gn_ctx *c, const float *x, const float *params, float *out, const MhaBufs &m,
                     int B, int T, int D, int NH, int causal, int rope);
int mha_backward_impl(gn_ctx *c, const float *x, const float *params, const float *gout, float *grads,
                      float *gin, const MhaBufs &m, int B, int T, int D, int NH, int causal, int rope,
                      float scale);

// gradW = scale * dz^T x ; gradB = scale * colsum(dz) (gB may be null) ;
// gin = dz W (optionally * act'(gin_aux)), gin may be null (gn_runtime.hip)
hipError_t dense_bwd_core(gn_ctx *c, const float *x, const float *W, const float *dz, float *gW,
                          float *gB, float *gin, int B, int in, int out_n, float scale,
                          const float *gin_aux, int gin_deriv, hipEvent_t dz_ready = nullptr,
                          float *ms = nullptr, size_t ms_cap = 0, const float *gin_colscale = nullptr,
                          bool skip_dw = false, bool bias_main = false);
