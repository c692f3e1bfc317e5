// Host runtime of libgoneuron_hip.so: context, device-resident flat arena,
// the Sequential model plan and the batched training step.
//
// The step keeps the reference's per-sample semantics (Network.
// trainBatchSequential, internal/net/net.go:721-784: per-sample forward,
// backward accumulated into the flat grads, grads *= 1/B, Adam) but runs each
// layer once over the whole batch: per-sample mat-vecs become fp32 MFMA GEMMs,
// the gradient sums over samples become the K dimension of those GEMMs, and
// the 1/B average is folded into the dW/db writes.  Parameters, gradients and
// Adam moments live in one HBM allocation; nothing crosses PCIe inside a step.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "gn_common.h"
#include "gn_ctx.h"

using namespace gn;

// Scratch of gn_dense_backward_noalloc, one copy per GPU for the process's
// lifetime: dz (B x out, at most kNoAllocDz floats) followed by the partial
// sums of the bias column sums and of split-K GEMMs.  In host code the name
// only stands for the symbol: the device address comes from
// hipGetSymbolAddress at gn_init (noalloc_ptr), per device.
constexpr size_t kNoAllocFloats = (size_t)8 << 20;  // 32 MiB
constexpr size_t kNoAllocDz = (size_t)4 << 20;      // dz part: 16 MiB
static __device__ __align__(256) float scratch[kNoAllocFloats];

constexpr int kMaxDevices = 64;
static float *noalloc_ptr[kMaxDevices];
static std::mutex noalloc_mu;


// ---------------------------------------------------------------------------
// LCG of the reference (layer.go:61-81) and synthetic data
// ---------------------------------------------------------------------------
static inline float lcg_float(uint64_t &s) {
  s = s * 6364136223846793005ULL + 1ULL;
  return (float)(s >> 33) / (float)(1u << 31);
}

extern "C" int gn_fill_uniform(float *dst, int64_t n, uint64_t seed) {
  if (!dst && n) return GN_ERR_INVALID;
  uint64_t s = seed;
  for (int64_t i = 0; i < n; ++i) dst[i] = lcg_float(s);
  return GN_OK;
}

extern "C" int gn_fill_normal(float *dst, int64_t n, uint64_t seed) {
  if (!dst && n) return GN_ERR_INVALID;
  uint64_t s = seed;
  for (int64_t i = 0; i < n; ++i) {
    double u1 = (double)lcg_float(s);
    double u2 = (double)lcg_float(s);
    if (u1 < 1e-7) u1 = 1e-7;
    dst[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
  }
  return GN_OK;
}

extern "C" int gn_fill_class_ids(int32_t *dst, int64_t n, int32_t nclass, uint64_t seed) {
  if ((!dst && n) || nclass <= 0) return GN_ERR_INVALID;
  uint64_t s = seed;
  for (int64_t i = 0; i < n; ++i) {
    int32_t c = (int32_t)(lcg_float(s) * (float)nclass);
    dst[i] = c >= nclass ? nclass - 1 : c;
  }
  return GN_OK;
}

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------
extern "C" int gn_available(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n > 0 ? 1 : 0;
}

extern "C" int gn_init(int device_ordinal, gn_ctx **out) {
  if (!out) return GN_ERR_INVALID;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return GN_ERR_NO_DEVICE;
  if (device_ordinal < 0 || device_ordinal >= n) return GN_ERR_INVALID;
  std::unique_ptr<gn_ctx> c(new gn_ctx);
  c->device = device_ordinal;
  if (hipSetDevice(device_ordinal) != hipSuccess) return GN_ERR_HIP;
  if (hipGetDeviceProperties(&c->props, device_ordinal) != hipSuccess) return GN_ERR_HIP;
  if (device_ordinal >= kMaxDevices) return GN_ERR_INVALID;
  {
    // once per device, with that device current: the address of its copy of
    // the no-alloc scratch array
    std::lock_guard<std::mutex> lk(noalloc_mu);
    if (!noalloc_ptr[device_ordinal]) {
      float *p = nullptr;
      if (hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return GN_ERR_HIP;
      noalloc_ptr[device_ordinal] = p;
    }
    c->noalloc = noalloc_ptr[device_ordinal];
  }
  // both streams at the default priority
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) return GN_ERR_HIP;
  if (hipStreamCreateWithFlags(&c->aux, hipStreamNonBlocking) != hipSuccess) {
    (void)hipStreamDestroy(c->stream);
    return GN_ERR_HIP;
  }
  c->scratch_floats = (size_t)16 << 20;  // 64 MiB: colsum partials, split-K partials
  if (hipMalloc(&c->scratch, c->scratch_floats * sizeof(float)) != hipSuccess) {
    (void)hipStreamDestroy(c->stream);
    (void)hipStreamDestroy(c->aux);
    return GN_ERR_OOM;
  }
  if (hipMalloc(&c->scratch_aux, c->scratch_floats * sizeof(float)) != hipSuccess) {
    (void)hipFree(c->scratch);
    (void)hipStreamDestroy(c->stream);
    (void)hipStreamDestroy(c->aux);
    return GN_ERR_OOM;
  }
  *out = c.release();
  return GN_OK;
}

extern "C" void gn_shutdown(gn_ctx *c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  (void)hipStreamSynchronize(c->aux);
  for (hipEvent_t e : c->pool) (void)hipEventDestroy(e);
  (void)hipFree(c->scratch);
  (void)hipFree(c->scratch_aux);
  (void)hipStreamDestroy(c->stream);
  (void)hipStreamDestroy(c->aux);
  delete c;
}

extern "C" const char *gn_last_error(const gn_ctx *c) { return c ? c->err.c_str() : "null context"; }

extern "C" int gn_device_info(gn_ctx *c, gn_info *info) {
  ENTRY(c);
  if (!info) return set_err(c, GN_ERR_INVALID, "info is null");
  memset(info, 0, sizeof *info);
  snprintf(info->arch, sizeof info->arch, "%s", c->props.gcnArchName);
  info->cu_count = c->props.multiProcessorCount;
  info->hbm_bytes = (int64_t)c->props.totalGlobalMem;
  info->peak_fp32_mfma_tflops = 157.3;  // MI355X dense fp32 matrix
  info->peak_hbm_gbps = 8000.0;         // MI355X HBM3E
  return GN_OK;
}

extern "C" int gn_sync(gn_ctx *c) {
  ENTRY(c);
  HIP_OK(c, hipStreamSynchronize(c->stream));
  HIP_OK(c, hipStreamSynchronize(c->aux));
  return GN_OK;
}

extern "C" int gn_debug_fail_next(gn_ctx *c, int code) {
  if (!c) return GN_ERR_INVALID;
  c->fail_next = code < 0 ? code : GN_ERR_INJECTED;
  return GN_OK;
}

extern "C" int gn_timing_enable(gn_ctx *c, int enable) {
  ENTRY(c);
  HIP_OK(c, hipStreamSynchronize(c->stream));
  HIP_OK(c, hipStreamSynchronize(c->aux));
  c->timing = enable != 0;
  c->recs.clear();
  c->pool_used = 0;
  return GN_OK;
}

extern "C" int gn_timing_report(gn_ctx *c, int cls, int64_t *launches, double *total_ms) {
  ENTRY(c);
  HIP_OK(c, hipStreamSynchronize(c->stream));
  HIP_OK(c, hipStreamSynchronize(c->aux));
  int64_t n = 0;
  double ms = 0;
  for (const auto &r : c->recs) {
    if (r.cls != cls) continue;
    float t = 0;
    HIP_OK(c, hipEventElapsedTime(&t, r.a, r.b));
    ms += t;
    ++n;
  }
  if (launches) *launches = n;
  if (total_ms) *total_ms = ms;
  return GN_OK;
}

// Per-name totals of the timed launches since the last gn_timing_enable, in
// first-seen order: up to cap entries into out, the count into *n.
extern "C" int gn_timing_kernels(gn_ctx *c, gn_kernel_stat *out, int32_t cap, int32_t *n) {
  ENTRY(c);
  if (!n || (cap > 0 && !out)) return set_err(c, GN_ERR_INVALID, "bad timing_kernels args");
  HIP_OK(c, hipStreamSynchronize(c->stream));
  HIP_OK(c, hipStreamSynchronize(c->aux));
  std::vector<gn_kernel_stat> acc;
  for (const auto &r : c->recs) {
    float t = 0;
    HIP_OK(c, hipEventElapsedTime(&t, r.a, r.b));
    size_t k = 0;
    while (k < acc.size() && (acc[k].cls != r.cls || strcmp(acc[k].name, r.name) != 0)) ++k;
    if (k == acc.size()) {
      gn_kernel_stat z{};
      snprintf(z.name, sizeof z.name, "%s", r.name ? r.name : "?");
      z.cls = r.cls;
      acc.push_back(z);
    }
    acc[k].launches += 1;
    acc[k].ms += t;
    acc[k].units += r.units;
  }
  *n = (int32_t)acc.size();
  for (int32_t i = 0; i < cap && i < (int32_t)acc.size(); ++i) out[i] = acc[i];
  return GN_OK;
}

__global__ void floor_kernel() {}

extern "C" int gn_timing_floor(gn_ctx *c, int32_t blocks, int32_t reps) {
  ENTRY(c);
  if (blocks < 1 || reps < 0) return set_err(c, GN_ERR_INVALID, "bad timing_floor args");
  for (int32_t r = 0; r < reps; ++r) {
    KTimer kt(c, GN_KCLASS_OTHER, "floor", 0.0);
    hipLaunchKernelGGL(floor_kernel, dim3((unsigned)blocks), dim3(256), 0, c->stream);
    HIP_OK(c, hipGetLastError());
  }
  return GN_OK;
}

extern "C" int gn_malloc(gn_ctx *c, size_t bytes, void **dptr) {
  ENTRY(c);
  if (!dptr) return set_err(c, GN_ERR_INVALID, "dptr is null");
  *dptr = nullptr;
  if (hipMalloc(dptr, bytes ? bytes : 4) != hipSuccess)
    return set_err(c, GN_ERR_OOM, "hipMalloc(%zu) failed", bytes);
  return GN_OK;
}

extern "C" int gn_free(gn_ctx *c, void *p) {
  ENTRY(c);
  HIP_OK(c, hipStreamSynchronize(c->stream));
  HIP_OK(c, hipFree(p));
  return GN_OK;
}

extern "C" int gn_memcpy_h2d(gn_ctx *c, void *dst, const void *src, size_t bytes) {
  ENTRY(c);
  if ((!dst || !src) && bytes) return set_err(c, GN_ERR_INVALID, "null pointer");
  HIP_OK(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return GN_OK;
}

extern "C" int gn_memcpy_d2h(gn_ctx *c, void *dst, const void *src, size_t bytes) {
  ENTRY(c);
  if ((!dst || !src) && bytes) return set_err(c, GN_ERR_INVALID, "null pointer");
  HIP_OK(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return GN_OK;
}

extern "C" int gn_memset_zero(gn_ctx *c, void *dst, size_t bytes) {
  ENTRY(c);
  HIP_OK(c, hipMemsetAsync(dst, 0, bytes, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// Per-layer operators
// ---------------------------------------------------------------------------
// drop: a Dropout above the layer in training mode, whose output the GEMM
// writes too (its split-K reduction, or a dropout launch right after it)
// defer: when non-null and K splits, only the partial sums are written (to
// the context's scratch) and *defer receives the split count (else 1)
static hipError_t dense_fwd(gn_ctx *c, const float *x, const float *W, const float *b, float *out,
                            int B, int in, int out_n, int fwd, float *drop_out = nullptr,
                            const float *drop_mask = nullptr, float drop_scale = 0.f, int *defer = nullptr) {
  GemmArgs a{};
  a.M = B; a.N = out_n; a.K = in;
  a.A = x; a.lda = in;
  a.B = W; a.ldb = in;
  a.C = out; a.ldc = out_n;
  a.bias = b; a.act = fwd; a.alpha = 1.f;
  a.ws = c->scratch; a.ws_cap = c->scratch_floats;
  a.drop_out = drop_out;
  a.drop_mask = drop_mask;
  a.drop_scale = drop_scale;
  a.defer_splits = defer;
  KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(a));
  return launch_gemm('N', 'T', EPI_BIAS_ACT, a, c->stream);
}

// gradW = scale * dz^T x ; gradB = scale * colsum(dz) ; gin = dz W (optionally * act'(aux))
// With dz_ready, the parameter gradients go to ctx->aux (after dz_ready is
// recorded on the main stream, with aux's own scratch) and run next to the dX
// GEMM: the two GEMMs share the CUs, and each one's prologue and tail are
// covered by the other's tiles.
// ms / ms_cap: scratch of the kernels on the main stream (default: the
// context's).
hipError_t dense_bwd_core(gn_ctx *c, const float *x, const float *W, const float *dz, float *gW,
                          float *gB, float *gin, int B, int in, int out_n, float scale,
                          const float *gin_aux, int gin_deriv, hipEvent_t dz_ready, float *ms,
                          size_t ms_cap, const float *gin_colscale, bool skip_dw, bool bias_main) {
  hipError_t e;
  if (!ms) {
    ms = c->scratch;
    ms_cap = c->scratch_floats;
  }
  hipStream_t ws = c->stream;
  float *wscr = ms;
  size_t wcap = ms_cap;
  if (dz_ready) {
    if ((e = hipEventRecord(dz_ready, c->stream)) != hipSuccess) return e;
    if ((e = hipStreamWaitEvent(c->aux, dz_ready, 0)) != hipSuccess) return e;
    ws = c->aux;
    wscr = c->scratch_aux;
    wcap = c->scratch_floats;
  }
  // bias_main: the bias sums may ride on the dX GEMM's split-K reduction
  // launch (below) on the main stream; without it (steps with per-layer
  // updates, which wait for them on the second stream) they run here
  const bool cs_in_dx = gB && gin && bias_main;
  if (gB && !cs_in_dx) {
    KTimer kt(c, GN_KCLASS_OTHER, "colsum", f4((double)B * out_n + out_n), ws);
    e = launch_colsum(dz, B, out_n, out_n, scale, gB, wscr, wcap, ws);
    if (e != hipSuccess) return e;
  }
  GemmArgs a{};
  a.M = out_n; a.N = in; a.K = B;
  a.A = dz; a.lda = out_n;
  a.B = x; a.ldb = in;
  a.C = gW; a.ldc = in;
  a.alpha = scale;
  a.ws = wscr; a.ws_cap = wcap;
  if (!skip_dw) {
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_dw", gemm_flops(a), ws);
    e = launch_gemm('T', 'N', EPI_SCALE, a, ws);
    if (e != hipSuccess) return e;
  }
  if (gin) {
    GemmArgs d{};
    d.M = B; d.N = in; d.K = out_n;
    d.A = dz; d.lda = out_n;
    d.B = W; d.ldb = in;
    d.C = gin; d.ldc = in;
    d.alpha = 1.f;
    d.ws = ms; d.ws_cap = ms_cap;
    int cs_done = 0;
    if (cs_in_dx) {
      d.cs_src = dz; d.cs_dst = gB; d.cs_rows = B; d.cs_cols = out_n; d.cs_scale = scale;
      d.cs_done = &cs_done;
    }
    {
      KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(d));
      if (gin_aux) {
        d.aux = gin_aux; d.ldaux = in; d.act = gin_deriv; d.colscale = gin_colscale;
        e = launch_gemm('N', 'N', EPI_DACT, d, c->stream);
      } else {
        e = launch_gemm('N', 'N', EPI_SCALE, d, c->stream);
      }
    }
    if (e != hipSuccess) return e;
    if (cs_in_dx && !cs_done) {
      KTimer kt(c, GN_KCLASS_OTHER, "colsum", f4((double)B * out_n + out_n));
      e = launch_colsum(dz, B, out_n, out_n, scale, gB, ms, ms_cap, c->stream);
    }
  }
  return e;
}

extern "C" int gn_gemm(gn_ctx *c, int32_t transA, int32_t transB, int32_t M, int32_t N, int32_t K,
                       float alpha, const float *A, int32_t lda, const float *B, int32_t ldb,
                       float *Cm, int32_t ldc) {
  ENTRY(c);
  if (M < 0 || N < 0 || K < 0 || !A || !B || !Cm) return set_err(c, GN_ERR_INVALID, "bad gemm args");
  if (lda < (transA ? M : K) || ldb < (transB ? K : N) || ldc < N)
    return set_err(c, GN_ERR_INVALID, "leading dimension too small");
  GemmArgs a{};
  a.M = M; a.N = N; a.K = K;
  a.A = A; a.lda = lda; a.B = B; a.ldb = ldb; a.C = Cm; a.ldc = ldc; a.alpha = alpha;
  a.ws = c->scratch; a.ws_cap = c->scratch_floats;
  HIP_OK(c, launch_gemm(transA ? 'T' : 'N', transB ? 'T' : 'N', EPI_SCALE, a, c->stream));
  return GN_OK;
}

extern "C" int gn_dense_forward(gn_ctx *c, const float *x, const float *W, const float *bias,
                                float *out, int32_t B, int32_t in, int32_t out_n, int32_t act,
                                int32_t act_is_ptr) {
  ENTRY(c);
  if (!x || !W || !out || B < 0 || in <= 0 || out_n <= 0)
    return set_err(c, GN_ERR_INVALID, "bad dense_forward args");
  ActPlan ap;
  if (plan_act(act, act_is_ptr, ap)) return set_err(c, GN_ERR_INVALID, "unknown activation %d", act);
  HIP_OK(c, dense_fwd(c, x, W, bias, out, B, in, out_n, ap.jac ? F_IDENTITY : ap.fwd));
  if (ap.jac) HIP_OK(c, launch_row_act(out, B, out_n, ap.row_act, c->stream));
  return GN_OK;
}

__global__ void jac_rows_kernel(const float *__restrict__ o, const float *__restrict__ g,
                                float *__restrict__ dz, int C, int logsm) {
  __shared__ float sh[4];
  const int b = blockIdx.x, t = threadIdx.x;
  const float *orow = o + (size_t)b * C, *grow = g + (size_t)b * C;
  float *d = dz + (size_t)b * C;
  float s = 0.f;
  for (int i = t; i < C; i += 256) s += logsm ? grow[i] : grow[i] * orow[i];
  // block reduce
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((t & 63) == 0) sh[t >> 6] = s;
  __syncthreads();
  s = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  for (int i = t; i < C; i += 256)
    d[i] = logsm ? grow[i] - (float)exp((double)orow[i]) * s : grow[i] * orow[i] - orow[i] * s;
}

static int dense_backward_op(gn_ctx *c, const float *x, const float *W, const float *out,
                             const float *gout, float *gradW, float *gradB, float *gin, float *dz,
                             int32_t B, int32_t in, int32_t out_n, int32_t act, int32_t act_is_ptr,
                             float scale, float *ms, size_t ms_cap) {
  ActPlan ap;
  if (plan_act(act, act_is_ptr, ap)) return set_err(c, GN_ERR_INVALID, "unknown activation %d", act);
  if (ap.jac) {
    hipLaunchKernelGGL(jac_rows_kernel, dim3(B), dim3(256), 0, c->stream, out, gout, dz, out_n,
                       ap.row_act == ROW_LOGSOFTMAX ? 1 : 0);
    HIP_OK(c, hipGetLastError());
  } else {
    HIP_OK(c, launch_dact(gout, out, dz, (int64_t)B * out_n, ap.deriv, c->stream));
  }
  HIP_OK(c, dense_bwd_core(c, x, W, dz, gradW, gradB, gin, B, in, out_n, scale, nullptr, 0, nullptr,
                           ms, ms_cap));
  return GN_OK;
}

extern "C" int gn_dense_backward(gn_ctx *c, const float *x, const float *W, const float *out,
                                 const float *gout, float *gradW, float *gradB, float *gin,
                                 float *dz, int32_t B, int32_t in, int32_t out_n, int32_t act,
                                 int32_t act_is_ptr, float scale) {
  ENTRY(c);
  if (!x || !W || !out || !gout || !gradW || !dz || B <= 0 || in <= 0 || out_n <= 0)
    return set_err(c, GN_ERR_INVALID, "bad dense_backward args");
  return dense_backward_op(c, x, W, out, gout, gradW, gradB, gin, dz, B, in, out_n, act, act_is_ptr,
                           scale, nullptr, 0);
}

// gn_dense_backward without the dz workspace and without the context's
// scratch: dz and every partial sum live in this device's copy of `scratch`
// (noalloc_ptr), so the call allocates nothing.  Calls that overlap on one
// GPU (other streams, other contexts, other threads) share that array and
// race; the array keeps the last call's contents, and nothing in it needs to
// start at zero (every value is written before it is read).
extern "C" int gn_dense_backward_noalloc(gn_ctx *c, const float *x, const float *W, const float *out,
                                         const float *gout, float *gradW, float *gradB, float *gin,
                                         int32_t B, int32_t in, int32_t out_n, int32_t act,
                                         int32_t act_is_ptr, float scale) {
  ENTRY(c);
  if (!x || !W || !out || !gout || !gradW || B <= 0 || in <= 0 || out_n <= 0)
    return set_err(c, GN_ERR_INVALID, "bad dense_backward_noalloc args");
  if ((size_t)B * (size_t)out_n > kNoAllocDz)
    return set_err(c, GN_ERR_INVALID,
                   "dense_backward_noalloc: B x out = %lld floats exceeds the static scratch limit of "
                   "%zu floats (use gn_dense_backward with a workspace)",
                   (long long)B * out_n, kNoAllocDz);
  if (!c->noalloc) return set_err(c, GN_ERR_HIP, "no-alloc scratch address unavailable");
  return dense_backward_op(c, x, W, out, gout, gradW, gradB, gin, c->noalloc, B, in, out_n, act,
                           act_is_ptr, scale, c->noalloc + kNoAllocDz, kNoAllocFloats - kNoAllocDz);
}

extern "C" int gn_adam_step(gn_ctx *c, float *p, const float *g, float *m, float *v, int64_t n,
                            float lr, float b1, float b2, float eps, int32_t timestep) {
  ENTRY(c);
  if ((!p || !g || !m || !v) && n) return set_err(c, GN_ERR_INVALID, "null arena pointer");
  if ((((uintptr_t)p | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) & 15) != 0)
    return set_err(c, GN_ERR_INVALID, "arena pointers must be 16-byte aligned");
  if (b1 == 0) b1 = 0.9f;
  if (b2 == 0) b2 = 0.999f;
  if (eps == 0) eps = 1e-8f;
  // opt.go:237-242: bias corrections in float64 then rounded
  const double ts = (double)(timestep + 1);
  const float bias1 = (float)(1.0 - pow((double)b1, ts));
  const float bias2 = (float)(1.0 - pow((double)b2, ts));
  const float efflr = lr * (float)sqrt((double)bias2) / bias1;
  HIP_OK(c, launch_adam(p, g, m, v, n, efflr, b1, b2, 1.0f - b1, 1.0f - b2, eps, c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// Model
// ---------------------------------------------------------------------------
struct LayerRT {
  gn_layer_desc d{};
  int64_t poff = 0, pcount = 0;
  int in_len = 0, out_len = 0;  // per-sample feature counts
  float *out = nullptr;         // [maxB, out_len] activation output (owned unless alias)
  bool out_alias = false;       // Flatten: out is the input buffer
  float *gout = nullptr;        // dL/d(out) [maxB, out_len] (owned unless alias)
  bool gout_alias = false;
  ActPlan ap{};
  float *mask = nullptr;        // Dropout per-feature mask (Q9)
  float *dfac = nullptr;        // Dropout per-feature backward factor: mask > 0 ? scale : 0
  float scale = 1.f;
  ConvShape cs{};               // Conv2D
  PoolShape ps{};               // MaxPool2D
  int32_t *argmax = nullptr;    // MaxPool2D switches [maxB, out_len]
  int cfwd = 0, cderiv = 0;     // Conv2D scalar Activate / Derivative kinds
  // SequenceUnroller(LSTM): T steps of I inputs, H hidden
  int T = 0, I = 0, H = 0;
  float *WhT = nullptr;                          // transposed input-gate block of Wh
  float *xw = nullptr;                           // x_t . Wx_i for every (sample, step)
  float *igb = nullptr, *tcb = nullptr, *cbuf = nullptr, *hbuf = nullptr;
  float *Dg = nullptr, *S = nullptr, *wts = nullptr;
  double *gram = nullptr, *coef = nullptr;
  void *lsync = nullptr;                         // cooperative BPTT exchange words
  unsigned lepoch = 0;                           // its tag base
  // Gram / clip side by side: per-column tile counts, per-chain start flags,
  // launch number since the counts were zeroed and the batch they were laid
  // out for; events for the clip's stream
  unsigned *gcnt = nullptr, *gstart = nullptr, *gbail = nullptr;
  unsigned gepoch = 0;
  int gB = 0;
  hipEvent_t lev[2] = {nullptr, nullptr};
  bool lcoop = false;                            // cooperative BPTT usable
  // Embedding / PositionalEncoding / TransformerBlock / CLSPooling
  int V = 0, D = 0, NH = 0, FF = 0, causal = 0;
  int32_t *ids = nullptr;
  int32_t *bad = nullptr;  // Embedding: per-sample index-error flags [max batch]
  int *err = nullptr;      // LSTM: cooperative wait timeout flag
  int train = 1;           // training flag (SetTraining): Dropout, BatchNorm2D and MoE read it
  // RMSNorm over rows of D: per-row rms and g * x / rms for the gamma sums
  float *rmsv = nullptr, *gx = nullptr;
  float eps = 0.f;
  // SwiGLU: projections Z = [gate | up] and their gradients, [maxB, 2*out] each
  float *zbuf = nullptr, *dzbuf = nullptr;
  // BatchNorm2D: C channels of HW; per-plane (mean, var, std), gamma / beta
  // partial sums [2][maxB*C], running mean / var [C]
  int C = 0, HW = 0;
  float *bnst = nullptr, *bnpart = nullptr, *rmean = nullptr, *rvar = nullptr;
  // SequenceUnroller(GRU): pre-activations [B*T][3H], h before each step and
  // r * h_prev [B*T][H] (xw, WhT, Dg, S as for the LSTM, sized for 3 gates)
  float *gpre = nullptr, *ghprev = nullptr, *grh = nullptr;
  // MoE: E experts, top K; gate logits / probabilities / deltas [B][E], routes
  // [B][K], expert outputs and deltas [E][B][O]; noise stream states (the
  // network's own, then one per worker clone), advanced on the host
  int E = 0, K = 0;
  float *mlog = nullptr, *mprob = nullptr, *mdzg = nullptr, *meout = nullptr, *medz = nullptr;
  int32_t *mact = nullptr;
  std::vector<uint64_t> mrng;
  struct Tb {
    float *Q, *K, *V, *O, *RES1, *N1, *MID, *RES2, *st1, *st2;
    float *G1, *DZ1, *COMB, *G2, *GO, *GQ, *GK, *GV, *GX, *S;
    float *S3;  // token sums of gQ, gK, gV ([3][max batch][D])
    // LayerNorm backward block partials of norm 1 / norm 2: [blocks][2D]
    // (dgamma | dbeta) and [blocks][D] (column sums of dx, the token sums of
    // wOut's / ff2's dz); null when the norms are RMSNorm or the rows of a
    // block can span two samples
    float *LP1, *LP2, *TS1, *TS2;
    float *Z, *MG, *DZS;     // SwiGLU ff1: [gate | up] per token, token-0 mid grad, its dZ
    float *rcos, *rsin;      // RoPE angle tables [T][hd/2]
    float *SC;               // attention scores and their gradients (sizes the fused kernels do not hold)
  } tb{};
};

struct gn_model {
  gn_ctx *ctx = nullptr;
  int lstm_spin_limit = 1 << 18;  // polls per cooperative BPTT wait (see gn_debug_lstm_spin_limit)
  int lstm_clip_bail = 2048;      // polls of the clip's wait for a Gram kernel beside it
  std::vector<LayerRT> L;
  int loss_kind = 0;
  gn_adam_desc adam{};
  int maxB = 0, workers = 1;
  int64_t nparams = 0, region = 0;
  float *arena = nullptr, *params = nullptr, *grads = nullptr, *m = nullptr, *v = nullptr;
  int timestep = 0;
  float *loss_rows = nullptr;
  int loss_B = 0;  // rows of loss_rows the last training pass wrote
  float *xin = nullptr, *yin = nullptr;  // staging for host inputs
  int last_B = 0;
  bool last_predict = false;  // the last pass was an inference forward
  int skipped = 0;            // samples the last training step skipped (Embedding index errors)
  std::vector<void *> owned;   // state allocations (arena, tables, running statistics)
  std::vector<void *> bowned;  // batch-sized buffers (rebuilt by gn_model_reserve)
  // training flags of the trainBatchParallel worker clones: LightweightClone
  // copies each layer's flag when the clone is made (dropout.go:410-418,
  // batchnorm2d.go:786-808, moe.go:424) and Network.SetTraining never reaches
  // the clones (net.go:187-193), so they keep it for the network's lifetime
  std::vector<std::vector<char>> clone_train;
  std::vector<char> eff;  // flags in effect for the current pass, per layer
  // train steps update each layer's parameters on ctx->aux as soon as that
  // layer's backward is done, overlapping Adam with the rest of the backward
  bool overlap_adam = true;
  // the output Dense layer of training passes as the two fused kernels of
  // launch_tail_fwd / launch_tail_bwd when it qualifies (gn_debug_fused_tail);
  // tail_now: the current pass uses them
  bool tail_on = true;
  bool tail_now = false;
  int tail_src = -1;     // the Dense whose output (or Dropout above it) the output layer reads
  TailSplitIn tail_sp;   // its deferred split-K partials in the current pass (ws null: none)
  std::vector<hipEvent_t> sync_ev;  // one per layer + 1 (no timing)
  std::vector<hipEvent_t> dz_ev;    // one per layer: its dz is ready (no timing)
  std::vector<hipEvent_t> dw_ev;    // one per layer: its dW and bias sums on ctx->aux are done
  // the per-layer Adam updates run on a stream of the model's own, created by
  // its first overlapped train step and destroyed with the model, so a
  // context that later trains other models keeps two streams in use
  hipStream_t adam_s = nullptr;
  // the backward's parameter-gradient kernels (Dense dW and bias sums, the
  // transformer block's token sums and Q10 weight gradients) on ctx->aux
  // beside the input-gradient chain: always in steps with per-layer Adam
  // updates, elsewhere only when gn_debug_side_streams asks (as branches of a
  // captured C4 step they cost more than they overlap: 459 vs 392 us per
  // step); fork_ev / join_ev branch aux off the main stream and back
  bool side_ok = false;
  hipEvent_t fork_ev = nullptr, join_ev = nullptr;
  // per-layer updates launched by the current overlapped step: a step that
  // fails after one of them keeps its timestep (those layers hold step t)
  int step_updates = 0;
  // HIP graphs of the accumulate pass (forward, loss, backward) of small
  // models, keyed by the input pointers, the batch and the training flags in
  // effect: the first step with a key runs eagerly, the second is captured,
  // later ones replay.  Adam (or the launch carrying it, upd_fn) runs after
  // the graph as an ordinary launch (its coefficients change every step; an
  // update inside the graph with its coefficients from a device table
  // measured no faster: 36.7 vs 36.4 us per C1 step).
  struct StepGraph {
    const float *x, *y;
    int B;
    std::vector<char> eff;
    hipGraphExec_t exec;
    bool upd;  // captured for a train step (upd_want)
    std::function<hipError_t(const AdamStep &)> upd_fn;  // the launch it left out, or none
    const char *upd_name;
    double upd_units;
  };
  std::vector<StepGraph> graphs;
  bool graph_on = true;   // gn_model_set_graphs
  int emb = -1;           // the Embedding layer (its index-error flags mask samples), or -1
  bool graph_ok = true;   // false once a capture failed: eager from then on
  // Train steps of small models: when the backward's last launch can carry
  // Network.Step's update (the weight-gradient reduction of a first Conv2D,
  // or the gradient launch of a first Embedding: each gradient it writes is
  // updated by the thread that writes it, extra blocks update every other
  // layer), the pass leaves it out and the step launches it with the
  // update's coefficients after the pass or its graph: no Adam launch of its
  // own (C2 63.7 -> 60.3 us per step, same box).
  // upd_want asks the current pass for it; upd_fn, upd_name, upd_units
  // describe the launch left out (null: none, the step launches Adam).
  // gn_debug_step_update.
  bool upd_on = true;
  bool upd_want = false;
  std::function<hipError_t(const AdamStep &)> upd_fn;
  const char *upd_name = nullptr;
  double upd_units = 0;
  // a forward pass ran on the network's own layers (Predict, or training with
  // one worker; trainBatchParallel runs clones only, net.go:588-716): from
  // then on its Conv2D / pooling layers know their input height and width
  // (conv2d.go:746, maxpool2d.go:119-127), which ExtractLayerConfig reads
  bool master_dims = false;
};

static void drop_graphs(gn_model *M) {
  for (auto &g : M->graphs)
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
  M->graphs.clear();
}

// Adam coefficients of one Network.Step: Adam.NewStep increments the
// timestep before the update, whose bias corrections use timestep + 1
// (opt.go:237-258), in float64 then rounded.
struct AdamCoef {
  float efflr, b1, b2, omb1, omb2, eps;
};

// Adam.NewStep (opt.go:254-258) for the step that takes the timestep to t
static AdamCoef adam_coef(const gn_model *M, int t) {
  AdamCoef a;
  a.b1 = M->adam.beta1;
  a.b2 = M->adam.beta2;
  a.eps = M->adam.eps;
  const double ts = (double)(t + 1);
  const float bias1 = (float)(1.0 - pow((double)a.b1, ts));
  const float bias2 = (float)(1.0 - pow((double)a.b2, ts));
  a.efflr = M->adam.lr * (float)sqrt((double)bias2) / bias1;
  a.omb1 = 1.0f - a.b1;
  a.omb2 = 1.0f - a.b2;
  return a;
}

static AdamCoef adam_next(gn_model *M) {
  M->timestep++;
  return adam_coef(M, M->timestep);
}


static int model_alloc(gn_model *M, size_t floats, float **p) {
  void *q = nullptr;
  if (hipMalloc(&q, std::max<size_t>(floats, 1) * sizeof(float)) != hipSuccess) {
    *p = nullptr;
    return set_err(M->ctx, GN_ERR_OOM, "hipMalloc(%zu floats) failed", floats);
  }
  M->owned.push_back(q);
  *p = (float *)q;
  return GN_OK;
}

extern "C" void gn_model_destroy(gn_model *M) {
  if (!M) return;
  (void)hipSetDevice(M->ctx->device);
  (void)hipStreamSynchronize(M->ctx->stream);
  (void)hipStreamSynchronize(M->ctx->aux);
  drop_graphs(M);
  for (LayerRT &R : M->L)
    for (hipEvent_t e : R.lev)
      if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : M->sync_ev) (void)hipEventDestroy(e);
  for (hipEvent_t e : M->dw_ev) (void)hipEventDestroy(e);
  if (M->adam_s) {
    (void)hipStreamSynchronize(M->adam_s);
    (void)hipStreamDestroy(M->adam_s);
  }
  for (hipEvent_t e : M->dz_ev) (void)hipEventDestroy(e);
  if (M->fork_ev) (void)hipEventDestroy(M->fork_ev);
  if (M->join_ev) (void)hipEventDestroy(M->join_ev);
  for (void *p : M->bowned) (void)hipFree(p);
  for (void *p : M->owned) (void)hipFree(p);
  delete M;
}

// Reference initialisation into the host copy of the arena.
static void init_dense(float *p, int in, int out) {  // Dense.Build layer.go:300-320
  const float scale = (float)sqrt(2.0 / ((double)in + (double)out));
  uint64_t s = (uint64_t)(in * 1000 + out * 100 + 42);
  const int64_t nw = (int64_t)in * out;
  for (int64_t i = 0; i < nw; ++i) p[i] = lcg_float(s) * 2 * scale - scale;
  for (int i = 0; i < out; ++i) p[nw + i] = lcg_float(s) * 0.2f - 0.1f;
}

static void init_gru(float *p, int I, int H) {  // GRU.Build gru.go:120-147 (biases stay 0)
  const float scale = (float)sqrt(2.0 / ((double)I + (double)H));
  uint64_t s = (uint64_t)(I * 1000 + H * 100 + 242);
  const int64_t n = (int64_t)3 * H * I + (int64_t)2 * H * H;
  for (int64_t k = 0; k < n; ++k) p[k] = lcg_float(s) * 2 * scale - scale;
}

static void init_swiglu(float *p, int in, int out) {  // SwiGLU.Build swiglu.go:82-88
  const float scale = (float)sqrt(2.0 / ((double)in + (double)out));
  uint64_t s = (uint64_t)(in * 100 + out + 42);
  const int64_t n = 2 * (int64_t)in * out;
  for (int64_t i = 0; i < n; ++i) p[i] = lcg_float(s) * 2 * scale - scale;
}

static void init_conv(float *p, int inC, int outC, int k) {  // Conv2D.Build conv2d.go:114-135
  const float scale = (float)sqrt(2.0 / (double)(inC * k * k));
  uint64_t s = 42;
  const int64_t nw = (int64_t)outC * inC * k * k;
  for (int64_t i = 0; i < nw; ++i) p[i] = lcg_float(s) * 2 * scale - scale;
  for (int i = 0; i < outC; ++i) p[nw + i] = lcg_float(s) * 0.2f - 0.1f;
}

static void init_lstm(float *p, int in, int H) {  // LSTM.Build lstm.go:175-196
  const float sin_ = (float)sqrt(2.0 / (double)(in + 4 * H));
  const float srec = (float)sqrt(2.0 / (double)(H + 4 * H));
  float *wx = p, *wh = wx + (int64_t)4 * H * in, *b = wh + (int64_t)4 * H * H;
  uint64_t s = (uint64_t)(in * 1000 + H * 100 + 142);
  for (int i = 0; i < 4 * H; ++i) {
    b[i] = (i >= H && i < 2 * H) ? 1.0f : 0.0f;
    for (int j = 0; j < in; ++j) wx[(int64_t)i * in + j] = lcg_float(s) * 2 * sin_ - sin_;
    for (int j = 0; j < H; ++j) wh[(int64_t)i * H + j] = lcg_float(s) * 2 * srec - srec;
  }
}

static void init_embedding(float *p, int V, int D) {  // NewEmbedding embedding.go:51-57
  const float scale = (float)sqrt(3.0 / (double)D);
  uint64_t s = 42;
  for (int64_t i = 0; i < (int64_t)V * D; ++i) p[i] = scale * (2 * lcg_float(s) - 1);
}

static void init_posenc(float *p, int T, int D) {  // PositionalEncoding.Build transformer.go:50-66
  uint64_t s = (uint64_t)(T + D + 42);
  const float scale = (float)sqrt(1.0 / (double)D);
  for (int64_t i = 0; i < (int64_t)T * D; ++i) p[i] = lcg_float(s) * 2 * scale - scale;
}

// TransformerBlock flat layout (transformer.go:1035-1056): wQ, wK, wV, wOut
// (W [D][D] then b [D]), norm1, norm2 (LayerNorm: gamma, beta; RMSNorm:
// gamma), ff1 (Dense: W [FF][D], b; SwiGLU: W [FF][D] then V [FF][D], here
// at b1), ff2 (W [D][FF], b).  Build rebinds every sub-layer to fresh zero
// slices, so the reference starts the block at all-zero parameters.
struct TbOff {
  int64_t wq, bq, wk, bk, wv, bv, wo, bo, g1, be1, g2, be2, w1, b1, w2, b2, total;
};
static TbOff tb_offsets(int D, int FF, int act = GN_BLOCK_ACT_RELU, int norm = GN_BLOCK_NORM_LN) {
  TbOff o{};
  int64_t off = 0;
  const int64_t dd = (int64_t)D * D;
  const int64_t nn = norm == GN_BLOCK_NORM_RMS ? D : 2 * (int64_t)D;
  o.wq = off; o.bq = off + dd; off += dd + D;
  o.wk = off; o.bk = off + dd; off += dd + D;
  o.wv = off; o.bv = off + dd; off += dd + D;
  o.wo = off; o.bo = off + dd; off += dd + D;
  o.g1 = off; o.be1 = off + D; off += nn;
  o.g2 = off; o.be2 = off + D; off += nn;
  o.w1 = off; o.b1 = off + (int64_t)FF * D;
  off += act == GN_BLOCK_ACT_SWIGLU ? 2 * (int64_t)FF * D : (int64_t)FF * D + FF;
  o.w2 = off; o.b2 = off + (int64_t)D * FF; off += (int64_t)D * FF + D;
  o.total = off;
  return o;
}

// Square-first dimension inference of Conv2D / MaxPool2D forward
// (conv2d.go:733-746, maxpool2d.go:117-126).
static void infer_hw(int channel_size, int &H, int &W) {
  H = (int)sqrt((double)channel_size);
  W = (H * H == channel_size) ? H : (H > 0 ? channel_size / H : 0);
}

static int model_balloc(gn_model *M, size_t floats, float **p) {
  void *q = nullptr;
  if (hipMalloc(&q, std::max<size_t>(floats, 1) * sizeof(float)) != hipSuccess) {
    *p = nullptr;
    return set_err(M->ctx, GN_ERR_OOM, "hipMalloc(%zu floats) failed", floats);
  }
  M->bowned.push_back(q);
  *p = (float *)q;
  return GN_OK;
}

static void free_batch(gn_model *M) {
  for (void *p : M->bowned) (void)hipFree(p);
  M->bowned.clear();
  M->last_B = 0;
}

// Every buffer whose size follows the batch: layer outputs and output
// gradients, the state layers save for their backward, staging for host
// inputs.  Sized for M->maxB samples.
static int alloc_batch(gn_model *M) {
  gn_ctx *c = M->ctx;
  const int nlayers = (int)M->L.size();
  const int max_batch = M->maxB;
  int rc;
  for (int i = 0; i < nlayers; ++i) {
    LayerRT &R = M->L[i];
    if (R.d.kind == GN_LAYER_EMBEDDING) {
      float *tmp = nullptr;
      if ((rc = model_balloc(M, (size_t)max_batch * R.T, &tmp))) return rc;
      R.ids = reinterpret_cast<int32_t *>(tmp);
      if ((rc = model_balloc(M, (size_t)max_batch + 64, &tmp))) return rc;
      R.bad = reinterpret_cast<int32_t *>(tmp);
      HIP_OK(c, hipMemsetAsync(R.bad, 0, (size_t)max_batch * sizeof(int32_t), c->stream));
    }
    if (R.d.kind == GN_LAYER_TRANSFORMER) {
      // activations and gradients of the block
      const size_t rows = (size_t)max_batch * R.T, D = R.D, FF = R.FF;
      LayerRT::Tb &t = R.tb;
      // Q, K, V in one block (their projections run as one batched GEMM)
      if ((rc = model_balloc(M, 3 * rows * D, &t.Q))) return rc;
      t.K = t.Q + rows * D;
      t.V = t.K + rows * D;
      // gQ, gK, gV in one block too (their token sums run as one launch)
      if ((rc = model_balloc(M, 3 * rows * D, &t.GQ))) return rc;
      t.GK = t.GQ + rows * D;
      t.GV = t.GK + rows * D;
      float **dbufs[] = {&t.O, &t.RES1, &t.N1, &t.RES2, &t.G1, &t.COMB, &t.G2, &t.GO, &t.GX};
      for (float **b : dbufs)
        if ((rc = model_balloc(M, rows * D, b))) return rc;
      if ((rc = model_balloc(M, rows * FF, &t.MID))) return rc;
      if ((rc = model_balloc(M, rows * FF, &t.DZ1))) return rc;
      if ((rc = model_balloc(M, rows * 2, &t.st1))) return rc;
      if ((rc = model_balloc(M, rows * 2, &t.st2))) return rc;
      if ((rc = model_balloc(M, (size_t)max_batch * std::max(D, FF), &t.S))) return rc;
      if ((rc = model_balloc(M, 3 * (size_t)max_batch * D, &t.S3))) return rc;
      if (R.d.block_norm != GN_BLOCK_NORM_RMS && ln_bwd_part_supported(R.D) &&
          R.T % ln_bwd_rows_per_block() == 0) {
        const size_t nb = (size_t)ln_bwd_blocks((int)rows);
        if ((rc = model_balloc(M, nb * 2 * D, &t.LP1))) return rc;
        if ((rc = model_balloc(M, nb * 2 * D, &t.LP2))) return rc;
        if ((rc = model_balloc(M, nb * D, &t.TS1))) return rc;
        if ((rc = model_balloc(M, nb * D, &t.TS2))) return rc;
      }
      if (!attn_supported(R.T, R.D, R.NH) &&
          (rc = model_balloc(M, attn_gemm_floats(max_batch, R.T, R.NH), &t.SC)))
        return rc;
      if (R.d.block_act == GN_BLOCK_ACT_SWIGLU) {
        if ((rc = model_balloc(M, rows * 2 * FF, &t.Z))) return rc;
        if ((rc = model_balloc(M, (size_t)max_batch * FF, &t.MG))) return rc;
        if ((rc = model_balloc(M, (size_t)max_batch * 2 * FF, &t.DZS))) return rc;
      }
    }
    if (R.d.kind == GN_LAYER_LSTM_UNROLLER) {
      const size_t Bm = max_batch, T = R.T, H = R.H;
      if ((rc = model_balloc(M, Bm * T * H, &R.xw))) return rc;
      if ((rc = model_balloc(M, Bm * T * H, &R.igb))) return rc;
      if ((rc = model_balloc(M, Bm * T * H, &R.tcb))) return rc;
      if ((rc = model_balloc(M, Bm * T * H, &R.cbuf))) return rc;
      if ((rc = model_balloc(M, Bm * (T + 1) * H, &R.hbuf))) return rc;
      if ((rc = model_balloc(M, Bm * (T + 1) * 4 * H, &R.Dg))) return rc;
      if ((rc = model_balloc(M, Bm * 4 * H, &R.S))) return rc;
      if ((rc = model_balloc(M, Bm * (T + 1), &R.wts))) return rc;
      const int Wc = std::min(std::max(M->workers, 1), max_batch);
      const size_t chunk = (max_batch + Wc - 1) / Wc;
      const size_t nmax = (size_t)lstm_gram_pitch((int)(chunk * T));
      const size_t nchains = (max_batch + chunk - 1) / chunk;
      float *g = nullptr, *cf = nullptr;
      if ((rc = model_balloc(M, 2 * nchains * nmax * nmax, &g))) return rc;
      if ((rc = model_balloc(M, 2 * nchains * nmax, &cf))) return rc;
      R.gram = reinterpret_cast<double *>(g);
      R.coef = reinterpret_cast<double *>(cf);
      R.lsync = nullptr;
      R.err = nullptr;
      {
        // tile counts, then per chain a start flag and a bail flag
        const size_t ncnt = (size_t)lstm_gram_counters(max_batch, (int)T, M->workers) + 2 * nchains;
        float *cb = nullptr, *er = nullptr;
        if ((rc = model_balloc(M, ncnt, &cb))) return rc;
        if ((rc = model_balloc(M, 64, &er))) return rc;
        HIP_OK(c, hipMemsetAsync(cb, 0, ncnt * sizeof(unsigned), c->stream));
        HIP_OK(c, hipMemsetAsync(er, 0, sizeof(int), c->stream));
        R.gcnt = reinterpret_cast<unsigned *>(cb);
        R.gstart = R.gcnt + lstm_gram_counters(max_batch, (int)T, M->workers);
        R.gbail = R.gstart + nchains;
        R.err = reinterpret_cast<int *>(er);
        R.gepoch = 0;
        R.gB = 0;
        for (hipEvent_t &e : R.lev)
          if (!e) HIP_OK(c, hipEventCreateWithFlags(&e, hipEventDisableTiming));
      }
      R.lcoop = false;
      R.lepoch = 0;
      if (lstm_coop_eligible(max_batch, (int)H)) {
        const size_t bytes = lstm_coop_sync_bytes(max_batch, (int)H);
        float *sy = nullptr;
        if ((rc = model_balloc(M, (bytes + 3) / 4, &sy))) return rc;
        HIP_OK(c, hipMemsetAsync(sy, 0, bytes, c->stream));
        R.lsync = sy;
        R.lcoop = true;
      }
    }
    if (R.d.kind == GN_LAYER_MOE) {
      const size_t Bm = max_batch, E = R.E, O = R.d.out_size;
      float *tmp = nullptr;
      if ((rc = model_balloc(M, Bm * E, &R.mlog))) return rc;
      if ((rc = model_balloc(M, Bm * E, &R.mprob))) return rc;
      if ((rc = model_balloc(M, Bm * E, &R.mdzg))) return rc;
      if ((rc = model_balloc(M, E * Bm * O, &R.meout))) return rc;
      if ((rc = model_balloc(M, E * Bm * O, &R.medz))) return rc;
      if ((rc = model_balloc(M, Bm * R.K, &tmp))) return rc;
      R.mact = reinterpret_cast<int32_t *>(tmp);
    }
    if (R.d.kind == GN_LAYER_GRU_UNROLLER) {
      const size_t rows = (size_t)max_batch * R.T, H = R.H;
      if ((rc = model_balloc(M, rows * 3 * H, &R.xw))) return rc;
      if ((rc = model_balloc(M, rows * 3 * H, &R.gpre))) return rc;
      if ((rc = model_balloc(M, rows * H, &R.ghprev))) return rc;
      if ((rc = model_balloc(M, rows * H, &R.grh))) return rc;
      if ((rc = model_balloc(M, rows * 3 * H, &R.Dg))) return rc;
      if ((rc = model_balloc(M, (size_t)max_batch * 3 * H, &R.S))) return rc;
    }
    if (R.d.kind == GN_LAYER_BATCHNORM2D) {
      if ((rc = model_balloc(M, (size_t)max_batch * R.C * 3, &R.bnst))) return rc;
      if ((rc = model_balloc(M, (size_t)max_batch * R.C * 2, &R.bnpart))) return rc;
    }
    if (R.d.kind == GN_LAYER_SWIGLU) {
      if ((rc = model_balloc(M, (size_t)max_batch * 2 * R.out_len, &R.zbuf))) return rc;
      if ((rc = model_balloc(M, (size_t)max_batch * 2 * R.out_len, &R.dzbuf))) return rc;
    }
    if (R.d.kind == GN_LAYER_RMSNORM) {
      if ((rc = model_balloc(M, (size_t)max_batch * (R.in_len / R.D), &R.rmsv))) return rc;
      if ((rc = model_balloc(M, (size_t)max_batch * R.in_len, &R.gx))) return rc;
    }
    if (R.d.kind == GN_LAYER_LAYERNORM) {
      // per-row (mean, std); g * xhat for the gamma sums when the one-pass
      // backward does not fit the scratch; an input-gradient sink when the
      // layer is first (the backward kernels always write dx)
      if ((rc = model_balloc(M, (size_t)max_batch * (R.in_len / R.D) * 2, &R.rmsv))) return rc;
      if ((rc = model_balloc(M, (size_t)max_batch * R.in_len, &R.gx))) return rc;
      if (i == 0 && (rc = model_balloc(M, (size_t)max_batch * R.in_len, &R.zbuf))) return rc;
    }
    if (R.d.kind == GN_LAYER_MHA) {
      const size_t rows = (size_t)max_batch * R.T, D = R.D;
      LayerRT::Tb &t = R.tb;
      if ((rc = model_balloc(M, 3 * rows * D, &t.Q))) return rc;
      t.K = t.Q + rows * D;
      t.V = t.K + rows * D;
      if ((rc = model_balloc(M, 3 * rows * D, &t.GQ))) return rc;
      t.GK = t.GQ + rows * D;
      t.GV = t.GK + rows * D;
      if ((rc = model_balloc(M, rows * D, &t.O))) return rc;
      if ((rc = model_balloc(M, rows * D, &t.GO))) return rc;
      if ((rc = model_balloc(M, (size_t)max_batch * D, &t.S))) return rc;
      if ((rc = model_balloc(M, 3 * (size_t)max_batch * D, &t.S3))) return rc;
      if (R.d.block_norm != GN_BLOCK_NORM_RMS && ln_bwd_part_supported(R.D) &&
          R.T % ln_bwd_rows_per_block() == 0) {
        const size_t nb = (size_t)ln_bwd_blocks((int)rows);
        if ((rc = model_balloc(M, nb * 2 * D, &t.LP1))) return rc;
        if ((rc = model_balloc(M, nb * 2 * D, &t.LP2))) return rc;
        if ((rc = model_balloc(M, nb * D, &t.TS1))) return rc;
        if ((rc = model_balloc(M, nb * D, &t.TS2))) return rc;
      }
      if (!attn_supported(R.T, R.D, R.NH) &&
          (rc = model_balloc(M, attn_gemm_floats(max_batch, R.T, R.NH), &t.SC)))
        return rc;
    }
    if (R.d.kind == GN_LAYER_MAXPOOL2D) {
      float *am = nullptr;
      if ((rc = model_balloc(M, (size_t)max_batch * R.out_len, &am))) return rc;
      R.argmax = reinterpret_cast<int32_t *>(am);
    }
    if (R.d.kind == GN_LAYER_FLATTEN) {
      // reshape.go:64-96: identity both ways; share the neighbours' buffers
      R.out_alias = true;
      R.gout_alias = true;
      R.gout = i > 0 ? M->L[i - 1].gout : nullptr;
      continue;
    }
    if ((rc = model_balloc(M, (size_t)max_batch * R.out_len, &R.out))) return rc;
    if (R.d.kind == GN_LAYER_POSENC && i > 0) {
      // PositionalEncoding.Backward returns its input gradient unchanged
      // (transformer.go:112-118): share the buffer with the layer below
      R.gout = M->L[i - 1].gout;
      R.gout_alias = true;
    } else if ((rc = model_balloc(M, (size_t)max_batch * R.out_len, &R.gout))) {
      return rc;
    }
  }
  if ((rc = model_balloc(M, (size_t)max_batch, &M->loss_rows))) return rc;
  if ((rc = model_balloc(M, (size_t)max_batch * M->L[0].in_len, &M->xin))) return rc;
  if ((rc = model_balloc(M, (size_t)max_batch * M->L.back().out_len, &M->yin))) return rc;
  return GN_OK;
}

extern "C" int gn_model_create(gn_ctx *c, const gn_layer_desc *layers, int32_t nlayers,
                               int32_t loss_kind, const gn_adam_desc *adam, int32_t max_batch,
                               int32_t workers, gn_model **out) {
  ENTRY(c);
  if (!layers || nlayers <= 0 || !out || max_batch <= 0)
    return set_err(c, GN_ERR_INVALID, "bad model_create args");
  if (loss_kind != GN_LOSS_MSE && loss_kind != GN_LOSS_CE)
    return set_err(c, GN_ERR_INVALID, "unknown loss %d", loss_kind);
  *out = nullptr;
  std::unique_ptr<gn_model> M(new gn_model);
  M->ctx = c;
  M->loss_kind = loss_kind;
  M->maxB = max_batch;
  M->workers = workers < 1 ? 1 : workers;
  if (adam) M->adam = *adam;
  if (M->adam.beta1 == 0) M->adam.beta1 = 0.9f;
  if (M->adam.beta2 == 0) M->adam.beta2 = 0.999f;
  if (M->adam.eps == 0) M->adam.eps = 1e-8f;
  M->L.resize(nlayers);

  // Shape propagation (the reference infers per-sample lengths at forward time)
  int len = layers[0].in_size;
  if (layers[0].kind == GN_LAYER_LSTM_UNROLLER || layers[0].kind == GN_LAYER_GRU_UNROLLER)
    len = layers[0].in_size * layers[0].seq_len;
  if (len <= 0) return set_err(c, GN_ERR_INVALID, "first layer needs in_size (input length)");
  int64_t off = 0;
  for (int i = 0; i < nlayers; ++i) {
    LayerRT &R = M->L[i];
    R.d = layers[i];
    R.in_len = len;
    switch (R.d.kind) {
      case GN_LAYER_DENSE:
        if (R.d.in_size != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: Dense in %d != incoming %d", i, R.d.in_size, len);
        if (R.d.out_size <= 0) return set_err(c, GN_ERR_INVALID, "layer %d: Dense out <= 0", i);
        if (plan_act(R.d.act, R.d.act_is_ptr, R.ap))
          return set_err(c, GN_ERR_INVALID, "layer %d: activation %d not supported", i, R.d.act);
        R.pcount = (int64_t)R.d.in_size * R.d.out_size + R.d.out_size;
        R.out_len = R.d.out_size;
        break;
      case GN_LAYER_DROPOUT:
        if (R.d.in_size != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: Dropout size %d != incoming %d", i, R.d.in_size, len);
        if (R.d.p < 0 || R.d.p > 1) return set_err(c, GN_ERR_INVALID, "dropout p out of [0,1]");
        R.out_len = len;
        break;
      case GN_LAYER_FLATTEN:
        R.out_len = len;
        break;
      case GN_LAYER_CONV2D: {
        ConvShape &cs = R.cs;
        cs.inC = R.d.in_channels;
        cs.outC = R.d.out_channels;
        cs.k = R.d.kernel;
        cs.stride = R.d.stride;
        cs.pad = R.d.padding;
        if (cs.inC <= 0 || cs.outC <= 0 || cs.k <= 0 || cs.stride <= 0 || cs.pad < 0)
          return set_err(c, GN_ERR_INVALID, "layer %d: bad Conv2D geometry", i);
        if (len % cs.inC)
          return set_err(c, GN_ERR_SHAPE, "layer %d: input %d not divisible by inChannels %d", i, len,
                         cs.inC);
        infer_hw(len / cs.inC, cs.H, cs.W);
        cs.oH = (cs.H + 2 * cs.pad - cs.k) / cs.stride + 1;
        cs.oW = (cs.W + 2 * cs.pad - cs.k) / cs.stride + 1;
        if (cs.H * cs.W * cs.inC != len || cs.oH <= 0 || cs.oW <= 0)
          return set_err(c, GN_ERR_SHAPE, "layer %d: Conv2D input %d is not C x H x W", i, len);
        if (plan_scalar_act(R.d.act, R.cfwd, R.cderiv))
          return set_err(c, GN_ERR_INVALID, "layer %d: activation %d not supported", i, R.d.act);
        R.pcount = (int64_t)cs.outC * cs.inC * cs.k * cs.k + cs.outC;
        R.out_len = cs.outC * cs.oH * cs.oW;
        break;
      }
      case GN_LAYER_MAXPOOL2D:
      case GN_LAYER_AVGPOOL2D: {  // avgpool2d.go:86-126 infers H, W the same way
        PoolShape &ps = R.ps;
        ps.C = R.d.in_channels <= 0 ? 1 : R.d.in_channels;  // maxpool2d.go:112-114 (Q8)
        ps.k = R.d.kernel;
        ps.stride = R.d.stride;
        ps.pad = R.d.padding;
        if (ps.k <= 0 || ps.stride <= 0 || ps.pad < 0)
          return set_err(c, GN_ERR_INVALID, "layer %d: bad pooling geometry", i);
        infer_hw(len / ps.C, ps.H, ps.W);
        ps.oH = (ps.H + 2 * ps.pad - ps.k) / ps.stride + 1;
        ps.oW = (ps.W + 2 * ps.pad - ps.k) / ps.stride + 1;
        if (ps.C * ps.H * ps.W != len || ps.oH <= 0 || ps.oW <= 0)
          return set_err(c, GN_ERR_SHAPE, "layer %d: pooling input %d is not C x H x W", i, len);
        R.out_len = ps.C * ps.oH * ps.oW;
        break;
      }
      case GN_LAYER_EMBEDDING:
        R.V = R.d.vocab;
        R.D = R.d.dim;
        R.T = len;  // tokens per sample
        if (R.V <= 0 || R.D <= 0) return set_err(c, GN_ERR_INVALID, "layer %d: bad Embedding", i);
        // below another layer it reads floor() of that layer's outputs as ids
        // and hands it a zero gradient (embedding.go:156-163); the first
        // Embedding's per-sample index-error flags cover every Embedding
        if (M->emb < 0) M->emb = i;
        R.pcount = (int64_t)R.V * R.D;
        R.out_len = R.T * R.D;
        break;
      case GN_LAYER_POSENC:
        R.T = R.d.seq_len;
        R.D = R.d.dim > 0 ? R.d.dim : (R.T > 0 ? len / R.T : 0);
        if (R.T <= 0 || R.D <= 0 || R.T * R.D != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: PositionalEncoding %dx%d != input %d", i, R.T, R.D, len);
        R.pcount = (int64_t)R.T * R.D;
        R.out_len = len;
        break;
      case GN_LAYER_TRANSFORMER:
        R.T = R.d.seq_len;
        R.D = R.d.dim;
        R.NH = R.d.num_heads;
        R.FF = R.d.ff_dim;
        R.causal = R.d.causal;
        if (R.T <= 0 || R.D <= 0 || R.FF <= 0 || R.T * R.D != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: TransformerBlock %dx%d != input %d", i, R.T, R.D, len);
        if (R.NH <= 0 || R.D % R.NH)
          return set_err(c, GN_ERR_SHAPE, "layer %d: dim %d is not a multiple of %d heads", i, R.D, R.NH);
        if (R.d.block_act < GN_BLOCK_ACT_RELU || R.d.block_act > GN_BLOCK_ACT_GELU ||
            R.d.block_norm < GN_BLOCK_NORM_LN || R.d.block_norm > GN_BLOCK_NORM_RMS)
          return set_err(c, GN_ERR_INVALID, "layer %d: unknown TransformerBlock act %d / norm %d", i,
                         R.d.block_act, R.d.block_norm);
        R.pcount = tb_offsets(R.D, R.FF, R.d.block_act, R.d.block_norm).total;
        R.out_len = len;
        break;
      case GN_LAYER_CLSPOOL:
        R.T = R.d.seq_len;
        R.D = R.d.dim;
        if (R.T <= 0 || R.D <= 0 || R.T * R.D != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: CLSPooling %dx%d != input %d", i, R.T, R.D, len);
        R.out_len = R.D;
        break;
      case GN_LAYER_GAP1D:  // transformer.go:1524-1600: mean over the seq_len rows of dim
        R.T = R.d.seq_len;
        R.D = R.d.dim;
        if (R.T <= 0 || R.D <= 0 || R.T * R.D != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: GlobalAveragePooling1D %dx%d != input %d", i, R.T,
                         R.D, len);
        R.out_len = R.D;
        break;
      case GN_LAYER_MHA:  // transformer.go:318-394: dim = input / seq_len when not given
        R.T = R.d.seq_len;
        R.D = R.d.dim > 0 ? R.d.dim : (R.T > 0 ? len / R.T : 0);
        R.NH = R.d.num_heads;
        R.causal = R.d.causal;
        if (R.T <= 0 || R.D <= 0 || R.T * R.D != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: MultiHeadAttention %dx%d != input %d", i, R.T, R.D, len);
        if (R.NH <= 0 || R.D % R.NH)
          return set_err(c, GN_ERR_SHAPE, "layer %d: dim %d is not a multiple of %d heads", i, R.D, R.NH);
        R.pcount = 4 * ((int64_t)R.D * R.D + R.D);
        R.out_len = len;
        break;
      case GN_LAYER_LAYERNORM:  // layernorm.go:193-304: rows of normalizedShape
        R.D = R.d.dim;
        if (R.D <= 0 || len % R.D)
          return set_err(c, GN_ERR_SHAPE, "layer %d: LayerNorm normalizedShape %d does not divide input %d",
                         i, R.D, len);
        if (!(R.d.eps >= 0)) return set_err(c, GN_ERR_INVALID, "layer %d: LayerNorm eps < 0", i);
        R.eps = R.d.eps > 0 ? R.d.eps : 1e-5f;  // the facade's eps (goneuron.go:220-227)
        R.pcount = 2 * (int64_t)R.D;               // [gamma | beta] (layernorm.go:83-118)
        R.out_len = len;
        break;
      case GN_LAYER_RMSNORM:  // rmsnorm.go:222-240: rows of normalizedShape
        R.D = R.d.dim;
        if (R.D <= 0 || len % R.D)
          return set_err(c, GN_ERR_SHAPE, "layer %d: RMSNorm normalizedShape %d does not divide input %d",
                         i, R.D, len);
        if (!(R.d.eps >= 0)) return set_err(c, GN_ERR_INVALID, "layer %d: RMSNorm eps < 0", i);
        R.eps = R.d.eps > 0 ? R.d.eps : 1e-5f;  // the facade's eps (goneuron.go:234)
        R.pcount = R.D;
        R.out_len = len;
        break;
      case GN_LAYER_BATCHNORM2D:  // batchnorm2d.go:103-135: gamma 1, beta 0 when affine
        R.C = R.d.in_channels;
        if (R.C <= 0 || len % R.C)
          return set_err(c, GN_ERR_SHAPE, "layer %d: BatchNorm2D channels %d do not divide input %d", i,
                         R.C, len);
        if (!(R.d.eps >= 0) || !(R.d.momentum >= 0 && R.d.momentum <= 1))
          return set_err(c, GN_ERR_INVALID, "layer %d: BatchNorm2D eps < 0 or momentum outside [0,1]", i);
        R.HW = len / R.C;
        R.eps = R.d.eps > 0 ? R.d.eps : 1e-5f;  // the facade's eps (goneuron.go:216)
        R.pcount = R.d.no_affine ? 0 : 2 * (int64_t)R.C;
        R.out_len = len;
        break;
      case GN_LAYER_SWIGLU:  // swiglu.go:73-100: [W | V], each out x in, no biases
        if (R.d.in_size != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: SwiGLU in %d != incoming %d", i, R.d.in_size, len);
        if (R.d.out_size <= 0) return set_err(c, GN_ERR_INVALID, "layer %d: SwiGLU out <= 0", i);
        R.pcount = 2 * (int64_t)R.d.in_size * R.d.out_size;
        R.out_len = R.d.out_size;
        break;
      case GN_LAYER_MOE:  // moe.go:47-138: [gating W (E x I), b | per expert W (O x I), b]
        R.E = R.d.num_experts;
        R.K = R.d.top_k;
        if (R.d.in_size != len)
          return set_err(c, GN_ERR_SHAPE, "layer %d: MoE in %d != incoming %d", i, R.d.in_size, len);
        if (R.d.out_size <= 0 || R.E <= 0 || R.E > MOE_MAX_E || R.K <= 0 || R.K > R.E)
          return set_err(c, GN_ERR_INVALID, "layer %d: bad MoE sizes (experts <= %d, 0 < k <= experts)",
                         i, MOE_MAX_E);
        R.pcount = (int64_t)R.E * R.d.in_size + R.E +
                   (int64_t)R.E * ((int64_t)R.d.out_size * R.d.in_size + R.d.out_size);
        R.out_len = R.d.out_size;
        break;
      case GN_LAYER_GRU_UNROLLER:  // gru.go:110-167: [Wx 3H x I | Wh 2H x H | b 3H]
        R.T = R.d.seq_len;
        R.I = R.d.in_size;
        R.H = R.d.out_size;
        if (R.T <= 0 || R.I <= 0 || !gru_supported(R.H))
          return set_err(c, GN_ERR_INVALID, "layer %d: bad SequenceUnroller(GRU) sizes (hidden <= 1024)", i);
        if (i != 0 && len != R.T * R.I)
          return set_err(c, GN_ERR_SHAPE, "layer %d: SequenceUnroller(GRU) takes %d x %d, gets %d", i,
                         R.T, R.I, len);
        R.in_len = R.T * R.I;
        len = R.in_len;
        R.pcount = (int64_t)3 * R.H * R.I + (int64_t)2 * R.H * R.H + 3 * R.H;
        R.out_len = R.d.return_sequences ? R.T * R.H : R.H;  // unroller.go:21-43
        break;
      case GN_LAYER_LSTM_UNROLLER: {
        R.T = R.d.seq_len;
        R.I = R.d.in_size;
        R.H = R.d.out_size;
        if (R.T <= 0 || R.I <= 0 || R.H <= 0 || R.H > 1024)
          return set_err(c, GN_ERR_INVALID, "layer %d: bad SequenceUnroller(LSTM) sizes", i);
        if (i != 0 && len != R.T * R.I)
          return set_err(c, GN_ERR_SHAPE, "layer %d: SequenceUnroller(LSTM) takes %d x %d, gets %d", i,
                         R.T, R.I, len);
        R.in_len = R.T * R.I;  // in_size is the per-step input size here
        len = R.in_len;
        R.pcount = (int64_t)4 * R.H * R.I + (int64_t)4 * R.H * R.H + 4 * R.H;
        R.out_len = R.d.return_sequences ? R.T * R.H : R.H;  // unroller.go:21-43
        break;
      }
      default:
        return set_err(c, GN_ERR_UNSUPPORTED, "layer %d: kind %d not built in this library", i,
                       R.d.kind);
    }
    R.poff = off;
    off += R.pcount;
    len = R.out_len;
  }
  // any layer may be the output layer (Network.Forward hands its output to the
  // loss, net.go:212-223); a non-Dense one gets dL/dy itself, with no
  // activation applied by the loss kernel
  if (M->L.back().d.kind != GN_LAYER_DENSE) M->L.back().ap = ActPlan{ROW_NONE, F_IDENTITY, D_ONE, false};
  M->nparams = off;
  M->region = (off + 63) / 64 * 64;

  // Arena: params | grads | m | v (each region 256 B aligned)
  int rc = model_alloc(M.get(), (size_t)M->region * 4, &M->arena);
  if (rc) return rc;
  M->params = M->arena;
  M->grads = M->arena + M->region;
  M->m = M->arena + 2 * M->region;
  M->v = M->arena + 3 * M->region;
  HIP_OK(c, hipMemsetAsync(M->arena, 0, (size_t)M->region * 4 * sizeof(float), c->stream));

  // Initial parameters (the reference's seeded LCG per layer) and the state
  // that does not depend on the batch size; the batch-sized buffers follow in
  // alloc_batch, which gn_model_reserve reruns for a larger batch.
  std::vector<float> host((size_t)std::max<int64_t>(off, 1), 0.f);
  for (int i = 0; i < nlayers; ++i) {
    LayerRT &R = M->L[i];
    // training flags as the layers are constructed: Dropout and BatchNorm2D
    // start in training mode (dropout.go:56, batchnorm2d.go:88), MoE does not
    // (NewMoE leaves its flag false, moe.go:46-90)
    R.train = R.d.kind == GN_LAYER_MOE ? 0 : 1;
    if (R.d.kind == GN_LAYER_DENSE) init_dense(host.data() + R.poff, R.d.in_size, R.d.out_size);
    if (R.d.kind == GN_LAYER_CONV2D) init_conv(host.data() + R.poff, R.cs.inC, R.cs.outC, R.cs.k);
    if (R.d.kind == GN_LAYER_EMBEDDING) init_embedding(host.data() + R.poff, R.V, R.D);
    if (R.d.kind == GN_LAYER_POSENC) init_posenc(host.data() + R.poff, R.T, R.D);
    if (R.d.kind == GN_LAYER_TRANSFORMER && R.d.use_rope) {
      // parameters stay 0 (Q11); applyRoPE's angles (transformer.go:215-221)
      // in float32, computed once
      LayerRT::Tb &t = R.tb;
      const int hd = R.D / R.NH, half = hd / 2;
      std::vector<float> cs((size_t)R.T * std::max(half, 1)), sn(cs.size());
      for (int tt = 0; tt < R.T; ++tt)
        for (int k = 0; k < half; ++k) {
          const float theta = (float)pow(10000.0, -(double)(2 * k) / (double)hd);
          const float m = (float)tt * theta;
          cs[(size_t)tt * half + k] = (float)cos((double)m);
          sn[(size_t)tt * half + k] = (float)sin((double)m);
        }
      if ((rc = model_alloc(M.get(), cs.size(), &t.rcos))) return rc;
      if ((rc = model_alloc(M.get(), sn.size(), &t.rsin))) return rc;
      HIP_OK(c, hipMemcpyAsync(t.rcos, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice,
                               c->stream));
      HIP_OK(c, hipMemcpyAsync(t.rsin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice,
                               c->stream));
      // the host vectors go out of scope: finish the copies first
      HIP_OK(c, hipStreamSynchronize(c->stream));
    }
    if (R.d.kind == GN_LAYER_LSTM_UNROLLER) {
      init_lstm(host.data() + R.poff, R.I, R.H);
      if ((rc = model_alloc(M.get(), (size_t)R.H * R.H, &R.WhT))) return rc;
    }
    if (R.d.kind == GN_LAYER_MOE) {
      // parameters stay 0: Build rebinds the gating and expert layers to one
      // fresh zero block (moe.go:122-135)
      R.mrng.assign(65, 42);  // NewRNG(42) in the layer and in every worker clone
    }
    if (R.d.kind == GN_LAYER_GRU_UNROLLER) {
      init_gru(host.data() + R.poff, R.I, R.H);
      if ((rc = model_alloc(M.get(), 2 * (size_t)R.H * R.H, &R.WhT))) return rc;
    }
    if (R.d.kind == GN_LAYER_BATCHNORM2D) {
      if (R.pcount) std::fill(host.begin() + R.poff, host.begin() + R.poff + R.C, 1.0f);
      if ((rc = model_alloc(M.get(), R.C, &R.rmean))) return rc;
      if ((rc = model_alloc(M.get(), R.C, &R.rvar))) return rc;
      std::vector<float> ones(R.C, 1.0f);
      HIP_OK(c, hipMemsetAsync(R.rmean, 0, R.C * sizeof(float), c->stream));
      HIP_OK(c, hipMemcpyAsync(R.rvar, ones.data(), R.C * sizeof(float), hipMemcpyHostToDevice,
                               c->stream));
      HIP_OK(c, hipStreamSynchronize(c->stream));  // `ones` goes out of scope
    }
    if (R.d.kind == GN_LAYER_SWIGLU) init_swiglu(host.data() + R.poff, R.d.in_size, R.d.out_size);
    if (R.d.kind == GN_LAYER_RMSNORM)
      std::fill(host.begin() + R.poff, host.begin() + R.poff + R.D, 1.0f);  // rmsnorm.go:80-82
    if (R.d.kind == GN_LAYER_LAYERNORM)  // gamma 1, beta 0 (layernorm.go:83-118)
      std::fill(host.begin() + R.poff, host.begin() + R.poff + R.D, 1.0f);
    if (R.d.kind == GN_LAYER_MHA && R.d.use_rope) {
      // parameters stay 0 (Build rebinds wQ, wK, wV, wOut to a fresh zero
      // buffer, transformer.go:367-379); the rotary angles once
      std::vector<float> cs, sn;
      rope_tables(R.T, R.D / R.NH, cs, sn);
      if ((rc = model_alloc(M.get(), cs.size(), &R.tb.rcos))) return rc;
      if ((rc = model_alloc(M.get(), sn.size(), &R.tb.rsin))) return rc;
      HIP_OK(c, hipMemcpyAsync(R.tb.rcos, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice,
                               c->stream));
      HIP_OK(c, hipMemcpyAsync(R.tb.rsin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice,
                               c->stream));
      HIP_OK(c, hipStreamSynchronize(c->stream));  // the host tables go out of scope
    }
    if (R.d.kind == GN_LAYER_DROPOUT) {
      // Q9: Dropout.Reset reseeds RNG(42) before every sample (dropout.go:399-401),
      // so one mask of the first `size` draws serves every sample and step.
      std::vector<float> mk(R.d.in_size);
      uint64_t s = 42;
      for (int k = 0; k < R.d.in_size; ++k) mk[k] = lcg_float(s) < R.d.p ? 0.f : 1.f;
      const float keep = 1.0f - R.d.p;
      R.scale = 1.0f / keep;
      if ((rc = model_alloc(M.get(), R.d.in_size, &R.mask))) return rc;
      HIP_OK(c, hipMemcpyAsync(R.mask, mk.data(), mk.size() * sizeof(float), hipMemcpyHostToDevice,
                               c->stream));
      std::vector<float> fac(R.d.in_size);
      for (int k = 0; k < R.d.in_size; ++k) fac[k] = mk[k] > 0.f ? R.scale : 0.f;
      if ((rc = model_alloc(M.get(), R.d.in_size, &R.dfac))) return rc;
      HIP_OK(c, hipMemcpyAsync(R.dfac, fac.data(), fac.size() * sizeof(float), hipMemcpyHostToDevice,
                               c->stream));
      HIP_OK(c, hipStreamSynchronize(c->stream));  // `mk` goes out of scope
    }
  }
  HIP_OK(c, hipMemcpyAsync(M->params, host.data(), (size_t)off * sizeof(float),
                           hipMemcpyHostToDevice, c->stream));

  if ((rc = alloc_batch(M.get()))) return rc;
  HIP_OK(c, hipStreamSynchronize(c->stream));
  *out = M.release();
  return GN_OK;
}

// Network.TrainBatch and PredictBatch take any batch size: a batch above the
// size the buffers were made for rebuilds the batch-sized buffers (layer
// outputs and gradients, saved state, staging) and keeps everything else —
// parameters, gradients, Adam moments and timestep, BatchNorm2D running
// statistics, MoE noise streams, training flags.
extern "C" int gn_model_reserve(gn_model *M, int32_t max_batch) {
  if (!M) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  if (max_batch <= 0) return set_err(c, GN_ERR_INVALID, "max_batch %d <= 0", max_batch);
  if (max_batch <= M->maxB) return GN_OK;
  HIP_OK(c, hipStreamSynchronize(c->stream));
  HIP_OK(c, hipStreamSynchronize(c->aux));
  const int old = M->maxB;
  drop_graphs(M);  // they hold the old batch buffers
  free_batch(M);
  M->maxB = max_batch;
  int rc = alloc_batch(M);
  if (rc) {  // back to the old size; the caller's model stays usable
    const std::string msg = c->err;
    free_batch(M);
    M->maxB = old;
    if (alloc_batch(M)) return set_err(c, GN_ERR_OOM, "%s; restoring batch %d failed too", msg.c_str(), old);
    return set_err(c, rc, "%s", msg.c_str());
  }
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return GN_OK;
}

extern "C" int gn_model_nparams(gn_model *M, int64_t *n) {
  if (!M || !n) return GN_ERR_INVALID;
  *n = M->nparams;
  return GN_OK;
}

extern "C" int gn_model_layer_params(gn_model *M, int32_t layer, int64_t *offset, int64_t *count) {
  if (!M || layer < 0 || layer >= (int)M->L.size()) return GN_ERR_INVALID;
  if (offset) *offset = M->L[layer].poff;
  if (count) *count = M->L[layer].pcount;
  return GN_OK;
}

extern "C" int gn_model_out_size(gn_model *M, int32_t *n) {
  if (!M || !n) return GN_ERR_INVALID;
  *n = M->L.back().out_len;
  return GN_OK;
}

extern "C" int gn_model_layer_count(gn_model *M, int32_t *n) {
  if (!M || !n) return GN_ERR_INVALID;
  *n = (int32_t)M->L.size();
  return GN_OK;
}

extern "C" int gn_model_layer_desc(gn_model *M, int32_t i, gn_layer_desc *d) {
  if (!M || !d) return GN_ERR_INVALID;
  if (i < 0 || i >= (int)M->L.size()) return set_err(M->ctx, GN_ERR_INVALID, "layer %d out of range", i);
  *d = M->L[i].d;
  return GN_OK;
}

extern "C" int gn_model_loss_kind(gn_model *M, int32_t *k) {
  if (!M || !k) return GN_ERR_INVALID;
  *k = M->loss_kind;
  return GN_OK;
}

static int arena_copy(gn_model *M, float *region, float *host, int64_t off, int64_t n, bool d2h) {
  gn_ctx *c = M->ctx;
  ENTRY(c);
  if (off < 0 || n < 0 || off + n > M->nparams || (!host && n))
    return set_err(c, GN_ERR_INVALID, "arena range [%lld,+%lld) outside %lld", (long long)off,
                   (long long)n, (long long)M->nparams);
  if (d2h)
    HIP_OK(c, hipMemcpyAsync(host, region + off, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
  else
    HIP_OK(c, hipMemcpyAsync(region + off, host, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return GN_OK;
}

extern "C" int gn_model_get_params(gn_model *M, float *dst, int64_t off, int64_t n) {
  if (!M) return GN_ERR_INVALID;
  return arena_copy(M, M->params, dst, off, n, true);
}
extern "C" int gn_model_set_params(gn_model *M, const float *src, int64_t off, int64_t n) {
  if (!M) return GN_ERR_INVALID;
  return arena_copy(M, M->params, const_cast<float *>(src), off, n, false);
}
extern "C" int gn_model_get_grads(gn_model *M, float *dst, int64_t off, int64_t n) {
  if (!M) return GN_ERR_INVALID;
  return arena_copy(M, M->grads, dst, off, n, true);
}
extern "C" int gn_model_get_adam(gn_model *M, float *mdst, float *vdst, int64_t off, int64_t n,
                                 int32_t *timestep) {
  if (!M) return GN_ERR_INVALID;
  int rc = GN_OK;
  if (mdst && (rc = arena_copy(M, M->m, mdst, off, n, true))) return rc;
  if (vdst && (rc = arena_copy(M, M->v, vdst, off, n, true))) return rc;
  if (timestep) *timestep = M->timestep;
  return GN_OK;
}
extern "C" int gn_model_set_adam(gn_model *M, const float *msrc, const float *vsrc, int64_t off,
                                 int64_t n, int32_t timestep) {
  if (!M) return GN_ERR_INVALID;
  if (timestep < 0) return set_err(M->ctx, GN_ERR_INVALID, "negative Adam timestep");
  int rc = GN_OK;
  if (msrc && (rc = arena_copy(M, M->m, const_cast<float *>(msrc), off, n, false))) return rc;
  if (vsrc && (rc = arena_copy(M, M->v, const_cast<float *>(vsrc), off, n, false))) return rc;
  M->timestep = timestep;
  return GN_OK;
}
extern "C" int gn_model_arena(gn_model *M, float **p, float **g, float **m, float **v) {
  if (!M) return GN_ERR_INVALID;
  if (p) *p = M->params;
  if (g) *g = M->grads;
  if (m) *m = M->m;
  if (v) *v = M->v;
  return GN_OK;
}

// Network.SetTraining (net.go:187-193): every layer of the network itself;
// worker clones keep the flags they were made with.
extern "C" int gn_model_set_training(gn_model *M, int32_t t) {
  if (!M) return GN_ERR_INVALID;
  for (LayerRT &R : M->L) R.train = t ? 1 : 0;
  return GN_OK;
}

extern "C" int gn_model_get_training(gn_model *M, int32_t layer, int32_t *t) {
  if (!M || !t || layer < 0 || layer >= (int)M->L.size()) return GN_ERR_INVALID;
  *t = M->L[layer].train;
  return GN_OK;
}

// Flags in effect for a pass over B samples: the network's own for inference
// and for trainBatchSequential; for trainBatchParallel those of the worker
// clones that run the chunks, clones being made (with the network's current
// flags) the first time that many workers are needed (net.go:129-152).
static int pass_flags(gn_model *M, int B, bool train) {
  const int n = (int)M->L.size();
  M->eff.assign(n, 0);
  for (int i = 0; i < n; ++i) M->eff[i] = (char)M->L[i].train;
  if (!train || M->workers <= 1) return GN_OK;
  const int W = std::min(M->workers, B);
  while ((int)M->clone_train.size() < W) M->clone_train.push_back(M->eff);
  for (int i = 0; i < n; ++i) {
    const char f = M->clone_train[0][i];
    for (int w = 1; w < W; ++w)
      if (M->clone_train[w][i] != f)
        return set_err(M->ctx, GN_ERR_UNSUPPORTED,
                       "layer %d: worker clones made at different times hold different training "
                       "flags; chunks with mixed flags are not built", i);
    M->eff[i] = f;
  }
  return GN_OK;
}

// A standalone MultiHeadAttention's buffers, sized for the model's max batch
static MhaBufs mha_bufs(const gn_model *M, const LayerRT &R) {
  const LayerRT::Tb &t = R.tb;
  return MhaBufs{t.Q, t.K, t.V, t.O, t.GO, t.GQ, t.GK, t.GV, t.S, t.S3, t.rcos, t.rsin, t.SC,
                 (int64_t)M->maxB * R.D};
}

// ---------------------------------------------------------------------------
// TransformerBlock (post-norm, transformer.go:1080-1279) over B samples.
// ---------------------------------------------------------------------------
static hipError_t gemm_nt(gn_ctx *c, const float *A, const float *Bw, const float *bias, float *C,
                          int M, int N, int K, int epi, int act, const float *aux) {
  GemmArgs a{};
  a.M = M; a.N = N; a.K = K;
  a.A = A; a.lda = K; a.B = Bw; a.ldb = K;
  a.C = C; a.ldc = N; a.alpha = 1.f; a.bias = bias; a.act = act;
  a.aux = aux; a.ldaux = N;
  a.ws = c->scratch; a.ws_cap = c->scratch_floats;
  KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(a));
  return launch_gemm('N', 'T', epi, a, c->stream);
}

// C[M,N] = A[M,K] W[K,N] (+ epilogue)
static hipError_t gemm_nn(gn_ctx *c, const float *A, const float *Wm, float *C, int M, int N, int K,
                          int epi, int act, const float *aux, int aux_div) {
  GemmArgs a{};
  a.M = M; a.N = N; a.K = K;
  a.A = A; a.lda = K; a.B = Wm; a.ldb = N;
  a.C = C; a.ldc = N; a.alpha = 1.f; a.act = act;
  a.aux = aux; a.ldaux = N; a.aux_div = aux_div;
  a.ws = c->scratch; a.ws_cap = c->scratch_floats;
  KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
  return launch_gemm('N', 'N', epi, a, c->stream);
}

// Q10 weight gradient of a per-token Dense: dW[M,N] = scale * S^T Xlast, with
// S [B, M] the per-sample token sums of dz and Xlast the last token's input
// row of every sample (row stride T*N).
// Q10 gradients of one Linear in the block: dW = scale * S^T x_last and
// db = scale * colsum(S) from its per-sample token sums S [B][M], one launch
static hipError_t tb_tok_dw(gn_ctx *c, const float *S, const float *X, float *dW, float *db, int B,
                            int T, int M, int N, float scale, hipStream_t st) {
  TokDwSet set{};
  set.S[0] = S;
  set.X[0] = X + (int64_t)(T - 1) * N;
  set.dW[0] = dW;
  set.db[0] = db;
  KTimer kt(c, GN_KCLASS_OTHER, "tok_dw", f4((double)B * M + (double)B * N + (double)M * N + M), st);
  return launch_tok_dw(set, 1, B, M, N, M, T * N, scale, st);
}

// Block norm k (0: norm1, 1: norm2) forward: LayerNorm (stats = mean, std)
// or RMSNorm(dim, 1e-5) (stats = rms), transformer.go:928-934.
// cls (LayerNorm only, may be null): token 0 of every sample also written
// there (the output of a CLSPooling above the block).
static hipError_t tb_norm_fwd(gn_ctx *c, const LayerRT &R, const float *P, const TbOff &o, int k,
                              const float *x, float *y, float *st, int rows, float *cls = nullptr) {
  const float *g = P + (k == 0 ? o.g1 : o.g2), *be = P + (k == 0 ? o.be1 : o.be2);
  const bool rms = R.d.block_norm == GN_BLOCK_NORM_RMS;
  // read x, write y and the per-row statistics
  KTimer kt(c, GN_KCLASS_OTHER, rms ? "rms_fwd" : "ln_fwd",
            f4(2.0 * rows * R.D + (rms ? 1 : 2) * rows + (cls ? (double)rows / R.T * R.D : 0.0)));
  if (rms) return launch_rms_fwd(x, g, y, st, rows, R.D, 1e-5f, c->stream);
  return launch_ln_fwd(x, g, be, y, st, rows, R.D, 1e-5f, c->stream, cls, R.T);
}

// The block's norms run the one-pass LayerNorm backward with its partials
// kept (t.LP*, t.TS*): the block's parameter gradients then come from one
// tb_param_kernel launch, and a CLSPooling above the block needs no
// gradient scatter (the norm-2 backward reads the pooled rows).
static bool tb_fused_params(const LayerRT &R) { return R.tb.LP1 != nullptr; }
// A CLSPooling above a block whose last norm is a LayerNorm: the norm's
// forward writes the pooled rows, and with the fused parameter path its
// backward reads the pooled gradient (no cls_fwd / cls_bwd launch).
static bool tb_cls_fusable(const LayerRT &R, const LayerRT &up) {
  return up.d.kind == GN_LAYER_CLSPOOL && R.d.kind == GN_LAYER_TRANSFORMER &&
         R.d.block_norm != GN_BLOCK_NORM_RMS && up.T == R.T && up.D == R.D && tb_fused_params(R);
}

// Block norm backward: dx into dx, gamma (and LayerNorm beta) gradients.
static hipError_t tb_norm_bwd(gn_ctx *c, const LayerRT &R, const float *P, float *G, const TbOff &o,
                              int k, const float *g, const float *x, const float *st, float *dx,
                              int rows, float scale) {
  const int D = R.D;
  const int64_t og = k == 0 ? o.g1 : o.g2, ob = k == 0 ? o.be1 : o.be2;
  LayerRT::Tb &t = const_cast<LayerRT &>(R).tb;
  const bool rms = R.d.block_norm == GN_BLOCK_NORM_RMS;
  hipError_t e;
  if (!rms) {
    // read g, x and the statistics, write dx; gamma / beta sums from the
    // kernel's per-block partials
    KTimer kt(c, GN_KCLASS_OTHER, "ln_bwd", f4(3.0 * rows * D + 2.0 * rows + 2.0 * D));
    e = launch_ln_bwd_params(g, x, P + og, st, dx, G + og, G + ob, rows, D, scale, c->scratch,
                             c->scratch_floats, c->stream);
    if (e != hipErrorNotSupported) return e;
    (void)hipGetLastError();
  }
  {
    // read g, x and the statistics, write dx and g * xhat
    KTimer kt(c, GN_KCLASS_OTHER, rms ? "rms_bwd" : "ln_bwd", f4(4.0 * rows * D + (rms ? 1 : 2) * rows));
    if (rms) {
      e = launch_rms_bwd(g, x, P + og, st, dx, t.GX, rows, D, c->stream);
    } else {
      e = launch_ln_bwd(g, x, P + og, st, dx, t.GX, rows, D, c->stream);
    }
  }
  if (e != hipSuccess) return e;
  // gamma (and for LayerNorm beta) gradients in one launch pair
  const float *src[2] = {t.GX, g};
  float *dst[2] = {G + og, G + ob};
  const int nm = rms ? 1 : 2;
  KTimer kt(c, GN_KCLASS_OTHER, "colsum", nm * f4((double)rows * D + D));
  return launch_colsum_multi(src, dst, nm, rows, D, D, scale, c->scratch, c->scratch_floats, c->stream);
}

// cls (may be null): the output of a CLSPooling above, written by norm 2
static int tb_forward(gn_model *M, LayerRT &R, const float *X, int B, float *cls) {
  gn_ctx *c = M->ctx;
  const int D = R.D, FF = R.FF, rows = B * R.T;
  const TbOff o = tb_offsets(D, FF, R.d.block_act, R.d.block_norm);
  const float *P = M->params + R.poff;
  LayerRT::Tb &t = R.tb;
  // per-token projections: Q/K/V = X W^T + b (Dense with Linear activation),
  // one launch for the three (equal strides between wQ, wK, wV, their biases
  // and the Q, K, V buffers)
  {
    GemmArgs a{};
    a.M = rows; a.N = D; a.K = D;
    a.A = X; a.lda = D; a.B = P + o.wq; a.ldb = D;
    a.C = t.Q; a.ldc = D; a.alpha = 1.f; a.bias = P + o.bq; a.act = F_IDENTITY;
    a.ws = c->scratch; a.ws_cap = c->scratch_floats;
    a.nbatch = 3;
    a.bstride_B = o.wk - o.wq;
    a.bstride_bias = o.bk - o.bq;
    a.bstride_C = t.K - t.Q;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", gemm_flops(a));
    HIP_OK(c, launch_gemm('N', 'T', EPI_BIAS_ACT, a, c->stream));
  }
  if (R.d.use_rope) {  // transformer.go:457-461; the backward reads the rotated Q, K too
    KTimer kt(c, GN_KCLASS_OTHER, "rope", 2 * f4(2.0 * rows * D));
    HIP_OK(c, launch_rope(t.Q, t.rcos, t.rsin, rows, R.T, R.NH, D / R.NH, 0, c->stream));
    HIP_OK(c, launch_rope(t.K, t.rcos, t.rsin, rows, R.T, R.NH, D / R.NH, 0, c->stream));
  }
  {
    KTimer kt(c, GN_KCLASS_OTHER, "attn_fwd", attn_flops(B, R.T, R.NH, D / R.NH, R.causal, false));
    if (t.SC)
      HIP_OK(c, launch_attn_fwd_gemm(t.Q, t.K, t.V, t.O, B, R.T, D, R.NH, R.causal, t.SC, c->stream));
    else
      HIP_OK(c, launch_attn_fwd(t.Q, t.K, t.V, t.O, B, R.T, D, R.NH, R.causal, c->stream));
  }
  // res1 = x + wOut(o): the residual add rides in the GEMM epilogue
  HIP_OK(c, gemm_nt(c, t.O, P + o.wo, P + o.bo, t.RES1, rows, D, D, EPI_BIAS_ADD, 0, X));
  HIP_OK(c, tb_norm_fwd(c, R, P, o, 0, t.RES1, t.N1, t.st1, rows));
  if (R.d.block_act == GN_BLOCK_ACT_SWIGLU) {
    // Z = [gate | up] for every token (one GEMM against [W | V]), MID = swish(gate) * up
    HIP_OK(c, gemm_nt(c, t.N1, P + o.w1, nullptr, t.Z, rows, 2 * FF, D, EPI_BIAS_ACT, F_IDENTITY,
                      nullptr));
    KTimer kt(c, GN_KCLASS_OTHER, "swiglu_fwd", f4(3.0 * rows * FF));
    HIP_OK(c, launch_swiglu_fwd(t.Z, t.MID, rows, FF, c->stream));
  } else {
    // ReLU, or GELU as a value activation: identity forward (ActTypeNone)
    const int f = R.d.block_act == GN_BLOCK_ACT_GELU ? F_IDENTITY : F_RELU;
    HIP_OK(c, gemm_nt(c, t.N1, P + o.w1, P + o.b1, t.MID, rows, FF, D, EPI_BIAS_ACT, f, nullptr));
  }
  HIP_OK(c, gemm_nt(c, t.MID, P + o.w2, P + o.b2, t.RES2, rows, D, FF, EPI_BIAS_ADD, 0, t.N1));
  HIP_OK(c, tb_norm_fwd(c, R, P, o, 1, t.RES2, R.out, t.st2, rows, cls));
  return GN_OK;
}

// side: a stream for the parameter-gradient kernels (token sums and the Q10
// weight gradients read what the main stream has written and write only S,
// S3 and this layer's gradients), branched off the main stream after each
// input they read; null runs them on the main stream.
// gpool (fused parameter path only, may be null): the gradient of a
// CLSPooling above the block, read by the norm-2 backward in place of a
// scattered R.gout.
static int tb_backward(gn_model *M, LayerRT &R, const float *X, float *gin, int B, float scale,
                       hipStream_t side, const float *gpool) {
  gn_ctx *c = M->ctx;
  const hipStream_t ss = side ? side : c->stream;
  auto fork = [&]() -> hipError_t {
    if (!side) return hipSuccess;
    const hipError_t e = hipEventRecord(M->fork_ev, c->stream);
    return e != hipSuccess ? e : hipStreamWaitEvent(side, M->fork_ev, 0);
  };
  const int D = R.D, FF = R.FF, T = R.T, rows = B * T;
  const TbOff o = tb_offsets(D, FF, R.d.block_act, R.d.block_norm);
  const float *P = M->params + R.poff;
  float *G = M->grads + R.poff;
  LayerRT::Tb &t = R.tb;
  float *cs = c->scratch;
  const size_t cap = c->scratch_floats;
  const bool fused = tb_fused_params(R);
  if (gpool && !fused) return set_err(c, GN_ERR_INVALID, "pooled gradient without the fused block backward");
  // fused: the parameter-gradient jobs, run as one launch once their inputs exist
  TbParamSet pset{};
  double pbytes = 0;
  const int nblk = ln_bwd_blocks(rows), np = T / ln_bwd_rows_per_block();
  auto lin_job = [&](const float *S, int snp, int64_t sps, const float *Xl, int Mo, int Ni, int64_t wo,
                     int64_t bo) {
    TbParamJob &j = pset.lin[pset.nlin++];
    j.S = S; j.np = snp; j.ps = sps;
    j.X = Xl + (int64_t)(T - 1) * Ni; j.ldx = (int64_t)T * Ni;
    j.dW = G + wo; j.db = G + bo; j.M = Mo; j.N = Ni;
    pbytes += f4((double)B * snp * Mo + (double)B * Ni + (double)Mo * Ni + Mo);
  };
  // tsx (may be null): a [B][T][FF] matrix whose token sums the same launch writes to t.S
  auto norm_bwd_fused = [&](int k, const float *g, const float *gp, const float *x, const float *st,
                            float *dx, float *lp, float *ts, const float *tsx = nullptr) -> hipError_t {
    KTimer kt(c, GN_KCLASS_OTHER, "ln_bwd",
              f4((gp ? 2.0 : 3.0) * rows * D + 2.0 * rows + (double)nblk * 3 * D) +
                  (tsx ? token_sum_bytes(B, T, FF) : 0.0));
    const hipError_t e = launch_ln_bwd_part(gp ? nullptr : g, gp, T, x, P + (k == 0 ? o.g1 : o.g2), st, dx, lp,
                                            ts, rows, D, c->stream, tsx, t.S, B, T, FF);
    TbLnJob &j = pset.ln[pset.nln++];
    j.part = lp; j.nblk = nblk; j.N = D;
    j.dgam = G + (k == 0 ? o.g1 : o.g2); j.dbet = G + (k == 0 ? o.be1 : o.be2);
    pbytes += f4((double)nblk * 2 * D + 2.0 * D);
    return e;
  };
  // norm 2 (LayerNorm: Q18 formula; RMSNorm: Q19), gamma / beta column sums
  if (fused) {
    HIP_OK(c, norm_bwd_fused(1, R.gout, gpool, t.RES2, t.st2, t.G1, t.LP2, t.TS2));
    // ff2 (Linear): dz2 = dRES2, its token sums from the norm's block partials
    lin_job(t.TS2, np, D, t.MID, D, FF, o.w2, o.b2);
  } else {
    HIP_OK(c, tb_norm_bwd(c, R, P, G, o, 1, R.gout, t.RES2, t.st2, t.G1, rows, scale));
    HIP_OK(c, fork());
    {
      // ff2 (Linear): dz2 = dRES2; the bias gradient sums every token, i.e. the
      // per-sample token sums S that the Q10 weight gradient needs anyway
      KTimer kt(c, GN_KCLASS_OTHER, "token_sum", token_sum_bytes(B, T, D), ss);
      HIP_OK(c, launch_token_sum(t.G1, t.S, B, T, D, ss));
    }
    HIP_OK(c, tb_tok_dw(c, t.S, t.MID, G + o.w2, G + o.b2, B, T, D, FF, scale, ss));
  }
  if (R.d.block_act == GN_BLOCK_ACT_SWIGLU) {
    // ff1 = SwiGLU called per token: its one saved entry (the last token's
    // input, gate and up) serves the first Backward (token 0); the later ones
    // return nil, so tokens 1.. get no feed-forward gradient (swiglu.go:126-133,
    // 175-179).  mg = dRES2[token 0] W2; dZ from the last token's Z.
    GemmArgs a{};
    a.M = B; a.N = FF; a.K = D;
    a.A = t.G1; a.lda = T * D;
    a.B = P + o.w2; a.ldb = FF;
    a.C = t.MG; a.ldc = FF; a.alpha = 1.f;
    a.ws = cs; a.ws_cap = cap;
    {
      KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
      HIP_OK(c, launch_gemm('N', 'N', EPI_SCALE, a, c->stream));
    }
    {
      KTimer kt(c, GN_KCLASS_OTHER, "swiglu_bwd", f4(5.0 * B * FF));
      HIP_OK(c, launch_swiglu_bwd(t.MG, t.Z + (int64_t)(T - 1) * 2 * FF, T * 2 * FF, t.DZS, B, FF,
                                  c->stream));
    }
    // [dW | dV] = scale * dZ^T x_last
    GemmArgs w{};
    w.M = 2 * FF; w.N = D; w.K = B;
    w.A = t.DZS; w.lda = 2 * FF;
    w.B = t.N1 + (int64_t)(T - 1) * D; w.ldb = T * D;
    w.C = G + o.w1; w.ldc = D; w.alpha = scale;
    w.ws = cs; w.ws_cap = cap;
    {
      KTimer kt(c, GN_KCLASS_GEMM, "gemm_dw", gemm_flops(w));
      HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, w, c->stream));
    }
    // combined = dRES2, plus dZ [W; V] on each sample's token 0
    HIP_OK(c, hipMemcpyAsync(t.COMB, t.G1, (size_t)rows * D * sizeof(float), hipMemcpyDeviceToDevice,
                             c->stream));
    GemmArgs d{};
    d.M = B; d.N = D; d.K = 2 * FF;
    d.A = t.DZS; d.lda = 2 * FF;
    d.B = P + o.w1; d.ldb = D;
    d.C = t.COMB; d.ldc = T * D; d.alpha = 1.f;
    d.aux = t.G1; d.ldaux = T * D;
    d.ws = cs; d.ws_cap = cap;
    KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(d));
    HIP_OK(c, launch_gemm('N', 'N', EPI_BIAS_ADD, d, c->stream));
  } else {
    // ff1: dz1 = (dz2 W2) * act'(last token's pre-activation) (Q10); ReLU from
    // its output, GELU (identity forward) from MID, which is the pre-activation
    const int dk = R.d.block_act == GN_BLOCK_ACT_GELU ? D_GELU : D_RELU;
    HIP_OK(c, gemm_nn(c, t.G1, P + o.w2, t.DZ1, rows, FF, D, EPI_DACT, dk, t.MID, T));
    if (fused) {
      // the token sums of dz1 come with the norm-1 backward's launch below
      lin_job(t.S, 1, FF, t.N1, FF, D, o.w1, o.b1);
    } else {
      HIP_OK(c, fork());
      {
        KTimer kt(c, GN_KCLASS_OTHER, "token_sum", token_sum_bytes(B, T, FF), ss);
        HIP_OK(c, launch_token_sum(t.DZ1, t.S, B, T, FF, ss));
      }
      HIP_OK(c, tb_tok_dw(c, t.S, t.N1, G + o.w1, G + o.b1, B, T, FF, D, scale, ss));
    }
    // combined = dRES2 + dz1 W1
    HIP_OK(c, gemm_nn(c, t.DZ1, P + o.w1, t.COMB, rows, D, FF, EPI_BIAS_ADD, 0, t.G1, 0));
  }
  // norm 1
  if (fused) {
    HIP_OK(c, norm_bwd_fused(0, t.COMB, nullptr, t.RES1, t.st1, t.G2, t.LP1, t.TS1,
                             R.d.block_act == GN_BLOCK_ACT_SWIGLU ? nullptr : t.DZ1));
    lin_job(t.TS1, np, D, t.O, D, D, o.wo, o.bo);  // wOut (Linear): dz = dRES1
  } else {
    HIP_OK(c, tb_norm_bwd(c, R, P, G, o, 0, t.COMB, t.RES1, t.st1, t.G2, rows, scale));
    HIP_OK(c, fork());
    {
      // wOut (Linear): dz = dRES1
      KTimer kt(c, GN_KCLASS_OTHER, "token_sum", token_sum_bytes(B, T, D), ss);
      HIP_OK(c, launch_token_sum(t.G2, t.S, B, T, D, ss));
    }
    HIP_OK(c, tb_tok_dw(c, t.S, t.O, G + o.wo, G + o.bo, B, T, D, D, scale, ss));
  }
  HIP_OK(c, gemm_nn(c, t.G2, P + o.wo, t.GO, rows, D, D, EPI_SCALE, 0, nullptr, 0));
  const int64_t sst = (int64_t)M->maxB * D;  // stride of the three token-sum blocks
  // the fused attention backward forms the token sums of gQ, gK, gV itself
  // (not when RoPE rotates gQ and gK after it)
  const bool attn_sums = fused && !t.SC && !R.d.use_rope;
  {
    KTimer kt(c, GN_KCLASS_OTHER, "attn_bwd", attn_flops(B, T, R.NH, D / R.NH, R.causal, true));
    if (t.SC)
      HIP_OK(c, launch_attn_bwd_gemm(t.Q, t.K, t.V, t.GO, t.GQ, t.GK, t.GV, B, T, D, R.NH, R.causal, t.SC,
                                     c->stream));
    else
      HIP_OK(c, launch_attn_bwd(t.Q, t.K, t.V, t.GO, t.GQ, t.GK, t.GV, B, T, D, R.NH, R.causal, c->stream,
                                attn_sums ? t.S3 : nullptr, sst));
  }
  if (R.d.use_rope) {  // transformer.go:660-664: conjugate rotation before wQ/wK
    KTimer kt(c, GN_KCLASS_OTHER, "rope", 2 * f4(2.0 * rows * D));
    HIP_OK(c, launch_rope(t.GQ, t.rcos, t.rsin, rows, T, R.NH, D / R.NH, 1, c->stream));
    HIP_OK(c, launch_rope(t.GK, t.rcos, t.rsin, rows, T, R.NH, D / R.NH, 1, c->stream));
  }
  const int64_t bo[3] = {o.bq, o.bk, o.bv};
  const int64_t wo3[3] = {o.wq, o.wk, o.wv};
  HIP_OK(c, fork());
  if (!attn_sums) {
    // gQ, gK, gV are one [3][max batch][T][D] block: one token-sum launch,
    // blockIdx.z picking the member, B samples each
    KTimer kt(c, GN_KCLASS_OTHER, "token_sum", 3 * token_sum_bytes(B, T, D), ss);
    HIP_OK(c, launch_token_sum_multi(t.GQ, t.S3, B, T, D, 3, t.GK - t.GQ, sst, ss));
  }
  if (fused) {
    // dWq, dWk, dWv and their biases join the jobs: every parameter gradient
    // of the block in one launch
    for (int z = 0; z < 3; ++z) lin_job(t.S3 + z * sst, 1, D, X, D, D, wo3[z], bo[z]);
    KTimer kt(c, GN_KCLASS_OTHER, "tb_params", pbytes, ss);
    HIP_OK(c, launch_tb_params(pset, B, scale, ss));
  } else {
    // dWq, dWk, dWv and their biases (Q10: token sums times the last token's
    // input, token sums summed over the batch) in one launch
    TokDwSet set{};
    for (int z = 0; z < 3; ++z) {
      set.S[z] = t.S3 + z * sst;
      set.X[z] = X + (int64_t)(T - 1) * D;
      set.dW[z] = G + wo3[z];
      set.db[z] = G + bo[z];
    }
    KTimer kt(c, GN_KCLASS_OTHER, "tok_dw", 3 * f4((double)B * D + (double)B * D + (double)D * D + D), ss);
    HIP_OK(c, launch_tok_dw(set, 3, B, D, D, D, T * D, scale, ss));
  }
  if (gin) {  // gIn = dRES1 + gQ Wq + gK Wk + gV Wv
    const int64_t pst = (int64_t)rows * D;
    hipError_t eg = hipErrorNotSupported;
    {
      // one GEMM over K = 3D in three segments (gQ | gK | gV against Wq; Wk;
      // Wv) with dRES1 added in the epilogue
      GemmArgs a{};
      a.M = rows; a.N = D; a.K = 3 * D;
      a.A = t.GQ; a.lda = D; a.B = P + o.wq; a.ldb = D;
      a.C = gin; a.ldc = D; a.alpha = 1.f;
      a.aux = t.G2; a.ldaux = D;
      a.kseg = D;
      a.seg_A = t.GK - t.GQ;
      a.seg_B = o.wk - o.wq;
      a.ws = cs; a.ws_cap = cap;
      if (gemm_segments_ok(a)) {
        KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
        eg = launch_gemm('N', 'N', EPI_BIAS_ADD, a, c->stream);
      }
    }
    if (eg == hipSuccess) {
    } else if (eg != hipErrorNotSupported) {
      HIP_OK(c, eg);
    } else if ((size_t)3 * pst <= c->scratch_floats) {
      // the three products in one batched launch into the scratch, then
      // added to dRES1 in the order of three accumulating launches
      GemmArgs a{};
      a.M = rows; a.N = D; a.K = D;
      a.A = t.GQ; a.lda = D; a.B = P + o.wq; a.ldb = D;
      a.C = c->scratch; a.ldc = D; a.alpha = 1.f;
      a.nbatch = 3;
      a.bstride_A = t.GK - t.GQ;
      a.bstride_B = o.wk - o.wq;
      a.bstride_C = pst;
      {
        KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
        HIP_OK(c, launch_gemm('N', 'N', EPI_SCALE, a, c->stream));
      }
      KTimer kt(c, GN_KCLASS_OTHER, "add3", f4(5.0 * pst));
      HIP_OK(c, launch_add3(t.G2, c->scratch, pst, gin, pst, c->stream));
    } else {
      HIP_OK(c, gemm_nn(c, t.GQ, P + o.wq, gin, rows, D, D, EPI_BIAS_ADD, 0, t.G2, 0));
      HIP_OK(c, gemm_nn(c, t.GK, P + o.wk, gin, rows, D, D, EPI_BIAS_ADD, 0, gin, 0));
      HIP_OK(c, gemm_nn(c, t.GV, P + o.wv, gin, rows, D, D, EPI_BIAS_ADD, 0, gin, 0));
    }
  }
  return GN_OK;
}

// Forward over B samples.  Returns the output pointer of the last layer.
// `for_loss`: the output layer keeps pre-activations for the row kernel.
static int model_forward(gn_model *M, const float *x, int B, bool for_loss) {
  gn_ctx *c = M->ctx;
  if (!for_loss || M->workers <= 1) M->master_dims = true;
  const float *cur = x;
  bool pe_done = false;  // the PositionalEncoding output was written with the embedding rows
  bool drop_done = false;  // the Dropout's output was written by the Dense GEMM below it
  bool pool_done = false;  // the MaxPool2D's outputs were written by the Conv2D below it
  bool cls_done = false;   // the CLSPooling's output was written by the block below it
  const int n = (int)M->L.size();
  for (int i = 0; i < n; ++i) {
    LayerRT &R = M->L[i];
    switch (R.d.kind) {
      case GN_LAYER_DENSE: {
        const float *W = M->params + R.poff;
        const float *b = W + (int64_t)R.d.in_size * R.d.out_size;
        const bool last = (i == n - 1);
        if (last && for_loss && M->tail_now) break;  // launch_tail_fwd computes z with the loss rows
        int fwd = R.ap.fwd;
        if (R.ap.jac || (last && for_loss)) fwd = F_IDENTITY;  // row kernel finishes it
        // a Dropout above in training mode: its output from the GEMM's split-K
        // reduction (dropout.go:85-130 per element, the same expression)
        LayerRT *dr = !last && !R.ap.jac && M->L[i + 1].d.kind == GN_LAYER_DROPOUT && M->eff[i + 1] &&
                              M->L[i + 1].out_len == R.out_len
                          ? &M->L[i + 1]
                          : nullptr;
        // the Dense that feeds the fused output kernels leaves its split-K
        // reduce (and epilogue, and Dropout) to them
        const bool feed = for_loss && M->tail_now && i == M->tail_src && !R.ap.jac;
        int splits = 1;
        HIP_OK(c, dense_fwd(c, cur, W, b, R.out, B, R.d.in_size, R.d.out_size, fwd,
                            dr ? dr->out : nullptr, dr ? dr->mask : nullptr, dr ? dr->scale : 0.f,
                            feed ? &splits : nullptr));
        if (feed && splits > 1) {
          TailSplitIn &sp = M->tail_sp;
          sp.ws = c->scratch;
          sp.splits = splits;
          sp.bias = b;
          sp.act = fwd;
          sp.xo = R.out;
          sp.dout = dr ? dr->out : nullptr;
          sp.mask = dr ? dr->mask : nullptr;
          sp.scale = dr ? dr->scale : 0.f;
        }
        drop_done = dr != nullptr;
        if (R.ap.jac && !(last && for_loss)) {  // the loss kernel finishes the output layer's rows
          KTimer kt(c, GN_KCLASS_OTHER, "row_act", f4(2.0 * B * R.out_len));
          HIP_OK(c, launch_row_act(R.out, B, R.out_len, R.ap.row_act, c->stream));
        }
        break;
      }
      case GN_LAYER_DROPOUT:
        if (drop_done) {
          drop_done = false;
        } else if (M->eff[i]) {
          KTimer kt(c, GN_KCLASS_OTHER, "dropout", f4(2.0 * B * R.out_len + R.out_len));
          HIP_OK(c, launch_dropout(cur, R.mask, R.scale, R.out, B, R.out_len, c->stream));
        } else
          HIP_OK(c, hipMemcpyAsync(R.out, cur, (size_t)B * R.out_len * sizeof(float),
                                   hipMemcpyDeviceToDevice, c->stream));
        break;
      case GN_LAYER_FLATTEN:
        R.out = const_cast<float *>(cur);
        break;
      case GN_LAYER_CONV2D: {
        const float *W = M->params + R.poff;
        const float *b = W + (int64_t)R.cs.outC * R.cs.inC * R.cs.k * R.cs.k;
        // a 2x2 stride-2 MaxPool2D above: its outputs and switches in the same pass
        LayerRT *pl = i + 1 < n && M->L[i + 1].d.kind == GN_LAYER_MAXPOOL2D ? &M->L[i + 1] : nullptr;
        if (pl && !conv_fwd_pool_fusable(R.cs, pl->ps, B)) pl = nullptr;
        KTimer kt(c, GN_KCLASS_OTHER, "conv_fwd", conv_flops(R.cs, B));
        HIP_OK(c, launch_conv_fwd(cur, W, b, R.out, R.cs, B, R.cfwd, c->stream, pl ? pl->out : nullptr,
                                  pl ? pl->argmax : nullptr));
        pool_done = pl != nullptr;
        break;
      }
      case GN_LAYER_MAXPOOL2D: {  // read the input, write outputs and int32 switches
        if (pool_done) {
          pool_done = false;
          break;
        }
        KTimer kt(c, GN_KCLASS_OTHER, "maxpool_fwd", f4((double)B * R.in_len + 2.0 * B * R.out_len));
        HIP_OK(c, launch_maxpool_fwd(cur, R.out, R.argmax, R.ps, B, c->stream));
        break;
      }
      case GN_LAYER_AVGPOOL2D: {
        KTimer kt(c, GN_KCLASS_OTHER, "avgpool_fwd", f4((double)B * R.in_len + (double)B * R.out_len));
        HIP_OK(c, launch_avgpool_fwd(cur, R.out, R.ps, B, c->stream));
        break;
      }
      case GN_LAYER_EMBEDDING: {  // read the ids and their rows, write rows and int32 ids
        LayerRT *pe = i + 1 < n ? &M->L[i + 1] : nullptr;
        if (pe && pe->d.kind == GN_LAYER_POSENC && pe->T == R.T && pe->D == R.D) {
          // and the PositionalEncoding output in the same pass
          KTimer kt(c, GN_KCLASS_OTHER, "embed_pe_fwd",
                    f4(2.0 * B * R.T + 3.0 * B * R.T * R.D + (double)R.T * R.D));
          HIP_OK(c, launch_embed_pe(cur, M->params + R.poff, M->params + pe->poff, R.ids, R.out, pe->out, B,
                                    R.T, R.V, R.D, M->L[M->emb].bad, c->stream, i != M->emb));
          pe_done = true;
          break;
        }
        KTimer kt(c, GN_KCLASS_OTHER, "embed_fwd", f4(2.0 * B * R.T + 2.0 * B * R.T * R.D));
        HIP_OK(c, launch_embed(cur, M->params + R.poff, R.ids, R.out, B, R.T, R.V, R.D, M->L[M->emb].bad,
                               c->stream, i != M->emb));
        break;
      }
      case GN_LAYER_POSENC: {
        if (pe_done) {  // written with the embedding rows
          pe_done = false;
          break;
        }
        KTimer kt(c, GN_KCLASS_OTHER, "pe_add", f4(2.0 * B * R.T * R.D + (double)R.T * R.D));
        HIP_OK(c, launch_pe_add(cur, M->params + R.poff, R.out, B, R.T * R.D, c->stream));
        break;
      }
      case GN_LAYER_CLSPOOL: {
        if (cls_done) {
          cls_done = false;
          break;
        }
        KTimer kt(c, GN_KCLASS_OTHER, "cls_fwd", f4(2.0 * B * R.D));
        HIP_OK(c, launch_cls_fwd(cur, R.out, B, R.T * R.D, R.D, c->stream));
        break;
      }
      case GN_LAYER_TRANSFORMER: {
        // a CLSPooling above gets token 0 of each sample from the block's last norm
        LayerRT *up = i + 1 < n ? &M->L[i + 1] : nullptr;
        float *cls = nullptr;
        if (up && tb_cls_fusable(R, *up)) {
          cls = up->out;
          cls_done = true;
        }
        int r = tb_forward(M, R, cur, B, cls);
        if (r) return r;
        break;
      }
      case GN_LAYER_MHA: {
        int r = mha_forward_impl(c, cur, M->params + R.poff, R.out, mha_bufs(M, R), B, R.T, R.D, R.NH,
                                 R.causal, R.d.use_rope);
        if (r) return r;
        break;
      }
      case GN_LAYER_LAYERNORM: {
        const int rows = B * (R.in_len / R.D);
        KTimer kt(c, GN_KCLASS_OTHER, "ln_fwd", f4(2.0 * rows * R.D + 2.0 * rows));
        HIP_OK(c, launch_ln_fwd(cur, M->params + R.poff, M->params + R.poff + R.D, R.out, R.rmsv, rows, R.D,
                                R.eps, c->stream));
        break;
      }
      case GN_LAYER_GAP1D: {
        KTimer kt(c, GN_KCLASS_OTHER, "gap1d_fwd", f4((double)B * R.T * R.D + (double)B * R.D));
        HIP_OK(c, launch_gap1d_fwd(cur, R.out, B, R.T, R.D, c->stream));
        break;
      }
      case GN_LAYER_SWIGLU: {
        const int out2 = 2 * R.d.out_size;
        {
          KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", 2.0 * B * out2 * R.d.in_size);
          GemmArgs g{};  // Z[b] = [W x_b | V x_b]
          g.M = B; g.N = out2; g.K = R.d.in_size;
          g.A = cur; g.lda = R.d.in_size;
          g.B = M->params + R.poff; g.ldb = R.d.in_size;
          g.C = R.zbuf; g.ldc = out2; g.alpha = 1.0f;
          g.ws = c->scratch; g.ws_cap = c->scratch_floats;
          HIP_OK(c, launch_gemm('N', 'T', EPI_SCALE, g, c->stream));
        }
        KTimer kt(c, GN_KCLASS_OTHER, "swiglu_fwd", f4(3.0 * B * R.d.out_size));
        HIP_OK(c, launch_swiglu_fwd(R.zbuf, R.out, B, R.d.out_size, c->stream));
        break;
      }
      case GN_LAYER_MOE: {
        const int I = R.d.in_size, O = R.d.out_size, E = R.E, K = R.K;
        const float *P = M->params + R.poff;
        const int64_t e1 = (int64_t)O * I + O;
        HIP_OK(c, gemm_nt(c, cur, P, P + (int64_t)E * I, R.mlog, B, E, I, EPI_BIAS_ACT, F_IDENTITY,
                          nullptr));
        MoeRoute rt{};
        rt.B = B; rt.E = E; rt.K = K; rt.training = M->eff[i];
        const int W = std::min(M->workers, B);
        if (M->workers > 1) rt.chunk = (B + W - 1) / W;  // trainBatchParallel chunks
        for (int k = 0; k < 65; ++k) rt.base[k] = R.mrng[k];
        {
          KTimer kt(c, GN_KCLASS_OTHER, "moe_route", f4(2.0 * B * E + (double)B * K));
          HIP_OK(c, launch_moe_route(R.mlog, R.mprob, R.mact, rt, c->stream));
        }
        for (int e = 0; e < E; ++e) {  // every expert on every sample; the route picks k of them
          const float *We = P + (int64_t)E * I + E + e * e1;
          HIP_OK(c, gemm_nt(c, cur, We, We + (int64_t)O * I, R.meout + (int64_t)e * B * O, B, O, I,
                            EPI_BIAS_ACT, F_LEAKY, nullptr));
        }
        KTimer kt(c, GN_KCLASS_OTHER, "moe_combine", f4((double)K * B * O + (double)B * O));
        HIP_OK(c, launch_moe_combine(R.meout, R.mprob, R.mact, R.out, B, O, E, K, c->stream));
        if (M->eff[i]) {  // E draws per sample on its stream
          if (M->workers > 1) {
            for (int w = 0; w < W; ++w) {
              const int n = std::max(0, std::min(rt.chunk, B - w * rt.chunk));
              for (int64_t d = 0; d < (int64_t)n * E; ++d) R.mrng[1 + w] = R.mrng[1 + w] * 6364136223846793005ull + 1;
            }
          } else {
            for (int64_t d = 0; d < (int64_t)B * E; ++d) R.mrng[0] = R.mrng[0] * 6364136223846793005ull + 1;
          }
        }
        break;
      }
      case GN_LAYER_GRU_UNROLLER: {
        const int H = R.H, G3 = 3 * H;
        const float *Wx = M->params + R.poff;
        const float *Wh = Wx + (int64_t)G3 * R.I;
        const float *bias = Wh + (int64_t)2 * H * H;
        {
          KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", 2.0 * B * R.T * G3 * R.I);
          GemmArgs g{};  // xw[b*T + t] = b + Wx x_t (gru.go:194-210)
          g.M = B * R.T; g.N = G3; g.K = R.I;
          g.A = cur; g.lda = R.I;
          g.B = Wx; g.ldb = R.I;
          g.C = R.xw; g.ldc = G3; g.alpha = 1.0f;
          g.bias = bias; g.act = F_IDENTITY;
          g.ws = c->scratch; g.ws_cap = c->scratch_floats;
          HIP_OK(c, launch_gemm('N', 'T', EPI_BIAS_ACT, g, c->stream));
        }
        {
          KTimer kt(c, GN_KCLASS_OTHER, "transpose", f4(4.0 * H * H));
          HIP_OK(c, launch_transpose(Wh, R.WhT, 2 * H, H, c->stream));
        }
        // recurrence: the hidden-state products 2 x 3H x H per sample and step
        KTimer kt(c, GN_KCLASS_OTHER, "gru_fwd", 2.0 * 3 * H * H * B * R.T);
        HIP_OK(c, launch_gru_fwd(R.xw, R.WhT, R.gpre, R.ghprev, R.grh, R.out, B, R.T, H, c->stream,
                                 R.d.return_sequences ? 1 : 0));
        break;
      }
      case GN_LAYER_BATCHNORM2D: {  // running stats advance in training mode only
        KTimer kt(c, GN_KCLASS_OTHER, "bn_fwd", f4(2.0 * B * R.in_len + 3.0 * B * R.C));
        HIP_OK(c, launch_bn_fwd(cur, R.pcount ? M->params + R.poff : nullptr, R.out, R.bnst, R.rmean,
                                R.rvar, B, R.C, R.HW, R.eps, R.d.momentum, M->eff[i], c->stream));
        break;
      }
      case GN_LAYER_RMSNORM: {
        KTimer kt(c, GN_KCLASS_OTHER, "rms_fwd", f4(2.0 * B * R.in_len + (double)B * (R.in_len / R.D)));
        HIP_OK(c, launch_rms_fwd(cur, M->params + R.poff, R.out, R.rmsv, B * (R.in_len / R.D), R.D,
                                 R.eps, c->stream));
        break;
      }
      case GN_LAYER_LSTM_UNROLLER: {
        const float *Wx = M->params + R.poff;
        const float *Wh = Wx + (int64_t)4 * R.H * R.I;
        const float *bias = Wh + (int64_t)4 * R.H * R.H;
        {
          KTimer kt(c, GN_KCLASS_GEMM, "gemm_fwd", 2.0 * B * R.T * R.H * R.I);
          GemmArgs g{};  // xw[b*T + t][i] = x[b, t, :] . Wx[i, :] (input-gate rows, Q13)
          g.M = B * R.T; g.N = R.H; g.K = R.I;
          g.A = cur; g.lda = R.I;
          g.B = Wx; g.ldb = R.I;
          g.C = R.xw; g.ldc = R.H; g.alpha = 1.0f;
          g.ws = c->scratch; g.ws_cap = c->scratch_floats;
          HIP_OK(c, launch_gemm('N', 'T', EPI_SCALE, g, c->stream));
        }
        {
          KTimer kt(c, GN_KCLASS_OTHER, "transpose", f4(2.0 * R.H * R.H));
          HIP_OK(c, launch_transpose(Wh, R.WhT, R.H, R.H, c->stream));
        }
        // recurrence: Q13 leaves only the input gate with Wh h, 2 x H x H per sample and step
        KTimer kt(c, GN_KCLASS_OTHER, "lstm_fwd", 2.0 * R.H * R.H * B * R.T);
        HIP_OK(c, launch_lstm_fwd(R.xw, R.WhT, bias, R.igb, R.tcb, R.cbuf, R.hbuf, R.out, B, R.T,
                                  R.H, c->stream, R.d.return_sequences ? 1 : 0));
        break;
      }
      default:
        return set_err(c, GN_ERR_UNSUPPORTED, "layer kind %d", R.d.kind);
    }
    cur = R.out;
  }
  return GN_OK;
}

// Backward over B samples.  The output layer's dz is in L.back().gout.
// With `ac`, each layer's parameters get their Adam update on ctx->aux once
// the layer's backward kernels are queued (no later kernel of the backward
// reads them), and the main stream waits for all updates at the end.
// products (multiply-adds) up to which the fused output-layer kernels take a
// Dense layer's GEMM work
constexpr double kTailMaxMacs = 16.0 * (1 << 20);

static int model_backward(gn_model *M, const float *x, int B, float scale, const AdamCoef *ac) {
  gn_ctx *c = M->ctx;
  const int n = (int)M->L.size();
  // parameter gradients on ctx->aux beside the input-gradient chain (the
  // per-kernel timing pass keeps one stream, so each kernel is timed alone)
  const bool side = !c->timing && (ac || M->side_ok);
  auto grow = [&](std::vector<hipEvent_t> &v, int want) -> int {
    while ((int)v.size() < want) {
      hipEvent_t e;
      HIP_OK(c, hipEventCreateWithFlags(&e, hipEventDisableTiming));
      v.push_back(e);
    }
    return GN_OK;
  };
  if (ac && grow(M->sync_ev, n + 1)) return GN_ERR_HIP;
  if (side && (grow(M->dz_ev, n) || grow(M->dw_ev, n))) return GN_ERR_HIP;
  if (side && !M->fork_ev) HIP_OK(c, hipEventCreateWithFlags(&M->fork_ev, hipEventDisableTiming));
  if (side && !M->join_ev) HIP_OK(c, hipEventCreateWithFlags(&M->join_ev, hipEventDisableTiming));
  bool aux_used = false;
  if (ac && !M->adam_s)  // default priority, like the context's streams
    HIP_OK(c, hipStreamCreateWithFlags(&M->adam_s, hipStreamNonBlocking));
  std::vector<char> dw_aux(n, 0);  // layer i's dW went to ctx->aux
  bool is_dz = true;  // gout of the current layer already holds dz
  bool drop_done = false;  // the Dropout below was folded into the Dense above's dX epilogue
  int bias_done = -1;      // a Dense layer whose bias gradient launch_tail_bwd wrote
  int dw_done = -1;        // ... and whose weight gradient it wrote
  int pool_bwd_done = -1;  // a MaxPool2D whose input gradient launch_tail_bwd wrote
  const float *cls_gpool = nullptr;  // a CLSPooling's gradient left for the block below
  float *pe_grad = nullptr;  // a PositionalEncoding's gradient left for the Embedding below
  for (int i = n - 1; i >= 0; --i) {
    LayerRT &R = M->L[i];
    const float *in = i == 0 ? x : M->L[i - 1].out;
    LayerRT *below = i > 0 ? &M->L[i - 1] : nullptr;
    // Layers below that are Flatten alias their gout to ours.
    switch (R.d.kind) {
      case GN_LAYER_DENSE: {
        const float *W = M->params + R.poff;
        float *gW = M->grads + R.poff;
        float *gB = gW + (int64_t)R.d.in_size * R.d.out_size;
        float *dz = R.gout;
        if (!is_dz && R.ap.jac) {  // a hidden Softmax / LogSoftmax: the row Jacobian (layer.go:504-560)
          KTimer kt(c, GN_KCLASS_OTHER, "row_jac", f4(3.0 * B * R.out_len));
          HIP_OK(c, launch_row_jac(R.gout, R.out, dz, B, R.out_len, R.ap.row_act, c->stream));
        } else if (!is_dz) {  // read the gradient and the saved output, write dz
          KTimer kt(c, GN_KCLASS_OTHER, "dact", f4(3.0 * B * R.out_len));
          HIP_OK(c, launch_dact(R.gout, R.out, dz, (int64_t)B * R.out_len, R.ap.deriv, c->stream));
        }
        float *gin = nullptr;
        const float *aux = nullptr, *cfac = nullptr;
        int deriv = 0;
        bool next_dz = false;
        if (below) {
          gin = below->gout;  // Flatten's gout aliases the buffer of the layer under it
          LayerRT *b2 = i >= 2 ? &M->L[i - 2] : nullptr;
          if (below->d.kind == GN_LAYER_DENSE && !below->ap.jac) {
            aux = below->out;  // fuse act' of the layer below into the dX epilogue
            deriv = below->ap.deriv;
            next_dz = true;
          } else if (below->d.kind == GN_LAYER_DROPOUT && M->eff[i - 1] && b2 &&
                     b2->d.kind == GN_LAYER_DENSE && !b2->ap.jac && b2->gout) {
            // Dense <- Dropout (training) <- Dense: the dropout factor and the
            // lower layer's act' in the dX epilogue, straight into its dz
            gin = b2->gout;
            aux = b2->out;
            deriv = b2->ap.deriv;
            cfac = below->dfac;
            next_dz = true;
            drop_done = true;
          }
        }
        // with the per-layer Adam on aux (large models), dW and db run there
        // next to dX; the layer's Adam is queued behind them.  The per-kernel
        // timing pass keeps them on one stream, so each GEMM is timed alone.
        if (i == n - 1 && M->tail_now) {
          // every gradient of the output layer in one kernel, and the bias
          // gradient of the Dense whose dz its dX is
          LayerRT *dn = next_dz ? (gin == below->gout ? below : &M->L[i - 2]) : nullptr;
          float *gb_below = dn ? M->grads + dn->poff + (int64_t)dn->d.in_size * dn->d.out_size : nullptr;
          const int C = R.d.out_size, nin = R.d.in_size;
          // Flatten over a 2x2 stride-2 MaxPool2D whose windows tile its
          // input: the pool's backward through its switches in the same pass
          LayerRT *pl = i >= 3 && below->d.kind == GN_LAYER_FLATTEN && M->L[i - 2].d.kind == GN_LAYER_MAXPOOL2D
                            ? &M->L[i - 2]
                            : nullptr;
          if (pl) {
            const PoolShape &q = pl->ps;
            const bool tiled = q.k == 2 && q.stride == 2 && q.pad == 0 && q.H % 2 == 0 && q.W % 2 == 0 &&
                               q.oH == q.H / 2 && q.oW == q.W / 2 && q.C * q.oH * q.oW == nin;
            if (!tiled || !M->L[i - 3].gout || aux || cfac || next_dz) pl = nullptr;
          }
          // the weight gradient of that Dense too, when it is small enough
          // that its GEMM's launch, not its work, would set its time
          const int dni = dn ? (int)(dn - &M->L[0]) : -1;
          const bool dwb = dn && (double)B * dn->d.in_size * dn->d.out_size <= kTailMaxMacs;
          const float *xdn = dni > 0 ? M->L[dni - 1].out : x;
          KTimer kt(c, GN_KCLASS_OTHER, "tail_bwd",
                    f4(2.0 * B * nin + 2.0 * C * nin + B * C + C + (gin ? (aux ? 2.0 : 1.0) * B * nin : 0.0) +
                       (gb_below ? nin : 0) + (pl ? 4.0 * B * nin : 0.0) +
                       (dwb ? (double)B * dn->d.in_size + (double)dn->d.in_size * dn->d.out_size : 0.0)));
          HIP_OK(c, launch_tail_bwd(in, W, dz, gW, gB, gin, aux, deriv, cfac, gb_below, B, nin, C, scale,
                                    c->stream, pl ? pl->argmax : nullptr, pl ? M->L[i - 3].gout : nullptr,
                                    pl ? pl->ps.H : 0, pl ? pl->ps.W : 0, dwb ? xdn : nullptr,
                                    dwb ? M->grads + dn->poff : nullptr, dwb ? dn->d.in_size : 0));
          dw_done = dwb ? dni : -1;
          pool_bwd_done = pl ? i - 2 : -1;
          bias_done = dn ? (int)(dn - &M->L[0]) : -1;
          is_dz = next_dz;
          break;
        }
        if (i == dw_done && i == bias_done && !gin) {  // every gradient of the layer is written
          is_dz = next_dz;
          break;
        }
        const bool sd = side && gin && i != dw_done;
        HIP_OK(c, dense_bwd_core(c, in, W, dz, gW, i == bias_done ? nullptr : gB, gin, B, R.d.in_size,
                                 R.d.out_size, scale, aux, deriv, sd ? M->dz_ev[i] : nullptr, nullptr, 0,
                                 cfac, i == dw_done, !ac));
        if (sd) {  // the layer's Adam (M->adam_s) waits for its dW and bias sums
          HIP_OK(c, hipEventRecord(M->dw_ev[i], c->aux));
          dw_aux[i] = 1;
          aux_used = true;
        }
        is_dz = next_dz;
        break;
      }
      case GN_LAYER_DROPOUT: {
        if (drop_done) {  // applied by the dX epilogue of the Dense above
          drop_done = false;
          break;
        }
        // dropout.go:283-290 in training mode; out of it the gradient passes
        // unchanged (dropout.go:241-247)
        // (a Flatten first in the network has no gradient buffer: nothing below needs one)
        if (below && below->gout && M->eff[i]) {
          KTimer kt(c, GN_KCLASS_OTHER, "dropout", f4(2.0 * B * R.out_len + R.out_len));
          HIP_OK(c, launch_dropout(R.gout, R.mask, R.scale, below->gout, B, R.out_len, c->stream));
        } else if (below && below->gout)
          HIP_OK(c, hipMemcpyAsync(below->gout, R.gout, (size_t)B * R.out_len * sizeof(float),
                                   hipMemcpyDeviceToDevice, c->stream));
        is_dz = false;
        break;
      }
      case GN_LAYER_FLATTEN:
        break;  // gout aliased by the layer above
      case GN_LAYER_MAXPOOL2D:
        if (i == pool_bwd_done) {
          is_dz = false;
          break;
        }
        if (below && below->gout) {  // read gradients and switches, write the input gradient
          KTimer kt(c, GN_KCLASS_OTHER, "maxpool_bwd", f4(2.0 * B * R.out_len + (double)B * R.in_len));
          HIP_OK(c, launch_maxpool_bwd(R.gout, R.argmax, below->gout, R.ps, B, c->stream));
        }
        is_dz = false;
        break;
      case GN_LAYER_AVGPOOL2D:  // avgpool2d.go:401-474
        if (below && below->gout) {
          KTimer kt(c, GN_KCLASS_OTHER, "avgpool_bwd", f4((double)B * R.out_len + (double)B * R.in_len));
          HIP_OK(c, launch_avgpool_bwd(R.gout, below->gout, R.ps, B, c->stream));
        }
        is_dz = false;
        break;
      case GN_LAYER_CONV2D: {
        // Conv2D.Backward (conv2d.go:1117-1168): the layer's own Derivative
        // is applied to gout here, so it never receives a fused dz.
        if (is_dz && i != n - 1) return set_err(c, GN_ERR_UNSUPPORTED, "fused dz into Conv2D");
        const float *W = M->params + R.poff;
        {  // dW and db: the taps plus the all-ones column
          // the first layer's reduction is the backward's last launch: with
          // the step's update it is left out, and carries the update of every
          // other layer in extra blocks
          ConvWgradReduce red{};
          const bool defer = M->upd_want && !below;
          {
            KTimer kt(c, GN_KCLASS_OTHER, "conv_wgrad",
                      conv_flops(R.cs, B) + 2.0 * B * R.cs.outC * R.cs.oH * R.cs.oW);
            HIP_OK(c, launch_conv_wgrad(in, R.gout, R.out, M->grads + R.poff, R.cs, B, R.cderiv, scale,
                                        c->scratch, c->scratch_floats, c->stream, defer ? &red : nullptr));
          }
          if (defer) {
            hipStream_t st = c->stream;
            float *rest = M->grads;
            const int64_t c0 = R.poff, c1 = R.poff + red.nslots, np = M->nparams;
            M->upd_fn = [=](const AdamStep &a) {
              AdamStep u = a;
              u.rest = rest;
              u.r0[0] = 0;
              u.r1[0] = c0;
              u.r0[1] = c1;
              u.r1[1] = np;
              return launch_conv_wgrad_reduce(red, &u, st);
            };
            M->upd_name = "wgrad_reduce_adam";
            M->upd_units = 4.0 * ((double)red.nblocks * red.nslots + red.nslots) + 28.0 * M->nparams;
          }
        }
        if (below && below->gout) {
          KTimer kt(c, GN_KCLASS_OTHER, "conv_dgrad", conv_flops(R.cs, B));
          HIP_OK(c, launch_conv_dgrad(R.gout, R.out, W, below->gout, R.cs, B, R.cderiv, c->stream));
        }
        is_dz = false;
        break;
      }
      case GN_LAYER_CLSPOOL:
        if (below && tb_cls_fusable(*below, R)) {
          cls_gpool = R.gout;  // the block's norm-2 backward reads it
        } else if (below && below->gout) {  // transformer.go:1714-1723: row 0 gets g, the rest 0
          KTimer kt(c, GN_KCLASS_OTHER, "cls_bwd", f4((double)B * R.D + (double)B * R.T * R.D));
          HIP_OK(c, launch_cls_bwd(R.gout, below->gout, B, R.T * R.D, R.D, c->stream));
        }
        is_dz = false;
        break;
      case GN_LAYER_TRANSFORMER: {
        const float *gpool = cls_gpool;
        cls_gpool = nullptr;
        int r = tb_backward(M, R, in, below ? below->gout : nullptr, B, scale, side ? c->aux : nullptr,
                            gpool);
        if (r) return r;
        if (side) {  // the layer's Adam (M->adam_s) waits for its weight gradients
          HIP_OK(c, hipEventRecord(M->dw_ev[i], c->aux));
          dw_aux[i] = 1;
          aux_used = true;
        }
        is_dz = false;
        break;
      }
      case GN_LAYER_MHA: {
        int r = mha_backward_impl(c, in, M->params + R.poff, R.gout, M->grads + R.poff,
                                  below ? below->gout : nullptr, mha_bufs(M, R), B, R.T, R.D, R.NH, R.causal,
                                  R.d.use_rope, scale);
        if (r) return r;
        is_dz = false;
        break;
      }
      case GN_LAYER_LAYERNORM: {  // layernorm.go:334-441 (Q18), gamma / beta sums over the rows
        const int rows = B * (R.in_len / R.D), N = R.D;
        const float *gam = M->params + R.poff;
        float *dg = M->grads + R.poff, *db = dg + N;
        float *dx = below && below->gout ? below->gout : R.zbuf;
        hipError_t e;
        {
          KTimer kt(c, GN_KCLASS_OTHER, "ln_bwd", f4(3.0 * rows * N + 2.0 * rows + 2.0 * N));
          e = launch_ln_bwd_params(R.gout, in, gam, R.rmsv, dx, dg, db, rows, N, scale, c->scratch,
                                   c->scratch_floats, c->stream);
        }
        if (e == hipErrorNotSupported) {  // partials beyond the scratch: g * xhat, then column sums
          (void)hipGetLastError();
          {
            KTimer kt(c, GN_KCLASS_OTHER, "ln_bwd", f4(4.0 * rows * N + 2.0 * rows));
            HIP_OK(c, launch_ln_bwd(R.gout, in, gam, R.rmsv, dx, R.gx, rows, N, c->stream));
          }
          const float *src[2] = {R.gx, R.gout};
          float *dst[2] = {dg, db};
          KTimer kt(c, GN_KCLASS_OTHER, "colsum", 2 * f4((double)rows * N + N));
          HIP_OK(c, launch_colsum_multi(src, dst, 2, rows, N, N, scale, c->scratch, c->scratch_floats,
                                        c->stream));
        } else {
          HIP_OK(c, e);
        }
        is_dz = false;
        break;
      }
      case GN_LAYER_GAP1D:
        if (below && below->gout) {
          KTimer kt(c, GN_KCLASS_OTHER, "gap1d_bwd", f4((double)B * R.D + (double)B * R.T * R.D));
          HIP_OK(c, launch_gap1d_bwd(R.gout, below->gout, B, R.T, R.D, c->stream));
        }
        is_dz = false;
        break;
      case GN_LAYER_SWIGLU: {  // swiglu.go:196-232
        {
          KTimer kt(c, GN_KCLASS_OTHER, "swiglu_bwd", f4(5.0 * B * R.d.out_size));
          HIP_OK(c, launch_swiglu_bwd(R.gout, R.zbuf, 2 * R.d.out_size, R.dzbuf, B, R.d.out_size,
                                      c->stream));
        }
        float *gin = nullptr;
        const float *aux = nullptr;
        int deriv = 0;
        bool next_dz = false;
        if (below) {
          gin = below->gout;
          if (below->d.kind == GN_LAYER_DENSE && !below->ap.jac) {
            aux = below->out;  // act' of the Dense below fused into the dX epilogue
            deriv = below->ap.deriv;
            next_dz = true;
          }
        }
        HIP_OK(c, dense_bwd_core(c, in, M->params + R.poff, R.dzbuf, M->grads + R.poff, nullptr, gin,
                                 B, R.d.in_size, 2 * R.d.out_size, scale, aux, deriv));
        is_dz = next_dz;
        break;
      }
      case GN_LAYER_MOE: {  // moe.go:242-313
        const int I = R.d.in_size, O = R.d.out_size, E = R.E, K = R.K;
        const float *P = M->params + R.poff;
        float *G = M->grads + R.poff;
        const int64_t e1 = (int64_t)O * I + O;
        {
          KTimer kt(c, GN_KCLASS_OTHER, "moe_deltas", f4(2.0 * K * B * O + 3.0 * B * E));
          HIP_OK(c, launch_moe_backward_deltas(R.gout, R.meout, R.mprob, R.mact, R.medz, R.mdzg, B, O, E,
                                               K, M->eff[i], c->stream));
        }
        // gating and expert Dense backward: W grads = scale dz^T x, b grads = scale colsum(dz)
        HIP_OK(c, dense_bwd_core(c, in, P, R.mdzg, G, G + (int64_t)E * I, nullptr, B, I, E, scale,
                                 nullptr, 0));
        for (int e = 0; e < E; ++e) {
          float *gW = G + (int64_t)E * I + E + e * e1;
          HIP_OK(c, dense_bwd_core(c, in, nullptr, R.medz + (int64_t)e * B * O, gW, gW + (int64_t)O * I,
                                   nullptr, B, I, O, scale, nullptr, 0));
        }
        if (below && below->gout) {  // dx = dz_gate Wg + sum_e dz_e W_e
          float *gin = below->gout;
          HIP_OK(c, gemm_nn(c, R.mdzg, P, gin, B, I, E, EPI_SCALE, 0, nullptr, 0));
          for (int e = 0; e < E; ++e)
            HIP_OK(c, gemm_nn(c, R.medz + (int64_t)e * B * O, P + (int64_t)E * I + E + e * e1, gin, B, I,
                              O, EPI_BIAS_ADD, 0, gin, 0));
        }
        is_dz = false;
        break;
      }
      case GN_LAYER_GRU_UNROLLER: {  // gru.go:347-510 per step, unroller.go:189-206
        const int H = R.H, T = R.T, I = R.I, G3 = 3 * H;
        const float *Wx = M->params + R.poff;
        const float *Wh = Wx + (int64_t)G3 * I;
        float *gWx = M->grads + R.poff, *gWh = gWx + (int64_t)G3 * I, *gb = gWh + (int64_t)2 * H * H;
        {  // the recursion: Wh products 2 x 2H x H per sample and step
          KTimer kt(c, GN_KCLASS_OTHER, "gru_bwd", 2.0 * 2 * H * H * B * T);
          HIP_OK(c, launch_gru_bwd(R.gout, R.gpre, R.ghprev, Wh, R.Dg, B, T, H, c->stream,
                                   R.d.return_sequences ? 1 : 0));
        }
        if (below && below->gout) {  // dx_t = Wx^T [dU | dR (never set, 0) | dC] (gru.go:481-500)
          GemmArgs a{};
          a.M = B * T; a.N = I; a.K = G3;
          a.A = R.Dg; a.lda = G3; a.B = Wx; a.ldb = I;
          a.C = below->gout; a.ldc = I; a.alpha = 1.f;
          a.ws = c->scratch; a.ws_cap = c->scratch_floats;
          KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
          HIP_OK(c, launch_gemm('N', 'N', EPI_SCALE, a, c->stream));
        }
        {
          KTimer kt(c, GN_KCLASS_OTHER, "token_sum", token_sum_bytes(B, T, G3));
          HIP_OK(c, launch_token_sum(R.Dg, R.S, B, T, G3, c->stream));
        }
        {
          KTimer kt(c, GN_KCLASS_OTHER, "colsum", f4((double)B * G3 + G3));
          HIP_OK(c, launch_colsum(R.S, B, G3, G3, scale, gb, c->scratch, c->scratch_floats, c->stream));
        }
        KTimer kt(c, GN_KCLASS_GEMM, "gemm_dw",
                  2.0 * G3 * I * B + 2 * 2.0 * H * H * B * T);
        GemmArgs a{};  // dWx = scale * (sum_t dG)^T x_last (inputBuf holds the last step's input)
        a.M = G3; a.N = I; a.K = B;
        a.A = R.S; a.lda = G3;
        a.B = in + (int64_t)(T - 1) * I; a.ldb = T * I;
        a.C = gWx; a.ldc = I; a.alpha = scale;
        a.ws = c->scratch; a.ws_cap = c->scratch_floats;
        HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, a, c->stream));
        GemmArgs u{};  // dWh_u = scale * dU^T h_prev over (sample, step)
        u.M = H; u.N = H; u.K = B * T;
        u.A = R.Dg; u.lda = G3;
        u.B = R.ghprev; u.ldb = H;
        u.C = gWh; u.ldc = H; u.alpha = scale;
        u.ws = c->scratch; u.ws_cap = c->scratch_floats;
        HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, u, c->stream));
        GemmArgs r{};  // dWh_r = scale * dC^T (r * h_prev): the candidate's use of the reset block
        r.M = H; r.N = H; r.K = B * T;
        r.A = R.Dg + 2 * H; r.lda = G3;
        r.B = R.grh; r.ldb = H;
        r.C = gWh + (int64_t)H * H; r.ldc = H; r.alpha = scale;
        r.ws = c->scratch; r.ws_cap = c->scratch_floats;
        HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, r, c->stream));
        is_dz = false;
        break;
      }
      case GN_LAYER_BATCHNORM2D: {  // batchnorm2d.go:611-660
        KTimer kt(c, GN_KCLASS_OTHER, "bn_bwd", f4(3.0 * B * R.in_len + 2.0 * B * R.C));
        const float *gb = R.pcount ? M->params + R.poff : nullptr;
        if (!M->eff[i]) {  // inference-mode backward (batchnorm2d.go:525-551): no parameter gradient
          if (R.pcount) HIP_OK(c, launch_fill(M->grads + R.poff, 0.0f, R.pcount, c->stream));
          HIP_OK(c, launch_bn_bwd_eval(R.gout, gb, R.rvar, below ? below->gout : nullptr, B, R.C, R.HW,
                                       R.eps, c->stream));
          is_dz = false;
          break;
        }
        HIP_OK(c, launch_bn_bwd(R.gout, in, gb, R.bnst, below ? below->gout : nullptr,
                                R.pcount ? R.bnpart : nullptr, B, R.C, R.HW, c->stream));
        if (R.pcount) {
          float *G = M->grads + R.poff;
          HIP_OK(c, launch_colsum(R.bnpart, B, R.C, R.C, scale, G, c->scratch, c->scratch_floats,
                                  c->stream));
          HIP_OK(c, launch_colsum(R.bnpart + (int64_t)B * R.C, B, R.C, R.C, scale, G + R.C, c->scratch,
                                  c->scratch_floats, c->stream));
        }
        is_dz = false;
        break;
      }
      case GN_LAYER_RMSNORM: {  // rmsnorm.go:301-329: dx, then gamma += g * (x / rms)
        KTimer kt(c, GN_KCLASS_OTHER, "rms_bwd", f4(5.0 * B * R.in_len));
        const int rows = B * (R.in_len / R.D);
        HIP_OK(c, launch_rms_bwd(R.gout, in, M->params + R.poff, R.rmsv, below ? below->gout : nullptr,
                                 R.gx, rows, R.D, c->stream));
        HIP_OK(c, launch_colsum(R.gx, rows, R.D, R.D, scale, M->grads + R.poff, c->scratch,
                                c->scratch_floats, c->stream));
        is_dz = false;
        break;
      }
      case GN_LAYER_POSENC: {  // gradW += g (transformer.go:112-118), summed over samples
        if (below && below->d.kind == GN_LAYER_EMBEDDING && below->T == R.T && below->D == R.D &&
            embed_grad_takes_pe(B, R.T, M->workers)) {
          pe_grad = M->grads + R.poff;  // summed by the Embedding's gradient launch
          is_dz = false;
          break;
        }
        KTimer kt(c, GN_KCLASS_OTHER, "colsum", f4((double)B * R.T * R.D + (double)R.T * R.D));
        HIP_OK(c, launch_colsum(R.gout, B, R.T * R.D, R.T * R.D, scale, M->grads + R.poff,
                                c->scratch, c->scratch_floats, c->stream));
        is_dz = false;
        break;
      }
      case GN_LAYER_EMBEDDING: {  // Q12: last sample of each worker chunk only
        // fill of the gradient table, then the contributing rows (one sample per chunk)
        const int Wc = std::max(1, std::min(M->workers, B));
        const int nch = (B + (B + Wc - 1) / Wc - 1) / ((B + Wc - 1) / Wc);
        float *peg = pe_grad;
        pe_grad = nullptr;
        const double units = f4((double)R.V * R.D + 2.0 * nch * R.T * R.D +
                                (peg ? (double)B * R.T * R.D + (double)R.T * R.D : 0.0));
        if ((size_t)2 * nch * R.T > c->scratch_floats)
          return set_err(c, GN_ERR_UNSUPPORTED, "embedding backward: %d contributing rows exceed the scratch",
                         nch * R.T);
        // a first Embedding's gradient launch is the backward's last: with
        // the step's update it is left out and carries the update (its own
        // rows and the PositionalEncoding's inline, every other layer in
        // extra blocks over at most two float4-aligned ranges)
        int64_t rr0[2] = {0, 0}, rr1[2] = {0, 0};
        bool defer = M->upd_want && !below &&
                     embed_grad_upd_ok(B, R.T, R.D, M->workers, M->grads + R.poff, M->grads, M->region);
        if (defer) {
          int64_t lo = R.poff, hi = R.poff + (int64_t)R.V * R.D;  // covered inline
          if (peg) {
            const int64_t p0 = peg - M->grads, p1 = p0 + (int64_t)R.T * R.D;
            if (p0 == hi) hi = p1;
            else if (p1 == lo) lo = p0;
            else defer = false;
          }
          const int64_t end = (M->nparams + 3) / 4 * 4;  // the region's zero padding past nparams is inert
          rr0[0] = 0, rr1[0] = lo, rr0[1] = hi, rr1[1] = end;
          if ((lo & 3) || (hi & 3) || end > M->region) defer = false;
        }
        if (defer) {
          const float *g = R.gout;
          const int32_t *ids = R.ids, *bad = M->L[M->emb].bad;
          float *gE = M->grads + R.poff, *rest = M->grads, *ws = c->scratch;
          const size_t wsf = c->scratch_floats;
          const int V = R.V, T = R.T, D = R.D, W = M->workers;
          hipStream_t st = c->stream;
          M->upd_fn = [=](const AdamStep &a) {
            AdamStep u = a;
            u.rest = rest;
            for (int r = 0; r < 2; ++r) {
              u.r0[r] = rr0[r];
              u.r1[r] = rr1[r];
            }
            return launch_embed_grad(g, ids, gE, V, B, T, D, W, scale, bad, st, ws, wsf, peg, &u);
          };
          M->upd_name = "embed_grad_adam";
          M->upd_units = units + 28.0 * M->nparams;
        } else {
          KTimer kt(c, GN_KCLASS_OTHER, "embed_grad", units);
          HIP_OK(c, launch_embed_grad(R.gout, R.ids, M->grads + R.poff, R.V, B, R.T, R.D, M->workers, scale,
                                      M->L[M->emb].bad, c->stream, c->scratch, c->scratch_floats, peg));
        }
        if (below && below->gout)  // indices carry no gradient (embedding.go:156-163)
          HIP_OK(c, launch_fill(below->gout, 0.0f, (int64_t)B * R.T, c->stream));
        is_dz = false;
        break;
      }
      case GN_LAYER_LSTM_UNROLLER: {
        const int H = R.H, T = R.T, I = R.I, G4 = 4 * H;
        const float *Wx = M->params + R.poff;
        const float *Wh = Wx + (int64_t)G4 * I;
        const float *bias = Wh + (int64_t)G4 * H;
        float *gWx = M->grads + R.poff, *gWh = gWx + (int64_t)G4 * I, *gb = gWh + (int64_t)G4 * H;
        {  // BPTT: Wh^T dG, 2 x 4H x H per sample and step
          KTimer kt(c, GN_KCLASS_OTHER, "lstm_bptt", 2.0 * G4 * H * B * T);
          bool done = false;
          if (R.lcoop && lstm_coop_eligible(B, H)) {
            const hipError_t e = launch_lstm_bwd_coop(R.gout, R.igb, R.tcb, R.cbuf, Wh, bias, R.Dg,
                                                      R.lsync, R.err, &R.lepoch, B, T, H,
                                                      M->lstm_spin_limit, c->stream, R.d.return_sequences ? 1 : 0);
            if (e == hipSuccess) {
              done = true;
            } else {  // refused (e.g. fewer free CUs than workgroups): per-sample kernel from now on
              (void)hipGetLastError();
              R.lcoop = false;
            }
          }
          if (!done)
            HIP_OK(c, launch_lstm_bwd(R.gout, R.igb, R.tcb, R.cbuf, Wh, bias, R.Dg, B, T, H, c->stream,
                                      R.d.return_sequences ? 1 : 0));
        }
        // Below another layer: its gradient dx_t = Wx^T dG_t from the unclipped
        // deltas (lstm.go:642-663; the unroller stacks the steps,
        // unroller.go:200-206), before lstm_weight scales dG in place
        auto lstm_gin = [&]() -> int {
          if (!below || !below->gout) return GN_OK;
          GemmArgs a{};
          a.M = T; a.N = I; a.K = G4;
          a.A = R.Dg; a.lda = G4; a.B = Wx; a.ldb = I;
          a.C = below->gout; a.ldc = I; a.alpha = 1.f;
          a.ws = c->scratch; a.ws_cap = c->scratch_floats;
          a.nbatch = B;
          a.bstride_A = (int64_t)(T + 1) * G4;
          a.bstride_C = (int64_t)T * I;
          KTimer kt(c, GN_KCLASS_GEMM, "gemm_dx", gemm_flops(a));
          HIP_OK(c, launch_gemm('N', 'N', EPI_SCALE, a, c->stream));
          return GN_OK;
        };
        // the clip chains: n = chunk x T steps each
        const int Wc = std::max(1, std::min(M->workers, B)), chunk = (B + Wc - 1) / Wc;
        const double nst = (double)chunk * T, nchain = (double)((B + chunk - 1) / chunk);
        if (!c->timing && R.gcnt) {
          // Gram and clip side by side: the clip (second stream) reads each
          // column tile as soon as the Gram kernel has counted it; a gate
          // queued before the Gram kernel holds it until every chain's clip
          // workgroup is resident.  The tile counts' layout follows B.
          if (R.gB != B) {  // counts and start flags of every chain the largest batch has
            const int Wm = std::max(1, std::min(M->workers, M->maxB));
            const int cm = (M->maxB + Wm - 1) / Wm;
            const size_t ncnt = (size_t)lstm_gram_counters(M->maxB, T, M->workers) +
                                2 * (size_t)((M->maxB + cm - 1) / cm);
            HIP_OK(c, hipMemsetAsync(R.gcnt, 0, ncnt * sizeof(unsigned), c->stream));
            R.gepoch = 0;
            R.gB = B;
          }
          const unsigned ep = ++R.gepoch;
          HIP_OK(c, hipEventRecord(R.lev[0], c->stream));
          HIP_OK(c, hipStreamWaitEvent(c->aux, R.lev[0], 0));
          HIP_OK(c, launch_lstm_clip(R.gram, R.coef, R.wts, B, T, M->workers, c->aux, R.gcnt, ep,
                                     R.gstart, R.err, M->lstm_spin_limit, R.gbail, M->lstm_clip_bail));
          HIP_OK(c, hipEventRecord(R.lev[1], c->aux));
          HIP_OK(c, launch_lstm_clip_gate(R.gstart, B, M->workers, ep, R.err, M->lstm_spin_limit,
                                          c->stream));
          HIP_OK(c, launch_lstm_gram(R.Dg, R.hbuf, in, R.gram, B, T, I, H, M->workers, c->stream,
                                     R.gcnt));
          int rc = lstm_gin();  // beside the clip
          if (rc) return rc;
          HIP_OK(c, hipStreamWaitEvent(c->stream, R.lev[1], 0));
          // the chains whose clip found no Gram kernel running beside it
          // (streams run one after the other); returns at once otherwise
          HIP_OK(c, launch_lstm_clip(R.gram, R.coef, R.wts, B, T, M->workers, c->stream, nullptr, ep,
                                     nullptr, nullptr, 0, R.gbail));
        } else {
          int rc = lstm_gin();
          if (rc) return rc;
          {  // Gram of the steps' contributions: n(n+1)/2 pairs, 2 (4H + H + I) FLOPs each, fp64
            KTimer kt(c, GN_KCLASS_OTHER, "lstm_gram", nchain * nst * (nst + 1) * (5.0 * H + I));
            HIP_OK(c, launch_lstm_gram(R.Dg, R.hbuf, in, R.gram, B, T, I, H, M->workers, c->stream));
          }
          {  // the clip recursion reads each chain's Gram once
            KTimer kt(c, GN_KCLASS_OTHER, "lstm_clip", nchain * 8.0 * nst * (nst + 1) / 2);
            HIP_OK(c, launch_lstm_clip(R.gram, R.coef, R.wts, B, T, M->workers, c->stream));
          }
        }
        {  // dG scaled in place by the step weights, plus the per-sample sums
          KTimer kt(c, GN_KCLASS_OTHER, "lstm_weight", f4(2.0 * B * (T + 1) * G4 + (double)B * G4));
          HIP_OK(c, launch_lstm_weight(R.Dg, R.wts, R.S, B, T, H, c->stream));
        }
        {
          KTimer kt(c, GN_KCLASS_OTHER, "colsum", f4((double)B * G4 + G4));
          HIP_OK(c, launch_colsum(R.S, B, G4, G4, scale, gb, c->scratch, c->scratch_floats, c->stream));
        }
        KTimer kt(c, GN_KCLASS_GEMM, "gemm_dw", 2.0 * G4 * I * B + 2.0 * G4 * H * B * (T + 1));
        GemmArgs a{};  // dWx = scale * S^T x_last
        a.M = G4; a.N = I; a.K = B;
        a.A = R.S; a.lda = G4;
        a.B = in + (int64_t)(T - 1) * I; a.ldb = T * I;
        a.C = gWx; a.ldc = I; a.alpha = scale;
        a.ws = c->scratch; a.ws_cap = c->scratch_floats;
        HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, a, c->stream));
        GemmArgs h{};  // dWh = scale * (w dG)^T hPrev, K over (sample, step)
        h.M = G4; h.N = H; h.K = B * (T + 1);
        h.A = R.Dg; h.lda = G4;
        h.B = R.hbuf; h.ldb = H;
        h.C = gWh; h.ldc = H; h.alpha = scale;
        h.ws = c->scratch; h.ws_cap = c->scratch_floats;
        HIP_OK(c, launch_gemm('T', 'N', EPI_SCALE, h, c->stream));
        is_dz = false;
        break;
      }
      default:
        return set_err(c, GN_ERR_UNSUPPORTED, "layer kind %d", R.d.kind);
    }
    if (ac && R.pcount > 0) {
      // While backward kernels still run, a 256-block grid (one block per CU
      // next to the GEMM's waves) keeps the update off their critical path;
      // the update of the first parameterised layer runs at full width.
      bool last = true;
      for (int j = 0; j < i; ++j)
        if (M->L[j].pcount > 0) last = false;
      // Adam on its own stream: after the layer's dX (main stream) and dW
      // (ctx->aux), so the next layers' dW GEMMs do not queue behind it.  The
      // first layer's update, whose gradients all come from the main stream,
      // follows them there, beside the end of the update before it.
      hipStream_t us = M->adam_s;
      if (last && !dw_aux[i]) {
        us = c->stream;
      } else {
        HIP_OK(c, hipEventRecord(M->sync_ev[i], c->stream));
        HIP_OK(c, hipStreamWaitEvent(M->adam_s, M->sync_ev[i], 0));
        if (dw_aux[i]) HIP_OK(c, hipStreamWaitEvent(M->adam_s, M->dw_ev[i], 0));
      }
      KTimer kt(c, GN_KCLASS_ADAM, "adam", 28.0 * R.pcount, us);
      ++M->step_updates;
      HIP_OK(c, launch_adam(M->params + R.poff, M->grads + R.poff, M->m + R.poff, M->v + R.poff,
                            R.pcount, ac->efflr, ac->b1, ac->b2, ac->omb1, ac->omb2, ac->eps, us,
                            last ? 16384 : 256));
    }
  }
  if (ac) {  // every dW on ctx->aux precedes an update the step now waits for
    HIP_OK(c, hipEventRecord(M->sync_ev[n], M->adam_s));
    HIP_OK(c, hipStreamWaitEvent(c->stream, M->sync_ev[n], 0));
  } else if (aux_used) {  // the pass ends when aux's gradients are done (a captured pass rejoins here)
    HIP_OK(c, hipEventRecord(M->join_ev, c->aux));
    HIP_OK(c, hipStreamWaitEvent(c->stream, M->join_ev, 0));
  }
  return GN_OK;
}

// The fused output-layer kernels serve a training pass when the output layer
// is a Dense with few outputs whose products are small enough that the
// GEMMs' launches, not their work, would set their time (kTailMaxMacs).
static bool tail_eligible(const gn_model *M, const float *in_ptr, int B) {
  const LayerRT &O = M->L.back();
  if (!M->tail_on || O.d.kind != GN_LAYER_DENSE || !O.gout) return false;
  const int C = O.d.out_size, in = O.d.in_size;
  if (!tail_supported(C, in) || (double)B * in * C > kTailMaxMacs) return false;
  const float *W = M->params + O.poff;
  return ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(in_ptr)) & 15) == 0;
}

static int model_accumulate(gn_model *M, const float *x, const float *y, int B,
                            const AdamCoef *ac = nullptr) {
  gn_ctx *c = M->ctx;
  if (B <= 0 || B > M->maxB) return set_err(c, GN_ERR_INVALID, "batch %d outside [1,%d]", B, M->maxB);
  if (!x || !y) return set_err(c, GN_ERR_INVALID, "null input");
  int rc = pass_flags(M, B, true);
  if (rc) return rc;
  M->last_predict = false;
  LayerRT &O = M->L.back();
  const int n = (int)M->L.size();
  int below = n - 2;  // Flatten aliases its input
  while (below >= 0 && M->L[below].d.kind == GN_LAYER_FLATTEN) --below;
  const float *oin = below >= 0 ? M->L[below].out : x;  // the output layer's input
  M->tail_now = tail_eligible(M, oin, B);
  // the Dense that writes that input: itself, or below a training Dropout
  // whose output its GEMM writes (model_forward's fusion)
  M->tail_src = -1;
  M->tail_sp = TailSplitIn();
  if (M->tail_now && below >= 0) {
    int src = below;
    if (M->L[src].d.kind == GN_LAYER_DROPOUT && src >= 1 && M->eff[src] &&
        M->L[src - 1].d.kind == GN_LAYER_DENSE && M->L[src - 1].out_len == M->L[src].out_len)
      --src;
    const int rb = O.d.out_size <= 4 ? 16 : O.d.out_size <= 16 ? 4 : 2;
    if (M->L[src].d.kind == GN_LAYER_DENSE && !M->L[src].ap.jac &&
        (size_t)rb * O.d.in_size * sizeof(float) <= 65536)
      M->tail_src = src;
  }
  rc = model_forward(M, x, B, true);
  if (rc) return rc;
  int row_act = O.ap.row_act;
  const int32_t *bad = M->emb >= 0 ? M->L[M->emb].bad : nullptr;
  if (M->tail_now) {  // read x, W and y; write the activation output, dz and the row losses
    const float *W = M->params + O.poff;
    const int in = O.d.in_size, C = O.d.out_size;
    KTimer kt(c, GN_KCLASS_OTHER, "tail_fwd",
              f4((double)B * in + (double)C * in + C + 3.0 * B * C + B));
    HIP_OK(c, launch_tail_fwd(oin, W, W + (int64_t)in * C, y, O.out, O.gout, M->loss_rows, B, in, C, row_act,
                              O.ap.deriv, M->loss_kind, bad, M->workers, c->stream, M->tail_sp));
  } else {  // read z and y, write the activation output and dz, one loss per row (the batch loss is
            // summed from the rows when it is read, gn_model_read_loss)
    KTimer kt(c, GN_KCLASS_OTHER, "out_rows", f4(4.0 * B * O.out_len + B));
    const hipError_t e = launch_out_rows_reg(O.out, y, O.gout, M->loss_rows, B, O.out_len, row_act,
                                             O.ap.deriv, M->loss_kind, bad, M->workers, c->stream);
    if (e == hipErrorNotSupported) {  // rows longer than 16384 classes
      (void)hipGetLastError();
      HIP_OK(c, launch_out_rows(O.out, y, O.out, O.gout, M->loss_rows, B, O.out_len, row_act,
                                O.ap.deriv, M->loss_kind, bad, M->workers, c->stream));
    } else {
      HIP_OK(c, e);
    }
  }
  M->loss_B = B;
  // grads *= 1/B: float32 reciprocal (net.go:767-770), float32(1/float64(B))
  // for the W-worker path (net.go:703-706).
  const float scale = M->workers > 1 ? (float)(1.0 / (double)B) : 1.0f / (float)B;
  rc = model_backward(M, x, B, scale, ac);
  if (rc) return rc;
  M->last_B = B;
  return GN_OK;
}

extern "C" int gn_model_step(gn_model *M) {
  if (!M) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  const AdamCoef a = adam_next(M);  // Adam.NewStep (opt.go:254-258)
  KTimer kt(c, GN_KCLASS_ADAM, "adam", 28.0 * M->nparams);  // read p, g, m, v; write p, m, v
  HIP_OK(c, launch_adam(M->params, M->grads, M->m, M->v, M->nparams, a.efflr, a.b1, a.b2, a.omb1,
                        a.omb2, a.eps, c->stream));
  return GN_OK;
}

// Steps whose launches can be replayed from a graph: no timing events, no
// host-advanced per-step state (MoE gating noise streams, the LSTM's
// cooperative BPTT epochs).
static bool graph_eligible(const gn_model *M) {
  if (!M->graph_on || !M->graph_ok || M->ctx->timing) return false;
  for (const LayerRT &R : M->L)
    if (R.d.kind == GN_LAYER_MOE || R.d.kind == GN_LAYER_LSTM_UNROLLER) return false;
  return true;
}

static int accumulate_graphed(gn_model *M, const float *x, const float *y, int B) {
  gn_ctx *c = M->ctx;
  if (B <= 0 || B > M->maxB) return set_err(c, GN_ERR_INVALID, "batch %d outside [1,%d]", B, M->maxB);
  if (!x || !y) return set_err(c, GN_ERR_INVALID, "null input");
  int rc = pass_flags(M, B, true);
  if (rc) return rc;
  gn_model::StepGraph *g = nullptr;
  for (auto &e : M->graphs)
    if (e.x == x && e.y == y && e.B == B && e.eff == M->eff && e.upd == M->upd_want) g = &e;
  if (g && g->exec) {  // replay: the host state the pass would have set
    M->last_predict = false;
    M->last_B = B;
    M->loss_B = B;
    HIP_OK(c, hipGraphLaunch(g->exec, c->stream));
    M->upd_fn = g->upd_fn;
    M->upd_name = g->upd_name;
    M->upd_units = g->upd_units;
    return GN_OK;
  }
  if (!g) {  // first step with this key: eager (also settles every lazy set-up)
    rc = model_accumulate(M, x, y, B);
    if (rc) return rc;
    if (M->graphs.size() >= 4) {  // keep the 4 newest keys
      if (M->graphs.front().exec) (void)hipGraphExecDestroy(M->graphs.front().exec);
      M->graphs.erase(M->graphs.begin());
    }
    M->graphs.push_back({x, y, B, M->eff, nullptr, M->upd_want, nullptr, nullptr, 0.0});
    return GN_OK;
  }
  // second step with this key: capture the pass, then launch it
  hipGraph_t graph = nullptr;
  HIP_OK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  rc = model_accumulate(M, x, y, B);
  hipError_t e = hipStreamEndCapture(c->stream, &graph);
  if (rc == GN_OK && e == hipSuccess && graph) {
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e == hipSuccess) {
      g->exec = ex;
      g->upd_fn = M->upd_fn;  // the launch the captured pass left out (or none)
      g->upd_name = M->upd_name;
      g->upd_units = M->upd_units;
      HIP_OK(c, hipGraphLaunch(ex, c->stream));
      return GN_OK;
    }
  } else if (graph) {
    (void)hipGraphDestroy(graph);
  }
  // the capture failed: nothing of it ran; this model stays eager from now on
  (void)hipGetLastError();
  M->graph_ok = false;
  drop_graphs(M);
  return model_accumulate(M, x, y, B);
}

// One training step: forward, loss, backward and Adam (Network.TrainBatch
// followed by Network.Step).  Per-layer updates overlapped with the backward
// pass pay off only when the update is long; small models update once at the
// end (the overlapped launches would slow their short backward kernels).
constexpr int64_t kOverlapAdamMin = (int64_t)8 << 20;
static int model_train_step(gn_model *M, const float *x, const float *y, int B) {
  if (!M->overlap_adam || M->nparams < kOverlapAdamMin) {
    M->upd_want = M->upd_on;
    M->upd_fn = nullptr;
    int rc = graph_eligible(M) ? accumulate_graphed(M, x, y, B) : model_accumulate(M, x, y, B);
    M->upd_want = false;
    if (rc) return rc;
    if (!M->upd_fn) return gn_model_step(M);
    // the backward's last launch, left out of the pass, with Network.Step's
    // update (Adam.NewStep, opt.go:254-258, then StepInPlace per parameter)
    gn_ctx *c = M->ctx;
    const AdamCoef a = adam_next(M);
    AdamStep u{};
    u.efflr = a.efflr;
    u.b1 = a.b1;
    u.b2 = a.b2;
    u.omb1 = a.omb1;
    u.omb2 = a.omb2;
    u.eps = a.eps;
    u.stride = M->region;
    KTimer kt(c, GN_KCLASS_OTHER, M->upd_name, M->upd_units);
    const hipError_t e = M->upd_fn(u);
    M->upd_fn = nullptr;
    HIP_OK(c, e);
    return GN_OK;
  }
  if (B <= 0 || B > M->maxB) return set_err(M->ctx, GN_ERR_INVALID, "batch %d outside [1,%d]", B, M->maxB);
  const int saved = M->timestep;
  const AdamCoef a = adam_next(M);
  M->step_updates = 0;
  int rc = model_accumulate(M, x, y, B, &a);
  // Failed before any layer was updated: the step did not happen.  Failed
  // after some layers' updates were launched: those layers hold step t and
  // the others do not, so the parameters are inconsistent (the caller
  // reloads a checkpoint); the timestep stays at t so a retry does not apply
  // bias correction t a second time to the updated layers.
  if (rc && M->step_updates == 0) M->timestep = saved;
  return rc;
}

extern "C" int gn_model_accumulate_device(gn_model *M, const float *x, const float *y, int32_t B) {
  if (!M) return GN_ERR_INVALID;
  ENTRY(M->ctx);
  return model_accumulate(M, x, y, B);
}

extern "C" int gn_model_train_step_device(gn_model *M, const float *x, const float *y, int32_t B) {
  if (!M) return GN_ERR_INVALID;
  ENTRY(M->ctx);
  return model_train_step(M, x, y, B);
}

// Device flags, read once the stream has drained:
//  - Embedding index errors (embedding.go:126-128): an inference pass fails
//    (ForwardBatch returns the error, net.go:447-450); a training step skips
//    the samples as the batch loop does and counts them (M->skipped);
//  - a cooperative BPTT wait that timed out (its gradients are then invalid).
static int check_flags(gn_model *M) {
  gn_ctx *c = M->ctx;
  if (M->L.empty()) return GN_OK;
  for (const LayerRT &Q : M->L)
    if (Q.d.kind == GN_LAYER_LSTM_UNROLLER && Q.err) {
      int flag = 0;
      HIP_OK(c, hipMemcpyAsync(&flag, Q.err, sizeof(int), hipMemcpyDeviceToHost, c->stream));
      HIP_OK(c, hipStreamSynchronize(c->stream));
      if (flag) {
        HIP_OK(c, hipMemsetAsync(Q.err, 0, sizeof(int), c->stream));
        return set_err(c, GN_ERR_HIP,
                       "LSTM: a cross-workgroup wait timed out (BPTT exchange or Gram/clip overlap)");
      }
    }
  if (M->emb < 0) return GN_OK;
  const LayerRT &R = M->L[M->emb];
  if (R.bad && M->last_B > 0) {
    const int B = M->last_B;
    std::vector<int32_t> f(B);
    HIP_OK(c, hipMemcpyAsync(f.data(), R.bad, (size_t)B * sizeof(int32_t), hipMemcpyDeviceToHost,
                             c->stream));
    HIP_OK(c, hipStreamSynchronize(c->stream));
    int nbad = 0, nskip = 0;
    for (int b = 0; b < B; ++b) nbad += f[b] ? 1 : 0;
    if (M->last_predict) {
      if (nbad)
        return set_err(c, GN_ERR_INDEX, "embedding index out of bounds [0, %d) in %d of %d samples",
                       R.V, nbad, B);
      return GN_OK;
    }
    if (M->workers > 1) {  // a worker stops at its chunk's first bad sample
      const int W = std::min(M->workers, B), chunk = (B + W - 1) / W;
      for (int c0 = 0; c0 < B; c0 += chunk) {
        const int c1 = std::min(B, c0 + chunk);
        int b = c0;
        while (b < c1 && !f[b]) ++b;
        nskip += c1 - b;
      }
    } else {
      nskip = nbad;
    }
    M->skipped = nskip;
  }
  return GN_OK;
}

// Samples the last training step skipped because an Embedding index was out
// of range (the reference's batch loop drops them silently, net.go:738-741).
extern "C" int gn_model_skipped_samples(gn_model *M, int32_t *n) {
  if (!M || !n) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  *n = 0;
  if (M->last_predict) return GN_OK;
  HIP_OK(c, hipStreamSynchronize(c->stream));
  int rc = check_flags(M);
  if (rc) return rc;
  *n = M->skipped;
  return GN_OK;
}

extern "C" int gn_model_set_graphs(gn_model *M, int32_t on) {
  if (!M) return GN_ERR_INVALID;
  ENTRY(M->ctx);
  HIP_OK(M->ctx, hipStreamSynchronize(M->ctx->stream));
  M->graph_on = on != 0;
  if (!M->graph_on) drop_graphs(M);
  return GN_OK;
}

extern "C" int gn_model_graph_count(gn_model *M, int32_t *n) {
  if (!M || !n) return GN_ERR_INVALID;
  int k = 0;
  for (const auto &g : M->graphs) k += g.exec ? 1 : 0;
  *n = k;
  return GN_OK;
}

extern "C" int gn_debug_lstm_spin_limit(gn_model *M, int32_t polls) {
  if (!M) return GN_ERR_INVALID;
  M->lstm_spin_limit = polls;
  return GN_OK;
}

extern "C" int gn_debug_fused_tail(gn_model *M, int32_t on) {
  if (!M) return GN_ERR_INVALID;
  ENTRY(M->ctx);
  HIP_OK(M->ctx, hipStreamSynchronize(M->ctx->stream));
  M->tail_on = on != 0;
  drop_graphs(M);  // captured passes hold the other path
  return GN_OK;
}

extern "C" int gn_debug_step_update(gn_model *M, int32_t on) {
  if (!M) return GN_ERR_INVALID;
  ENTRY(M->ctx);
  HIP_OK(M->ctx, hipStreamSynchronize(M->ctx->stream));
  M->upd_on = on != 0;
  drop_graphs(M);  // captured passes hold the other path
  return GN_OK;
}

extern "C" int gn_debug_side_streams(gn_model *M, int32_t on) {
  if (!M) return GN_ERR_INVALID;
  ENTRY(M->ctx);
  HIP_OK(M->ctx, hipStreamSynchronize(M->ctx->stream));
  HIP_OK(M->ctx, hipStreamSynchronize(M->ctx->aux));
  M->side_ok = on != 0;
  drop_graphs(M);  // captured passes hold the other arrangement
  return GN_OK;
}

extern "C" int gn_debug_lstm_clip_bail(gn_model *M, int32_t polls) {
  if (!M) return GN_ERR_INVALID;
  M->lstm_clip_bail = polls;
  return GN_OK;
}

extern "C" int gn_model_train_step(gn_model *M, const float *x, const float *y, int32_t B,
                                   float *loss_out) {
  if (!M) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  if (B <= 0 || B > M->maxB) return set_err(c, GN_ERR_INVALID, "batch %d outside [1,%d]", B, M->maxB);
  if (!x || !y) return set_err(c, GN_ERR_INVALID, "null input");
  HIP_OK(c, hipMemcpyAsync(M->xin, x, (size_t)B * M->L[0].in_len * sizeof(float),
                           hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipMemcpyAsync(M->yin, y, (size_t)B * M->L.back().out_len * sizeof(float),
                           hipMemcpyHostToDevice, c->stream));
  int rc = model_train_step(M, M->xin, M->yin, B);
  if (rc) return rc;
  if (loss_out) return gn_model_read_loss(M, loss_out);
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return check_flags(M);
}

extern "C" int gn_model_read_loss(gn_model *M, float *loss) {
  if (!M || !loss) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  // the batch loss of the last training pass, summed as the batch loop does:
  // running float32 sums per worker chunk, the chunks' sums in worker order,
  // divided by float32(B) (net.go:650-716 with W workers, :734-784 with one)
  const int B = M->loss_B;
  *loss = 0.0f;
  if (B <= 0) return GN_OK;
  std::vector<float> rows(B);
  HIP_OK(c, hipMemcpyAsync(rows.data(), M->loss_rows, (size_t)B * sizeof(float), hipMemcpyDeviceToHost,
                           c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  const int W = std::max(1, std::min(M->workers, B)), chunk = M->workers > 1 ? (B + W - 1) / W : B;
  float total = 0.0f;
  for (int c0 = 0; c0 < B; c0 += chunk) {
    float local = 0.0f;
    for (int i = c0; i < std::min(B, c0 + chunk); ++i) local += rows[i];
    total += local;
  }
  *loss = total / (float)B;
  return check_flags(M);
}

extern "C" int gn_model_predict(gn_model *M, const float *x, int32_t B, float *out) {
  if (!M) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  if (B <= 0 || B > M->maxB || !x || !out) return set_err(c, GN_ERR_INVALID, "bad predict args");
  // Sequential.Predict / PredictBatch set training=false and leave it so
  // (sequential.go:118-122, 133-134): later training steps run that way too
  for (LayerRT &R : M->L) R.train = 0;
  int rc = pass_flags(M, B, false);
  if (rc) return rc;
  HIP_OK(c, hipMemcpyAsync(M->xin, x, (size_t)B * M->L[0].in_len * sizeof(float),
                           hipMemcpyHostToDevice, c->stream));
  M->last_predict = true;
  rc = model_forward(M, M->xin, B, false);
  if (rc) return rc;
  M->last_B = B;
  LayerRT &O = M->L.back();
  HIP_OK(c, hipMemcpyAsync(out, O.out, (size_t)B * O.out_len * sizeof(float),
                           hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return check_flags(M);
}

extern "C" int gn_model_predict_device(gn_model *M, const float *x, int32_t B, float *out) {
  if (!M) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  if (B <= 0 || B > M->maxB || !x || !out) return set_err(c, GN_ERR_INVALID, "bad predict args");
  for (LayerRT &R : M->L) R.train = 0;  // ForwardBatch: SetTraining(false) (net.go:440)
  int rc = pass_flags(M, B, false);
  if (rc) return rc;
  M->last_predict = true;
  rc = model_forward(M, x, B, false);
  if (rc) return rc;
  M->last_B = B;
  LayerRT &O = M->L.back();
  HIP_OK(c, hipMemcpyAsync(out, O.out, (size_t)B * O.out_len * sizeof(float),
                           hipMemcpyDeviceToDevice, c->stream));
  return GN_OK;
}

extern "C" int gn_model_layer_output(gn_model *M, int32_t layer, float *dst, int64_t n) {
  if (!M || layer < 0 || layer >= (int)M->L.size() || !dst) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  LayerRT &R = M->L[layer];
  const int64_t have = (int64_t)M->last_B * R.out_len;
  if (n > have) return set_err(c, GN_ERR_INVALID, "asked %lld > %lld", (long long)n, (long long)have);
  HIP_OK(c, hipMemcpyAsync(dst, R.out, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return GN_OK;
}

static int running_stats_copy(gn_model *M, int32_t layer, float *mean, float *var, int32_t n,
                              bool d2h) {
  if (!M || layer < 0 || layer >= (int)M->L.size()) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  LayerRT &R = M->L[layer];
  if (R.d.kind != GN_LAYER_BATCHNORM2D)
    return set_err(c, GN_ERR_UNSUPPORTED, "layer %d is not BatchNorm2D", layer);
  if (n != R.C || !mean || !var)
    return set_err(c, GN_ERR_INVALID, "running stats hold %d channels, asked %d", R.C, n);
  const size_t bytes = (size_t)n * sizeof(float);
  const hipMemcpyKind k = d2h ? hipMemcpyDeviceToHost : hipMemcpyHostToDevice;
  HIP_OK(c, hipMemcpyAsync(d2h ? (void *)mean : (void *)R.rmean, d2h ? (void *)R.rmean : (void *)mean,
                           bytes, k, c->stream));
  HIP_OK(c, hipMemcpyAsync(d2h ? (void *)var : (void *)R.rvar, d2h ? (void *)R.rvar : (void *)var,
                           bytes, k, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return GN_OK;
}

extern "C" int gn_model_get_running_stats(gn_model *M, int32_t layer, float *mean, float *var,
                                          int32_t n) {
  return running_stats_copy(M, layer, mean, var, n, true);
}

extern "C" int gn_model_set_running_stats(gn_model *M, int32_t layer, const float *mean,
                                          const float *var, int32_t n) {
  return running_stats_copy(M, layer, const_cast<float *>(mean), const_cast<float *>(var), n, false);
}

extern "C" int gn_model_layer_argmax(gn_model *M, int32_t layer, int32_t *dst, int64_t n) {
  if (!M || layer < 0 || layer >= (int)M->L.size() || !dst) return GN_ERR_INVALID;
  gn_ctx *c = M->ctx;
  ENTRY(c);
  LayerRT &R = M->L[layer];
  // MaxPool2D: the argmax switch of every output; MoE: the k experts each
  // sample was routed to, in routing order
  const int32_t *src = R.d.kind == GN_LAYER_MOE ? R.mact : R.argmax;
  if (!src) return set_err(c, GN_ERR_UNSUPPORTED, "layer %d has no argmax switches or routes", layer);
  const int64_t have = (int64_t)M->last_B * (R.d.kind == GN_LAYER_MOE ? R.K : R.out_len);
  if (n > have) return set_err(c, GN_ERR_INVALID, "asked %lld > %lld", (long long)n, (long long)have);
  HIP_OK(c, hipMemcpyAsync(dst, src, n * sizeof(int32_t), hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return GN_OK;
}

// ---------------------------------------------------------------------------
// Model views for the checkpoint writers (gn_checkpoint.hip)
// ---------------------------------------------------------------------------
namespace gn {
int model_layer_count(gn_model *M) { return (int)M->L.size(); }
const gn_layer_desc *model_layer_desc(gn_model *M, int i) { return &M->L[i].d; }
int model_loss_kind(gn_model *M) { return M->loss_kind; }
std::vector<uint64_t> *model_noise_streams(gn_model *M, int i) {
  return M->L[i].d.kind == GN_LAYER_MOE ? &M->L[i].mrng : nullptr;
}
void model_set_timestep(gn_model *M, int t) { M->timestep = t; }
int model_timestep(gn_model *M) { return M->timestep; }
const gn_adam_desc &model_adam(gn_model *M) { return M->adam; }
bool model_master_dims(gn_model *M) { return M->master_dims; }
void model_layer_geom(gn_model *M, int i, ConvShape *cs, PoolShape *ps, float *eps) {
  if (cs) *cs = M->L[i].cs;
  if (ps) *ps = M->L[i].ps;
  if (eps) *eps = M->L[i].eps;
}
int model_error(gn_model *M, int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return set_err(M->ctx, code, "%s", buf);
}
}  // namespace gn
