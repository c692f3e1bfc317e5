// Memory-bound kernels of the training step: Adam over the flat arena, bias
// gradient column sums, activation derivatives, the output-layer row kernel
// (row activation + loss + loss gradient + activation Jacobian), dropout and
// the batch-mean loss.
//
// Rounding follows the reference's float32 expression order (the library is
// built with -ffp-contract=off and correctly rounded fp32 division and square
// root), and transcendentals go through double
// precision exactly where the Go code calls math.Exp / math.Log / math.Tanh
// on float64 arguments.
#include "gn_common.h"

#include <algorithm>

namespace gn {

constexpr int TPB = 256;

// ---------------------------------------------------------------------------
// Adam.StepInPlace over the arena (adam1, opt.go:244-251): 28 bytes of HBM
// traffic per parameter (read p,g,m,v; write p,m,v).
// ---------------------------------------------------------------------------
// Each thread handles U float4 groups per iteration (spaced one block apart,
// so every load instruction stays coalesced) and issues all 4*U loads before
// the arithmetic, which keeps enough bytes in flight per CU to run near the
// HBM limit: U = 4 for arenas above 8 Mi parameters (C3: 5.92 TB/s; U = 1
// 5.22), U = 1 below when the grid is not capped, where one pass of single
// groups finishes sooner (C4's 4.9 M parameters: 22.1 vs 23.8 us in a
// scratch harness).
constexpr int ADAM_U = 4;
constexpr int64_t kAdamSmall = 8 << 20;

template <int U>
__device__ __forceinline__ void adam_range(float *__restrict__ p, const float *__restrict__ g,
                                           float *__restrict__ m, float *__restrict__ v, int64_t n,
                                           float efflr, float b1, float b2, float omb1, float omb2,
                                           float eps) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  constexpr int ADAM_U = U;
  const int64_t n4 = n >> 2;
  const int64_t stride = (int64_t)gridDim.x * TPB * ADAM_U;
  f4v *p4 = reinterpret_cast<f4v *>(p);
  const f4v *g4 = reinterpret_cast<const f4v *>(g);
  f4v *m4 = reinterpret_cast<f4v *>(m);
  f4v *v4 = reinterpret_cast<f4v *>(v);
  for (int64_t i0 = (int64_t)blockIdx.x * TPB * ADAM_U + threadIdx.x; i0 < n4; i0 += stride) {
    f4v pp[ADAM_U], gg[ADAM_U], mm[ADAM_U], vv[ADAM_U];
#pragma unroll
    for (int u = 0; u < ADAM_U; ++u) {
      const int64_t i = i0 + (int64_t)u * TPB;
      if (i < n4) {
        pp[u] = __builtin_nontemporal_load(p4 + i);
        gg[u] = __builtin_nontemporal_load(g4 + i);
        mm[u] = __builtin_nontemporal_load(m4 + i);
        vv[u] = __builtin_nontemporal_load(v4 + i);
      }
    }
#pragma unroll
    for (int u = 0; u < ADAM_U; ++u) {
      const int64_t i = i0 + (int64_t)u * TPB;
      if (i < n4) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float pq = pp[u][q], mq = mm[u][q], vq = vv[u][q];
          adam1(pq, gg[u][q], mq, vq, efflr, b1, b2, omb1, omb2, eps);
          pp[u][q] = pq;
          mm[u][q] = mq;
          vv[u][q] = vq;
        }
        __builtin_nontemporal_store(pp[u], p4 + i);
        __builtin_nontemporal_store(mm[u], m4 + i);
        __builtin_nontemporal_store(vv[u], v4 + i);
      }
    }
  }
  // scalar tail (n % 4 elements), handled by the first threads of block 0
  if (blockIdx.x == 0) {
    const int64_t i = (n4 << 2) + threadIdx.x;
    if (i < n) adam1(p[i], g[i], m[i], v[i], efflr, b1, b2, omb1, omb2, eps);
  }
}

template <int U>
__global__ __launch_bounds__(TPB) void adam_kernel(float *__restrict__ p, const float *__restrict__ g,
                                                   float *__restrict__ m, float *__restrict__ v, int64_t n,
                                                   float efflr, float b1, float b2, float omb1, float omb2,
                                                   float eps) {
  adam_range<U>(p, g, m, v, n, efflr, b1, b2, omb1, omb2, eps);
}

hipError_t launch_adam(float *p, const float *g, float *m, float *v, int64_t n, float efflr,
                       float b1, float b2, float omb1, float omb2, float eps, hipStream_t s,
                       int max_blocks) {
  if (n <= 0) return hipSuccess;
  // The vector loop needs 16 B aligned pointers.  Ranges that start inside an
  // aligned group (a layer's slice of the arena, whose four regions share one
  // alignment) take their first 1-3 elements through the scalar tail path.
  const uintptr_t mis = reinterpret_cast<uintptr_t>(p) & 15;
  if (((reinterpret_cast<uintptr_t>(g) & 15) != mis) || ((reinterpret_cast<uintptr_t>(m) & 15) != mis) ||
      ((reinterpret_cast<uintptr_t>(v) & 15) != mis) || (mis & 3))
    return hipErrorInvalidValue;
  if (mis) {
    const int64_t head = std::min<int64_t>(n, (int64_t)((16 - mis) / 4));
    hipLaunchKernelGGL(adam_kernel<1>, dim3(1), dim3(TPB), 0, s, p, g, m, v, head, efflr, b1, b2, omb1,
                       omb2, eps);
    p += head;
    g += head;
    m += head;
    v += head;
    n -= head;
    if (n <= 0) return hipGetLastError();
  }
  const int64_t n4 = n >> 2;
  // single groups only where they make one pass (not under a block cap)
  const int u = n <= kAdamSmall && (n4 + TPB - 1) / TPB <= max_blocks ? 1 : ADAM_U;
  int64_t blocks = (n4 + TPB * u - 1) / (TPB * u);
  if (blocks > max_blocks) blocks = max_blocks;
  if (blocks < 1) blocks = 1;
  if (u == 1)
    hipLaunchKernelGGL(adam_kernel<1>, dim3((unsigned)blocks), dim3(TPB), 0, s, p, g, m, v, n, efflr,
                       b1, b2, omb1, omb2, eps);
  else
    hipLaunchKernelGGL(adam_kernel<ADAM_U>, dim3((unsigned)blocks), dim3(TPB), 0, s, p, g, m, v, n, efflr,
                       b1, b2, omb1, omb2, eps);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Bias gradient: db[o] = scale * sum_b dz[b, o]   (gradB += dz, layer.go:566;
// averaged by grads *= 1/B, net.go:767-770).  Blocks over 32-column strips
// (whole 128-byte lines) and, when the strips alone are too few to keep the
// chip's loads in flight, row chunks whose partials a second pass adds in
// chunk order.
// ---------------------------------------------------------------------------
// Up to three column sums of equal shape in one launch (blockIdx.z selects the
// matrix); each member is summed exactly as a launch of its own.
struct ColsumSet {
  const float *dz[3];
  float *out[3];
};

// Partials summed in chunk order, one thread per column (coalesced rows).
__global__ __launch_bounds__(TPB) void colsum_final(ColsumSet set, const float *__restrict__ part,
                                                    int chunks, int cols, float scale) {
  const int col = blockIdx.x * TPB + threadIdx.x;
  if (col >= cols) return;
  float *__restrict__ out = set.out[blockIdx.z];
  part += (size_t)blockIdx.z * chunks * cols + col;
  float s = 0.f;
  for (int c = 0; c < chunks; c += 8) {  // eight loads in flight, added in chunk order
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = c + u < chunks ? part[(size_t)(c + u) * cols] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (c + u < chunks) s += v[u];
  }
  out[col] = s * scale;
}

// One block per 32-column strip and row chunk (blockIdx.y; a single chunk
// writes the scaled sums, several write partials for colsum_final).  V4 (cols
// and ld multiples of 4, 16-byte aligned rows): thread t takes columns
// 4 (t % 8) .. +3 of the strip and rows t / 8, t / 8 + 32, ... of the chunk
// (whole 128-byte lines, CS_U loads in flight); otherwise column t % 32 and
// rows t / 32, t / 32 + 8, ....  Each thread's rows are summed in row order,
// then the row lanes of a column in lane order.
constexpr int CS_W = 32;  // columns per strip
constexpr int CS_U = 8;   // loads in flight per thread
template <bool V4>
__global__ __launch_bounds__(TPB) void colsum_strip(ColsumSet set, int rows, int cols, int ld,
                                                    int rows_per_chunk, float *__restrict__ part,
                                                    float scale) {
  constexpr int RL = V4 ? TPB / (CS_W / 4) : TPB / CS_W;  // row lanes
  __shared__ float red[RL][CS_W + 1];
  const float *__restrict__ dz = set.dz[blockIdx.z];
  float *__restrict__ out = set.out[blockIdx.z];
  const int t = threadIdx.x, c0 = blockIdx.x * CS_W;
  const int r0 = blockIdx.y * rows_per_chunk, r1 = min(rows, r0 + rows_per_chunk);
  if (V4) {
    const int q = t % (CS_W / 4), rl = t / (CS_W / 4), col = c0 + 4 * q;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (col < cols) {
      const float *p = dz + col;
      int r = r0 + rl;
      for (; r + (CS_U - 1) * RL < r1; r += CS_U * RL) {
        float4 v[CS_U];
#pragma unroll
        for (int u = 0; u < CS_U; ++u) v[u] = *reinterpret_cast<const float4 *>(p + (size_t)(r + u * RL) * ld);
#pragma unroll
        for (int u = 0; u < CS_U; ++u) {
          s.x += v[u].x; s.y += v[u].y; s.z += v[u].z; s.w += v[u].w;
        }
      }
      for (; r < r1; r += RL) {
        const float4 a = *reinterpret_cast<const float4 *>(p + (size_t)r * ld);
        s.x += a.x; s.y += a.y; s.z += a.z; s.w += a.w;
      }
    }
    red[rl][4 * q + 0] = s.x;
    red[rl][4 * q + 1] = s.y;
    red[rl][4 * q + 2] = s.z;
    red[rl][4 * q + 3] = s.w;
  } else {
    const int cl = t % CS_W, rl = t / CS_W, col = c0 + cl;
    float s = 0.f;
    if (col < cols) {
      const float *p = dz + col;
      int r = r0 + rl;
      for (; r + (CS_U - 1) * RL < r1; r += CS_U * RL) {
        float v[CS_U];
#pragma unroll
        for (int u = 0; u < CS_U; ++u) v[u] = p[(size_t)(r + u * RL) * ld];
#pragma unroll
        for (int u = 0; u < CS_U; ++u) s += v[u];
      }
      for (; r < r1; r += RL) s += p[(size_t)r * ld];
    }
    red[rl][cl] = s;
  }
  __syncthreads();
  if (t < CS_W && c0 + t < cols) {
    float v = 0.f;
#pragma unroll 8
    for (int j = 0; j < RL; ++j) v += red[j][t];
    if (gridDim.y == 1) out[c0 + t] = v * scale;
    else part[((size_t)blockIdx.z * gridDim.y + blockIdx.y) * cols + c0 + t] = v;
  }
}

// Row chunks: enough blocks to keep loads in flight across the chip (about
// 256 strip blocks in all), each chunk at least 256 rows; one chunk (a single
// launch) when the strips alone give that many blocks or the rows are few.
static int colsum_chunks(int rows, int cols, int n, size_t cap) {
  const int64_t strips = (int64_t)((cols + CS_W - 1) / CS_W) * n;
  int64_t chunks = std::min<int64_t>((256 + strips - 1) / strips, (rows + 255) / 256);
  if (chunks > 64) chunks = 64;
  if (chunks > 1 && (size_t)chunks * cols * n > cap) chunks = (int64_t)(cap / ((size_t)cols * n));
  return chunks < 1 ? 1 : (int)chunks;
}

hipError_t launch_colsum_multi(const float *const *dz, float *const *out, int n, int rows, int cols,
                               int ld, float scale, float *scratch, size_t scratch_cap,
                               hipStream_t s) {
  if (cols <= 0 || n <= 0) return hipSuccess;
  if (n > 3) return hipErrorInvalidValue;
  const int chunks = colsum_chunks(rows, cols, n, scratch_cap);
  if (n > 1 && chunks > 1 && (size_t)n * chunks * cols > scratch_cap) {
    for (int i = 0; i < n; ++i) {  // partials of all members do not fit: one at a time
      const hipError_t e = launch_colsum_multi(dz + i, out + i, 1, rows, cols, ld, scale, scratch,
                                               scratch_cap, s);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  ColsumSet set{};
  bool v4 = cols % 4 == 0 && ld % 4 == 0;
  for (int i = 0; i < n; ++i) {
    set.dz[i] = dz[i];
    set.out[i] = out[i];
    v4 = v4 && (reinterpret_cast<uintptr_t>(dz[i]) & 15) == 0;
  }
  const int rpc = (rows + chunks - 1) / chunks;
  const dim3 g((cols + CS_W - 1) / CS_W, chunks, n);
  if (v4)
    hipLaunchKernelGGL(colsum_strip<true>, g, dim3(TPB), 0, s, set, rows, cols, ld, rpc, scratch, scale);
  else
    hipLaunchKernelGGL(colsum_strip<false>, g, dim3(TPB), 0, s, set, rows, cols, ld, rpc, scratch, scale);
  if (chunks > 1)
    hipLaunchKernelGGL(colsum_final, dim3((cols + TPB - 1) / TPB, 1, n), dim3(TPB), 0, s, set,
                       scratch, chunks, cols, scale);
  return hipGetLastError();
}

hipError_t launch_colsum(const float *dz, int rows, int cols, int ld, float scale, float *out,
                         float *scratch, size_t scratch_cap, hipStream_t s) {
  return launch_colsum_multi(&dz, &out, 1, rows, cols, ld, scale, scratch, scratch_cap, s);
}

// ---------------------------------------------------------------------------
// Activation derivative from the saved output (Dense/Conv default branch:
// dz = grad * act.Derivative(preAct), layer.go:561-567).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float deriv_of(float out, int kind) {
  switch (kind) {
    case D_RELU: return out > 0.0f ? 1.0f : 0.0f;
    case D_SIGMOID: return out * (1.0f - out);
    case D_TANH: return 1.0f - out * out;
    case D_NAN: return __builtin_nanf("");
    case D_GELU: return gelu_deriv(out);
    default: return 1.0f;
  }
}

__device__ __forceinline__ float fwd_of(float v, int kind) {
  switch (kind) {
    case F_RELU: return v > 0.0f ? v : 0.0f;
    case F_SIGMOID: return 1.0f / (1.0f + (float)exp((double)(-v)));
    case F_TANH: return (float)tanh((double)v);
    case F_NAN: return __builtin_nanf("");
    case F_LEAKY: return v > 0.0f ? v : 0.1f * v;
    default: return v;
  }
}

__global__ __launch_bounds__(TPB) void dact_kernel(const float *__restrict__ g,
                                                   const float *__restrict__ out,
                                                   float *__restrict__ dz, int64_t n, int kind) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dz[i] = g[i] * deriv_of(out[i], kind);
}

hipError_t launch_dact(const float *g, const float *out, float *dz, int64_t n, int kind,
                       hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + TPB - 1) / TPB;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(dact_kernel, dim3((unsigned)blocks), dim3(TPB), 0, s, g, out, dz, n, kind);
  return hipGetLastError();
}

__global__ __launch_bounds__(TPB) void act_kernel(float *__restrict__ x, int64_t n, int kind) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    x[i] = fwd_of(x[i], kind);
}

hipError_t launch_act_inplace(float *x, int64_t n, int kind, hipStream_t s) {
  if (n <= 0 || kind == F_IDENTITY) return hipSuccess;
  int64_t blocks = (n + TPB - 1) / TPB;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(act_kernel, dim3((unsigned)blocks), dim3(TPB), 0, s, x, n, kind);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Block reductions over blockDim.x / 64 wave64s (at most 16).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float block_sum(float v, float *sh) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) sh[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nw; ++i) s += sh[i];
  return s;
}
__device__ __forceinline__ float block_max(float v, float *sh) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) sh[w] = v;
  __syncthreads();
  float m = sh[0];
  for (int i = 1; i < nw; ++i) m = fmaxf(m, sh[i]);
  return m;
}

// Row activation (Softmax.ActivateBatch activations.go:161-183 /
// LogSoftmax.ActivateBatch :204-236), in place over one row.
__device__ void row_activate(float *row, int C, int row_act, int fwd, float *sh) {
  const int t = threadIdx.x, nt = blockDim.x;
  if (row_act == ROW_SOFTMAX || row_act == ROW_LOGSOFTMAX) {
    float mx = -__builtin_inff();
    for (int i = t; i < C; i += nt) mx = fmaxf(mx, row[i]);
    mx = block_max(mx, sh);
    float s = 0.f;
    for (int i = t; i < C; i += nt) s += (float)exp((double)(row[i] - mx));
    s = block_sum(s, sh);
    if (row_act == ROW_SOFTMAX) {
      for (int i = t; i < C; i += nt) row[i] = (float)exp((double)(row[i] - mx)) / s;
    } else {
      const float ls = (float)log((double)s);
      for (int i = t; i < C; i += nt) row[i] = row[i] - mx - ls;
    }
  } else if (row_act == ROW_ELEMWISE) {
    for (int i = t; i < C; i += nt) row[i] = fwd_of(row[i], fwd);
  }
}

// Threads per row for the row kernels: long rows get 16 waves.
static int row_threads(int C) { return C >= 4096 ? 1024 : TPB; }

// Output layer: z (pre-activations, overwritten by the activation output),
// per-sample loss (loss.go:53-67 MSE, :120-141 CE), loss gradient
// (loss.go:90-105, :165-178) and dz through the activation (Q4):
//   Softmax    dz_k = sum_i g_i p_i (d_ik - p_k) = p_k g_k - p_k sum_i g_i p_i  (layer.go:504-529)
//   LogSoftmax dz_k = sum_i g_i (d_ik - exp(o_k)) = g_k - exp(o_k) sum_i g_i     (layer.go:530-560)
//   otherwise  dz_k = g_k * Derivative                                          (layer.go:561-567)
//
// Samples the batch loop skips (bad[b], an Embedding index error) add no loss
// and their dz row is 0, so no layer's gradient sees them: with workers == 1
// only the bad sample itself (net.go:738-741); with workers > 1 the worker
// returns at its chunk's first bad sample, so the rest of the chunk is
// skipped too and the chunk's loss is never stored (net.go:641-644, 653-655).
__global__ __launch_bounds__(1024) void out_rows_kernel(float *__restrict__ zo,
                                                       const float *__restrict__ y,
                                                       float *__restrict__ dz,
                                                       float *__restrict__ loss_rows, int C,
                                                       int row_act, int fwd, int deriv,
                                                       int loss_kind,
                                                       const int32_t *__restrict__ bad, int chunk) {
  __shared__ float sh[16];
  const int b = blockIdx.x, t = threadIdx.x, nt = blockDim.x;
  bool valid = true, keep_loss = true;
  if (bad) {
    if (chunk > 0) {
      const int c0 = (b / chunk) * chunk, c1 = min((int)gridDim.x, c0 + chunk);
      for (int i = c0; i < c1; ++i)
        if (bad[i]) {
          keep_loss = false;
          if (i <= b) valid = false;
        }
    } else {
      valid = keep_loss = !bad[b];
    }
  }
  float *o = zo + (size_t)b * C;
  const float *yr = y + (size_t)b * C;
  float *d = dz + (size_t)b * C;
  row_activate(o, C, row_act, fwd, sh);
  __syncthreads();
  // loss and its gradient g (kept in d)
  float l = 0.f;
  if (loss_kind == GN_LOSS_MSE) {
    const float factor = 2.0f / (float)C;
    for (int i = t; i < C; i += nt) {
      const float df = o[i] - yr[i];
      l += df * df;
      d[i] = factor * df;
    }
    l = block_sum(l, sh);
    l = l / (float)C;
  } else {
    for (int i = t; i < C; i += nt) {
      float pv = o[i];
      if (pv < 1e-10f) pv = 1e-10f;
      const float yi = yr[i];
      l -= yi * (float)log((double)pv);
      d[i] = o[i] - yi;
    }
    l = block_sum(l, sh);
  }
  if (t == 0) loss_rows[b] = keep_loss ? l : 0.0f;
  // Jacobian / derivative
  if (row_act == ROW_SOFTMAX) {
    float s1 = 0.f;
    for (int i = t; i < C; i += nt) s1 += d[i] * o[i];
    s1 = block_sum(s1, sh);
    for (int i = t; i < C; i += nt) d[i] = d[i] * o[i] - o[i] * s1;
  } else if (row_act == ROW_LOGSOFTMAX) {
    float s1 = 0.f;
    for (int i = t; i < C; i += nt) s1 += d[i];
    s1 = block_sum(s1, sh);
    for (int i = t; i < C; i += nt) d[i] = d[i] - (float)exp((double)o[i]) * s1;
  } else {
    for (int i = t; i < C; i += nt) d[i] = d[i] * deriv_of(o[i], deriv);
  }
  if (!valid) {
    __syncthreads();
    for (int i = t; i < C; i += nt) d[i] = 0.0f;
  }
}

hipError_t launch_out_rows(const float *z, const float *y, float *out, float *dz, float *loss_rows,
                           int B, int C, int row_act, int deriv, int loss_kind, const int32_t *bad,
                           int workers, hipStream_t s) {
  (void)z;  // activation is computed in place on `out` (which holds z)
  if (B <= 0) return hipSuccess;
  // fwd kind for ROW_ELEMWISE rides in the high bits of row_act
  const int fwd = row_act >> 8;
  const int W = workers < 1 ? 1 : (workers > B ? B : workers);
  const int chunk = workers > 1 ? (B + W - 1) / W : 0;
  hipLaunchKernelGGL(out_rows_kernel, dim3(B), dim3(row_threads(C)), 0, s, out, y, dz, loss_rows, C,
                     row_act & 0xff, fwd, deriv, loss_kind, bad, chunk);
  return hipGetLastError();
}

// The same row computation with each row held in registers (G threads per
// row, up to OR_PER values each): one pass over z and y, one exp per element
// for the row activation; rows of G = 64 threads are reduced by wave shuffles
// (four rows per block), longer groups through LDS (one row per block).
constexpr int OR_PER = 16;

// The float64 transcendentals out of line: inlined into the 16-way unrolled
// row loops they made the kernels ~60 KB of code, fetched again by every wave.
__device__ __attribute__((noinline)) float or_exp_diff(float a, float b) {
  return (float)exp((double)(a - b));
}
__device__ __attribute__((noinline)) float or_exp(float a) { return (float)exp((double)a); }
// The wide-row kernels (up to 16 values per thread, thousands of classes)
// take the float32 exp, within 1 ulp of the reference's float64 exp rounded
// to float32 (as the attention softmax does): 16 float64 exps per thread had
// set the row kernel's time.
__device__ __forceinline__ float or_exp_diff_i(float a, float b) { return expf(a - b); }
__device__ __forceinline__ float or_exp_i(float a) { return expf(a); }
__device__ __attribute__((noinline)) float or_log(float a) { return (float)log((double)a); }
__device__ __attribute__((noinline)) float or_fwd(float v, int kind) { return fwd_of(v, kind); }
__device__ __attribute__((noinline)) float or_deriv(float o, int kind) { return deriv_of(o, kind); }

template <int G>
__device__ __forceinline__ float group_sum(float v, float *sh, int slot) {
  v = wave_sum(v);
  if (G == 64) return v;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sh[slot * 16 + w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < G / 64; ++i) s += sh[slot * 16 + i];
  return s;
}
template <int G>
__device__ __forceinline__ float group_max(float v, float *sh, int slot) {
  v = wave_max(v);
  if (G == 64) return v;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sh[slot * 16 + w] = v;
  __syncthreads();
  float m = sh[slot * 16];
  for (int i = 1; i < G / 64; ++i) m = fmaxf(m, sh[slot * 16 + i]);
  return m;
}

// The validity of row b under the W-worker split (net.go:412-436): `valid`
// keeps its gradient (no bad sample at or before it in its worker's chunk),
// `keep_loss` its loss (no bad sample in the chunk); without a chunk split
// only the row's own flag counts.
__device__ __forceinline__ void row_validity(const int32_t *__restrict__ bad, int b, int B, int chunk,
                                             bool &valid, bool &keep_loss) {
  valid = keep_loss = true;
  if (!bad) return;
  if (chunk > 0) {
    const int c0 = (b / chunk) * chunk, c1 = min(B, c0 + chunk);
    for (int i = c0; i < c1; ++i)
      if (bad[i]) {
        keep_loss = false;
        if (i <= b) valid = false;
      }
  } else {
    valid = keep_loss = !bad[b];
  }
}

// One output row held in registers by a group of G threads (PER values each,
// element t + k*G): the row activation, the loss and the loss gradient through
// the activation's Jacobian / derivative.  o holds z on entry and the
// activation output on return; d receives dz.  Returns the row's loss.
template <int G, int PER>
__device__ __forceinline__ float out_row_math(float (&o)[PER], const float (&yv)[PER], float (&d)[PER],
                                              int t, int C, int row_act, int fwd, int deriv,
                                              int loss_kind, float *sh, int r) {
  // row activation (activations.go:161-183, 204-236)
  if (row_act == ROW_SOFTMAX || row_act == ROW_LOGSOFTMAX) {
    float mx = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (t + k * G < C) mx = fmaxf(mx, o[k]);
    mx = group_max<G>(mx, sh, r);
    float ef[PER], sm = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      if constexpr (PER >= 8)
        ef[k] = t + k * G < C ? or_exp_diff_i(o[k], mx) : 0.f;
      else
        ef[k] = t + k * G < C ? or_exp_diff(o[k], mx) : 0.f;
      sm += ef[k];
    }
    sm = group_sum<G>(sm, sh, r);
    if (row_act == ROW_SOFTMAX) {
#pragma unroll
      for (int k = 0; k < PER; ++k) o[k] = ef[k] / sm;
    } else {
      const float ls = or_log(sm);
#pragma unroll
      for (int k = 0; k < PER; ++k) o[k] = o[k] - mx - ls;
    }
  } else if (row_act == ROW_ELEMWISE) {
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (t + k * G < C) o[k] = or_fwd(o[k], fwd);
  }
  // loss and its gradient (loss.go:53-105, 120-178)
  float l = 0.f;
  if (loss_kind == GN_LOSS_MSE) {
    const float factor = 2.0f / (float)C;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const bool in = t + k * G < C;
      const float df = o[k] - yv[k];
      l += in ? df * df : 0.f;
      d[k] = factor * df;
    }
    l = group_sum<G>(l, sh, r) / (float)C;
  } else {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      if (t + k * G < C) {
        float pv = o[k];
        if (pv < 1e-10f) pv = 1e-10f;
        // a zero target adds 0 * log(pv) = +-0 to a sum that is never -0: the
        // float64 log is needed only for the others (and a NaN output)
        if (yv[k] != 0.f || pv != pv) l -= yv[k] * or_log(pv);
      }
      d[k] = o[k] - yv[k];
    }
    l = group_sum<G>(l, sh, r);
  }
  // the activation's Jacobian / derivative (layer.go:504-567)
  if (row_act == ROW_SOFTMAX) {
    float s1 = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (t + k * G < C) s1 += d[k] * o[k];
    s1 = group_sum<G>(s1, sh, r);
#pragma unroll
    for (int k = 0; k < PER; ++k) d[k] = d[k] * o[k] - o[k] * s1;
  } else if (row_act == ROW_LOGSOFTMAX) {
    float s1 = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (t + k * G < C) s1 += d[k];
    s1 = group_sum<G>(s1, sh, r);
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (t + k * G < C) d[k] = d[k] - (PER >= 8 ? or_exp_i(o[k]) : or_exp(o[k])) * s1;
  } else {
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (t + k * G < C) d[k] = d[k] * or_deriv(o[k], deriv);
  }
  return l;
}

template <int G, int NT>
__global__ __launch_bounds__(NT) void out_rows_reg_kernel(float *__restrict__ zo,
                                                          const float *__restrict__ y,
                                                          float *__restrict__ dz,
                                                          float *__restrict__ loss_rows, int B,
                                                          int C, int row_act, int fwd, int deriv,
                                                          int loss_kind,
                                                          const int32_t *__restrict__ bad, int chunk) {
  __shared__ float sh[16 * (NT / G) + 16];
  constexpr int RPB = NT / G;
  const int r = threadIdx.x / G, t = threadIdx.x % G;
  const int b = blockIdx.x * RPB + r;
  const bool row_ok = b < B;
  bool valid = true, keep_loss = true;
  if (row_ok) row_validity(bad, b, B, chunk, valid, keep_loss);
  float o[OR_PER], yv[OR_PER], d[OR_PER];
  const float *zr = zo + (size_t)(row_ok ? b : 0) * C, *yr = y + (size_t)(row_ok ? b : 0) * C;
#pragma unroll
  for (int k = 0; k < OR_PER; ++k) {
    const int i = t + k * G;
    const bool in = row_ok && i < C;
    o[k] = in ? zr[i] : 0.f;
    yv[k] = in ? yr[i] : 0.f;
  }
  const float l = out_row_math<G, OR_PER>(o, yv, d, t, C, row_act, fwd, deriv, loss_kind, sh, r);
  if (row_ok) {
    float *orow = zo + (size_t)b * C, *drow = dz + (size_t)b * C;
#pragma unroll
    for (int k = 0; k < OR_PER; ++k) {
      const int i = t + k * G;
      if (i < C) {
        orow[i] = o[k];
        drow[i] = valid ? d[k] : 0.0f;
      }
    }
    if (t == 0) loss_rows[b] = keep_loss ? l : 0.0f;
  }
}

// launch_out_rows for rows that fit the register kernels (C <= 16384);
// hipErrorNotSupported otherwise.
hipError_t launch_out_rows_reg(float *out, const float *y, float *dz, float *loss_rows, int B, int C,
                               int row_act, int deriv, int loss_kind, const int32_t *bad, int workers,
                               hipStream_t s) {
  if (B <= 0) return hipSuccess;
  const int fwd = row_act >> 8;
  const int W = workers < 1 ? 1 : (workers > B ? B : workers);
  const int chunk = workers > 1 ? (B + W - 1) / W : 0;
  if (C <= 256) {
    hipLaunchKernelGGL((out_rows_reg_kernel<64, 256>), dim3((B + 3) / 4), dim3(256), 0, s, out, y, dz,
                       loss_rows, B, C, row_act & 0xff, fwd, deriv, loss_kind, bad, chunk);
  } else if (C <= 256 * OR_PER) {
    hipLaunchKernelGGL((out_rows_reg_kernel<256, 256>), dim3(B), dim3(256), 0, s, out, y, dz,
                       loss_rows, B, C, row_act & 0xff, fwd, deriv, loss_kind, bad, chunk);
  } else if (C <= 512 * OR_PER) {
    hipLaunchKernelGGL((out_rows_reg_kernel<512, 512>), dim3(B), dim3(512), 0, s, out, y, dz,
                       loss_rows, B, C, row_act & 0xff, fwd, deriv, loss_kind, bad, chunk);
  } else if (C <= 1024 * OR_PER) {
    hipLaunchKernelGGL((out_rows_reg_kernel<1024, 1024>), dim3(B), dim3(1024), 0, s, out, y, dz,
                       loss_rows, B, C, row_act & 0xff, fwd, deriv, loss_kind, bad, chunk);
  } else {
    return hipErrorNotSupported;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The output Dense layer of a training pass when it has few outputs
// (C <= TAIL_MAXC): two kernels instead of the forward GEMM, the loss rows,
// the dW GEMM, the bias sums and the dX GEMM, whose launches cost more than
// their work at these sizes.
// ---------------------------------------------------------------------------

// Sums of 64 values over the 64 lanes of a wave: v[j] of every lane summed,
// the total of value j left in lane j (a halving butterfly: 63 shuffles
// instead of 64 x 6; the tree is fixed, so the sums are deterministic).
template <int OFF, int N>
__device__ __forceinline__ void lane_sums_step(float (&v)[64], int lane) {
  const bool up = (lane & OFF) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float send = up ? v[i] : v[i + N / 2];
    const float keep = up ? v[i + N / 2] : v[i];
    v[i] = keep + __shfl_xor(send, OFF, 64);
  }
}
__device__ __forceinline__ float lane_sums(float (&v)[64], int lane) {
  lane_sums_step<32, 64>(v, lane);
  lane_sums_step<16, 32>(v, lane);
  lane_sums_step<8, 16>(v, lane);
  lane_sums_step<4, 8>(v, lane);
  lane_sums_step<2, 4>(v, lane);
  lane_sums_step<1, 2>(v, lane);
  return v[0];
}

// Forward (z = x W^T + b, layer.go:405-470) fused with the loss rows: a block
// of NT threads takes RB rows (RB * CM = 64), its threads split K in float4
// steps (W's rows are read once per block), the waves' partial sums meet in
// LDS in wave order, and wave w then runs out_row_math on row w (and w + NW)
// with one element per lane; targets are loaded before the K loop.  Rows
// past B are computed on the last row and not stored.
template <int CM, int RB, int NT>
__global__ __launch_bounds__(NT) void tail_fwd_kernel(
    const float *__restrict__ x, const float *__restrict__ W, const float *__restrict__ bias,
    const float *__restrict__ y, float *__restrict__ out, float *__restrict__ dz,
    float *__restrict__ loss_rows, int B, int in, int C, int row_act, int fwd, int deriv,
    int loss_kind, const int32_t *__restrict__ bad, int chunk, TailSplitIn sp) {
  static_assert(CM * RB == 64, "one partial sum per lane");
  constexpr int NW = NT / 64, RPW = (RB + NW - 1) / NW;
  __shared__ float red[NW][64];
  extern __shared__ float4 xs4[];  // sp.ws: the block's RB input rows
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int b0 = blockIdx.x * RB;
  const bool in_row = lane < C;
  if (sp.ws) {
    // the layer below's split-K partials summed in split order, its bias and
    // activation, the Dropout above it: gemm_splitk_reduce's values, written
    // out for the backward and kept in LDS as this layer's input
    float *xs = reinterpret_cast<float *>(xs4);
    const size_t MN = (size_t)B * in;
    for (int e = t; e < RB * in; e += NT) {
      const int r = e / in, c = e - r * in, b = b0 + r;
      float xv = 0.f;
      if (b < B) {
        const size_t idx = (size_t)b * in + c;
        float v = sp.ws[idx];
        for (int s0 = 1; s0 < sp.splits; s0 += 8) {  // eight loads in flight, added in split order
          float u8[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) u8[u] = s0 + u < sp.splits ? sp.ws[(s0 + u) * MN + idx] : 0.f;
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (s0 + u < sp.splits) v += u8[u];
        }
        const float yv = fwd_of(v + sp.bias[c], sp.act);
        sp.xo[idx] = yv;
        xv = yv;
        if (sp.dout) {
          xv = sp.mask[c] > 0.f ? yv * sp.scale : 0.0f;
          sp.dout[idx] = xv;
        }
      }
      xs[e] = xv;
    }
    __syncthreads();
  }
  float yreg[RPW];
#pragma unroll
  for (int q = 0; q < RPW; ++q) {
    const int r = w + q * NW, b = b0 + r;
    yreg[q] = r < RB && b < B && in_row ? y[(size_t)b * C + lane] : 0.f;
  }
  const float bv = in_row ? bias[lane] : 0.f;
  const int in4 = in >> 2;
  const float4 *__restrict__ W4 = reinterpret_cast<const float4 *>(W);
  const float4 *xr[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r)
    xr[r] = reinterpret_cast<const float4 *>(x + (size_t)min(b0 + r, B - 1) * in);
  float acc[64];
#pragma unroll
  for (int j = 0; j < 64; ++j) acc[j] = 0.f;
#pragma unroll(CM <= 4 ? 2 : 1)
  for (int k4 = t; k4 < in4; k4 += NT) {
    float4 wv[CM], xv[RB];
#pragma unroll
    for (int o = 0; o < CM; ++o) wv[o] = o < C ? W4[(size_t)o * in4 + k4] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < RB; ++r) xv[r] = sp.ws ? xs4[r * in4 + k4] : xr[r][k4];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int o = 0; o < CM; ++o) {
        float a = acc[r * CM + o];
        a += xv[r].x * wv[o].x;
        a += xv[r].y * wv[o].y;
        a += xv[r].z * wv[o].z;
        a += xv[r].w * wv[o].w;
        acc[r * CM + o] = a;
      }
  }
  red[w][lane] = lane_sums(acc, lane);  // lane j: row j / CM, output j % CM
  __syncthreads();
#pragma unroll
  for (int q = 0; q < RPW; ++q) {
    const int r = w + q * NW;
    if (r >= RB) break;
    const int b = b0 + r;
    const bool row_ok = b < B;
    const int j = r * CM + lane;
    float z = 0.f;
    if (in_row) {
      z = red[0][j];
#pragma unroll
      for (int v = 1; v < NW; ++v) z += red[v][j];
      z += bv;
    }
    float o[1] = {z}, yv[1] = {yreg[q]}, d[1];
    bool valid = true, keep_loss = true;
    if (row_ok) row_validity(bad, b, B, chunk, valid, keep_loss);
    const float l = out_row_math<64, 1>(o, yv, d, lane, C, row_act, fwd, deriv, loss_kind, nullptr, 0);
    if (row_ok) {
      if (in_row) {
        out[(size_t)b * C + lane] = o[0];
        dz[(size_t)b * C + lane] = valid ? d[0] : 0.0f;
      }
      if (lane == 0) loss_rows[b] = keep_loss ? l : 0.0f;
    }
  }
}

// Backward of the same layer: gW = scale dz^T x, gB = scale colsum(dz) and
// gin = dz W with the dX GEMM's epilogue (a Dropout's factor, then act' of
// the layer below from its saved output), plus, when that layer is a Dense
// whose dz gin is, its bias gradient gB_below = scale colsum(gin).  A block
// of NT / 64 waves owns 64 columns of x / gin over every row (lane = column);
// the rows go in 64-row chunks whose dz rows are staged in LDS (zero past C),
// each wave taking 64 / (NT / 64) consecutive rows of a chunk with their x
// (and saved-output) loads issued together; the waves' partial sums meet in
// a fixed LDS tree.
// gB comes from block 0.
constexpr int TAIL_MAXC = 32;
constexpr int TAIL_ROWS = 64;
// With POOL, gin is the gradient of a Flatten over a 2x2 stride-2 MaxPool2D
// whose windows tile its pH x pW input planes: instead of gin, each value goes
// to the input position its switch names and the window's other three
// positions get 0 (maxpool_bwd_kernel for non-overlapping windows), into pgin.
template <int CM, int NT, bool POOL>
__global__ __launch_bounds__(NT) void tail_bwd_kernel(
    const float *__restrict__ x, const float *__restrict__ W, const float *__restrict__ dz,
    float *__restrict__ gW, float *__restrict__ gB, float *__restrict__ gin,
    const float *__restrict__ aux, int deriv, const float *__restrict__ cfac,
    float *__restrict__ gB_below, int B, int in, int C, float scale, const int32_t *__restrict__ parg,
    float *__restrict__ pgin, int pH, int pW, const float *__restrict__ xb, float *__restrict__ gWb,
    int inb) {
  constexpr int NW = NT / 64, RPW = TAIL_ROWS / NW, OPT = 64 * 64 / NT;  // OPT: staged x values per thread
  __shared__ float dzs[TAIL_ROWS * CM];
  __shared__ float part[NW / 2][CM + 1][64];  // the tree's upper halves (row CM: gin sums)
  extern __shared__ float gx_sh[];  // gWb: a chunk's gin rows [64][64], then its input rows [64][64]
  float *gsh = gx_sh, *xsh = gx_sh + 64 * 64;
  // gWb: blockIdx.y picks 64 input columns of the Dense below, whose weight
  // gradient gWb = scale gin^T xb the block sums for its 64 gin columns
  // (rows in order); the layer's own outputs come from the blocks of row 0
  const bool main_blk = blockIdx.y == 0;
  const int kc0 = blockIdx.y * 64;
  // waves 0-3 each own one 32 x 32 quarter of the 64 x 64 tile on fp32 MFMA
  // (v_mfma_f32_32x32x2f32: A[i = l%32][k = l/32], B[k = l/32][j = l%32];
  // result register r of lane l is row 8(r/4) + 4(l/32) + r%4, column l%32)
  typedef float tfx16 __attribute__((ext_vector_type(16)));
  tfx16 accb = tfx16{};
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int col = blockIdx.x * 64 + lane;
  const bool cok = col < in;
  const int cc = cok ? col : in - 1;
  const bool daux = gin && aux && deriv != D_ONE;
  float wcol[CM], acc[CM + 1];  // acc[CM]: this wave's sum of gin
#pragma unroll
  for (int o = 0; o < CM; ++o) {
    wcol[o] = o < C ? W[(size_t)o * in + cc] : 0.f;
    acc[o] = 0.f;
  }
  acc[CM] = 0.f;
  const float cf = cfac ? cfac[cc] : 1.0f;
  int pe0 = 0;  // POOL: flat index of the column's window corner in the pooled layer's input
  if (POOL) {
    const int ow = pW / 2, osz = (pH / 2) * ow;
    const int c = cc / osz, ph = (cc % osz) / ow, pw = cc % ow;
    pe0 = (c * pH + 2 * ph) * pW + 2 * pw;
  }
  for (int r0 = 0; r0 < B; r0 += TAIL_ROWS) {
    const int nr = min(TAIL_ROWS, B - r0);
    __syncthreads();
    for (int i = t; i < TAIL_ROWS * CM; i += NT) {
      const int r = i / CM, o = i % CM;
      dzs[i] = r < nr && o < C ? dz[(size_t)(r0 + r) * C + o] : 0.f;
    }
    __syncthreads();
    float xv[RPW], av[RPW];
    int am[RPW];
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int rr = w * RPW + q;
      const int r = r0 + min(rr, nr - 1);
      xv[q] = x[(size_t)r * in + cc];
      av[q] = daux ? aux[(size_t)r * in + cc] : 0.f;
      am[q] = POOL ? parg[(size_t)r * in + cc] : 0;
    }
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int rr = w * RPW + q;
      if (rr >= nr) break;
      const float *dr = dzs + rr * CM;
      float sd = 0.f;
#pragma unroll
      for (int o = 0; o < CM; ++o) {
        const float dv = dr[o];
        acc[o] += dv * xv[q];
        sd += dv * wcol[o];
      }
      if (gin || POOL) {
        float g = sd;
        if (aux) {  // the dX GEMM's EPI_DACT epilogue
          if (cfac) g = g * cf;
          g = deriv == D_ONE ? g * 1.0f : g * deriv_of(av[q], deriv);
        } else {
          g = g * 1.0f;  // EPI_SCALE with alpha 1
        }
        if (gWb) gsh[rr * 64 + lane] = g;
        if (!main_blk) {
        } else if (POOL) {
          if (cok) {
            float *dst = pgin + (size_t)(r0 + rr) * 4 * in;
#pragma unroll
            for (int dy = 0; dy < 2; ++dy)
#pragma unroll
              for (int dx = 0; dx < 2; ++dx) {
                const int e = pe0 + dy * pW + dx;
                dst[e] = am[q] == e ? g : 0.0f;
              }
          }
        } else if (cok) {
          gin[(size_t)(r0 + rr) * in + col] = g;
        }
        acc[CM] += g;
      }
    }
    if (gWb) {  // this chunk's rows of gin^T xb for the block's 64 x 64 tile
      if (nr & 1) gsh[nr * 64 + (t & 63)] = 0.f;  // the odd last row's MFMA partner
      __syncthreads();
      float xr[OPT];
#pragma unroll
      for (int o = 0; o < OPT; ++o) {
        const int e = t + o * NT, rr = e >> 6, kk = e & 63;
        xr[o] = rr < nr && kc0 + kk < inb ? xb[(size_t)(r0 + rr) * inb + kc0 + kk] : 0.f;
      }
#pragma unroll
      for (int o = 0; o < OPT; ++o) xsh[t + o * NT] = xr[o];
      __syncthreads();
      if (w < 4) {  // rows past nr hold zeros on both sides
        const int jt = w >> 1, kt = w & 1;
        for (int rr = 0; rr < nr; rr += 2) {
          const int r = rr + (lane >> 5);
          const float a = gsh[r * 64 + 32 * jt + (lane & 31)];
          const float b = xsh[r * 64 + 32 * kt + (lane & 31)];
          accb = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, accb, 0, 0, 0);
        }
      }
    }
  }
  if (gWb && w < 4) {
    const int jt = w >> 1, kt = w & 1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = blockIdx.x * 64 + 32 * jt + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      const int kk = kc0 + 32 * kt + (lane & 31);
      if (j < in && kk < inb) gWb[(size_t)j * inb + kk] = accb[r] * scale;
    }
  }
  if (!main_blk) return;
  // wave w adds wave w + h's sums, h = 8, 4, 2, 1
#pragma unroll
  for (int h = NW / 2; h >= 1; h >>= 1) {
    __syncthreads();
    if (w >= h && w < 2 * h) {
#pragma unroll
      for (int o = 0; o <= CM; ++o) part[w - h][o][lane] = acc[o];
    }
    __syncthreads();
    if (w < h) {
#pragma unroll
      for (int o = 0; o <= CM; ++o) acc[o] += part[w][o][lane];
    }
  }
  if (w == 0 && cok) {
#pragma unroll
    for (int o = 0; o < CM; ++o)
      if (o < C) gW[(size_t)o * in + col] = acc[o] * scale;
    if (gB_below) gB_below[col] = acc[CM] * scale;
  }
  if (gB && blockIdx.x == 0) {  // NT / 32 row ranges per output, added in order
    constexpr int P = NT / TAIL_MAXC;
    __syncthreads();
    float *bs = &part[0][0][0];
    const int per = (B + P - 1) / P;
    if (t < P * C) {
      const int o = t % C, q = t / C;
      float s = 0.f;
      for (int r = q * per; r < min(B, (q + 1) * per); ++r) s += dz[(size_t)r * C + o];
      bs[q * TAIL_MAXC + o] = s;
    }
    __syncthreads();
    if (t < C) {
      float s = bs[t];
      for (int q = 1; q < P; ++q) s += bs[q * TAIL_MAXC + t];
      gB[t] = s * scale;
    }
  }
}

bool tail_supported(int C, int in) { return C >= 1 && C <= TAIL_MAXC && in >= 1 && in % 4 == 0; }

hipError_t launch_tail_fwd(const float *x, const float *W, const float *bias, const float *y, float *out,
                           float *dz, float *loss_rows, int B, int in, int C, int row_act, int deriv,
                           int loss_kind, const int32_t *bad, int workers, hipStream_t s, const TailSplitIn &sp) {
  if (B <= 0) return hipSuccess;
  if (!tail_supported(C, in) || (reinterpret_cast<uintptr_t>(W) & 15) ||
      (!sp.ws && (reinterpret_cast<uintptr_t>(x) & 15)))
    return hipErrorInvalidValue;
  const int fwd = row_act >> 8;
  const int Wk = workers < 1 ? 1 : (workers > B ? B : workers);
  const int chunk = workers > 1 ? (B + Wk - 1) / Wk : 0;
  const int rb = C <= 4 ? 16 : C <= 16 ? 4 : 2;
  const size_t lds = sp.ws ? (size_t)rb * in * sizeof(float) : 0;
  if (lds > 65536 || (sp.ws && (!sp.bias || !sp.xo || (sp.dout && !sp.mask) || sp.splits < 1)))
    return hipErrorInvalidValue;
  if (C <= 4)
    hipLaunchKernelGGL((tail_fwd_kernel<4, 16, 512>), dim3((B + 15) / 16), dim3(512), lds, s, x, W, bias, y, out,
                       dz, loss_rows, B, in, C, row_act & 0xff, fwd, deriv, loss_kind, bad, chunk, sp);
  else if (C <= 16)
    hipLaunchKernelGGL((tail_fwd_kernel<16, 4, 512>), dim3((B + 3) / 4), dim3(512), lds, s, x, W, bias, y, out,
                       dz, loss_rows, B, in, C, row_act & 0xff, fwd, deriv, loss_kind, bad, chunk, sp);
  else
    hipLaunchKernelGGL((tail_fwd_kernel<32, 2, 512>), dim3((B + 1) / 2), dim3(512), lds, s, x, W, bias, y, out,
                       dz, loss_rows, B, in, C, row_act & 0xff, fwd, deriv, loss_kind, bad, chunk, sp);
  return hipGetLastError();
}

hipError_t launch_tail_bwd(const float *x, const float *W, const float *dz, float *gW, float *gB, float *gin,
                           const float *aux, int deriv, const float *cfac, float *gB_below, int B, int in,
                           int C, float scale, hipStream_t s, const int32_t *pool_arg, float *pool_gin, int pH,
                           int pW, const float *xb, float *gWb, int inb) {
  if (B <= 0) return hipSuccess;
  if (!tail_supported(C, in)) return hipErrorInvalidValue;
  const bool pool = pool_gin != nullptr;
  if (pool && (!pool_arg || aux || cfac || gB_below || pH < 2 || pW < 2 || pH % 2 || pW % 2 ||
               in % ((pH / 2) * (pW / 2)) != 0))
    return hipErrorInvalidValue;
  if (gWb && (!xb || inb < 1 || pool || !gin)) return hipErrorInvalidValue;
  const dim3 g((in + 63) / 64, gWb ? (inb + 63) / 64 : 1);
  const size_t lds = gWb ? 2 * 64 * 64 * sizeof(float) : 0;
#define TAIL_BWD(CM_, NT_, P_)                                                                                    \
  hipLaunchKernelGGL((tail_bwd_kernel<CM_, NT_, P_>), g, dim3(NT_), lds, s, x, W, dz, gW, gB, gin, aux, deriv,   \
                     cfac, gB_below, B, in, C, scale, pool_arg, pool_gin, pH, pW, xb, gWb, inb)
  if (pool) {
    if (C <= 4) TAIL_BWD(4, 512, true);
    else if (C <= 16) TAIL_BWD(16, 512, true);
    else TAIL_BWD(32, 512, true);
  } else {
    if (C <= 4) TAIL_BWD(4, 1024, false);
    else if (C <= 16) TAIL_BWD(16, 512, false);
    else TAIL_BWD(32, 512, false);
  }
#undef TAIL_BWD
  return hipGetLastError();
}

__global__ __launch_bounds__(TPB) void dropout_mask_kernel(float *__restrict__ mask, int n, float p) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t s = lcg_jump(42, (uint64_t)i + 1);
  const float u = (float)(s >> 33) / (float)(1u << 31);
  mask[i] = u < p ? 0.0f : 1.0f;
}

hipError_t launch_dropout_mask(float *mask, int n, float p, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(dropout_mask_kernel, dim3((n + TPB - 1) / TPB), dim3(TPB), 0, s, mask, n, p);
  return hipGetLastError();
}

// out = ((r + p[0]) + p[1]) + p[2], p[j] = p0 + j * pstride: three products
// added to a residual gradient in the order three accumulating launches
// would add them.
__global__ __launch_bounds__(TPB) void add3_kernel(const float *__restrict__ r, const float *__restrict__ p,
                                                   int64_t pstride, float *__restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v = r[i] + p[i];
    v = p[pstride + i] + v;
    out[i] = p[2 * pstride + i] + v;
  }
}

hipError_t launch_add3(const float *r, const float *p, int64_t pstride, float *out, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + TPB - 1) / TPB;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(add3_kernel, dim3((unsigned)blocks), dim3(TPB), 0, s, r, p, pstride, out, n);
  return hipGetLastError();
}

// dst[0, n) = v (a kernel, not a memset node: usable inside a captured graph)
__global__ __launch_bounds__(TPB) void fill_kernel(float *__restrict__ dst, float v, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = v;
}

hipError_t launch_fill(float *dst, float v, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + TPB - 1) / TPB;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(TPB), 0, s, dst, v, n);
  return hipGetLastError();
}

__global__ __launch_bounds__(1024) void row_act_kernel(float *__restrict__ x, int C, int row_act,
                                                       int fwd) {
  __shared__ float sh[16];
  row_activate(x + (size_t)blockIdx.x * C, C, row_act, fwd, sh);
}

// A hidden Softmax / LogSoftmax Dense's dz from the gradient g of its output
// o (layer.go:504-560), per row, g and dz may alias:
//   Softmax    dz_k = sum_i g_i o_i (d_ik - o_k) = g_k o_k - o_k sum_i g_i o_i
//   LogSoftmax dz_k = sum_i g_i (d_ik - exp(o_k)) = g_k - exp(o_k) sum_i g_i
__global__ __launch_bounds__(1024) void row_jac_kernel(const float *g, const float *__restrict__ o,
                                                       float *dz, int C, int row_act) {
  __shared__ float sh[16];
  const int t = threadIdx.x, nt = blockDim.x;
  const size_t off = (size_t)blockIdx.x * C;
  g += off;
  o += off;
  dz += off;
  float s1 = 0.f;
  if (row_act == ROW_SOFTMAX)
    for (int i = t; i < C; i += nt) s1 += g[i] * o[i];
  else
    for (int i = t; i < C; i += nt) s1 += g[i];
  s1 = block_sum(s1, sh);
  if (row_act == ROW_SOFTMAX)
    for (int i = t; i < C; i += nt) dz[i] = g[i] * o[i] - o[i] * s1;
  else
    for (int i = t; i < C; i += nt) dz[i] = g[i] - (float)exp((double)o[i]) * s1;
}

hipError_t launch_row_jac(const float *g, const float *out, float *dz, int B, int C, int row_act,
                          hipStream_t s) {
  row_act &= 0xff;
  if (B <= 0) return hipSuccess;
  if (row_act != ROW_SOFTMAX && row_act != ROW_LOGSOFTMAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(row_jac_kernel, dim3(B), dim3(row_threads(C)), 0, s, g, out, dz, C, row_act);
  return hipGetLastError();
}

hipError_t launch_row_act(float *out, int B, int C, int row_act, hipStream_t s) {
  if (B <= 0 || (row_act & 0xff) == ROW_NONE) return hipSuccess;
  hipLaunchKernelGGL(row_act_kernel, dim3(B), dim3(row_threads(C)), 0, s, out, C, row_act & 0xff,
                     row_act >> 8);
  return hipGetLastError();
}

// Dropout with the per-feature mask of Q9 (dropout.go:138-150 forward,
// :283-290 backward): out = mask ? x*scale : 0.
__global__ __launch_bounds__(TPB) void dropout_kernel(const float *__restrict__ x,
                                                      const float *__restrict__ mask, float scale,
                                                      float *__restrict__ out, int64_t total,
                                                      int n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float mk = mask[i % n];
    out[i] = mk > 0.f ? x[i] * scale : 0.0f;
  }
}

hipError_t launch_dropout(const float *x, const float *mask, float scale, float *out, int B, int n,
                          hipStream_t s) {
  const int64_t total = (int64_t)B * n;
  if (total <= 0) return hipSuccess;
  int64_t blocks = (total + TPB - 1) / TPB;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(dropout_kernel, dim3((unsigned)blocks), dim3(TPB), 0, s, x, mask, scale, out,
                     total, n);
  return hipGetLastError();
}

// SwiGLU gating (swiglu.go:165-171 forward, :206-216 backward) on the
// projections Z = [gate | up] of each row (2*out wide, from one GEMM against
// the parameter block [W | V]): y = (g sig(g)) u with sig(g) = 1/(1 +
// float32(exp(float64(-g)))); dUp = dy swish, dGate = dy (swish + sig (1 -
// swish)) u, written back as dZ = [dGate | dUp] for the parameter and input GEMMs.
__device__ __forceinline__ float swiglu_sig(float g) { return 1.0f / (1.0f + (float)exp((double)(-g))); }

__global__ __launch_bounds__(TPB) void swiglu_fwd_kernel(const float *__restrict__ Z,
                                                         float *__restrict__ y, int64_t total,
                                                         int out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / out;
    const int o = (int)(i - r * out);
    const float g = Z[r * 2 * out + o], u = Z[r * 2 * out + out + o];
    y[i] = (g * swiglu_sig(g)) * u;
  }
}

__global__ __launch_bounds__(TPB) void swiglu_bwd_kernel(const float *__restrict__ dy,
                                                         const float *__restrict__ Z, int64_t ldz,
                                                         float *__restrict__ dZ, int64_t total,
                                                         int out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / out;
    const int o = (int)(i - r * out);
    const float g = Z[r * ldz + o], u = Z[r * ldz + out + o];
    const float sig = swiglu_sig(g), swish = g * sig;
    dZ[r * 2 * out + out + o] = dy[i] * swish;
    const float dswish = swish + sig * (1.0f - swish);
    dZ[r * 2 * out + o] = dy[i] * dswish * u;
  }
}

hipError_t launch_swiglu_fwd(const float *Z, float *y, int B, int out, hipStream_t s) {
  const int64_t total = (int64_t)B * out;
  if (total <= 0) return hipSuccess;
  int64_t blocks = (total + TPB - 1) / TPB;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(swiglu_fwd_kernel, dim3((unsigned)blocks), dim3(TPB), 0, s, Z, y, total, out);
  return hipGetLastError();
}

hipError_t launch_swiglu_bwd(const float *dy, const float *Z, int ldz, float *dZ, int B, int out,
                             hipStream_t s) {
  const int64_t total = (int64_t)B * out;
  if (total <= 0) return hipSuccess;
  int64_t blocks = (total + TPB - 1) / TPB;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3((unsigned)blocks), dim3(TPB), 0, s, dy, Z, (int64_t)ldz,
                     dZ, total, out);
  return hipGetLastError();
}

}  // namespace gn
