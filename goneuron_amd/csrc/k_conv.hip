// Conv2D and MaxPool2D kernels (NCHW per sample, samples contiguous).
//
// Conv2D forward reproduces the reference's float32 summation order exactly so
// that pre-activations -- and the MaxPool argmax switches computed from them --
// are bit-identical to the per-sample CPU path:
//   k3 s1 p1 (conv2D3x3Optimized, conv2d.go:224-360): interior positions add,
//     per input channel, three row sums ((w0*a + w1*b) + w2*c); columns 0 and
//     W-1 of interior rows are never accumulated (pre = bias there, Q7); the
//     first and last rows add tap by tap with bounds checks; bias last.
//   other shapes (generic loop, conv2d.go:875-921): taps in (ic, kh, kw) order.
// MaxPool2D forward (maxpool2d.go:186-219): strict '>' scan of the window in
// (kh, kw) order from -Inf; the argmax is the flat index inside the sample.
// MaxPool2D backward (maxpool2d.go:392-408) is done as a gather: every input
// element sums the gradients of the windows whose argmax points at it, in
// increasing output position -- the order the reference's scatter adds them.
// Conv2D weight/bias gradients are an implicit GEMM over (sample, position)
// reduced per block and then across blocks in a fixed order.  The input
// gradient (the transposed convolution of conv2d.go:1117-1168) is an implicit
// GEMM over (oc, kh, kw) for stride 1, a per-element gather otherwise.
#include "gn_common.h"

#include <algorithm>

namespace gn {

constexpr int CT = 256;

__device__ __forceinline__ float act_fwd(float v, int kind) {
  switch (kind) {
    case F_RELU: return v > 0.0f ? v : 0.0f;
    case F_SIGMOID: return 1.0f / (1.0f + (float)exp((double)(-v)));
    case F_TANH: return (float)tanh((double)v);
    case F_NAN: return __builtin_nanf("");
    default: return v;
  }
}

__device__ __forceinline__ float act_deriv(float out, int kind) {
  switch (kind) {
    case D_RELU: return out > 0.0f ? 1.0f : 0.0f;
    case D_SIGMOID: return out * (1.0f - out);
    case D_TANH: return 1.0f - out * out;
    case D_NAN: return __builtin_nanf("");
    default: return 1.0f;
  }
}

__global__ __launch_bounds__(CT) void conv2d_fwd_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ w,
                                                        const float *__restrict__ bias,
                                                        float *__restrict__ out, ConvShape s,
                                                        int B, int fwd) {
  // blockIdx.y = b * outC + oc: one output plane, threads over its positions
  const int osz = s.oH * s.oW;
  const int plane = blockIdx.y;
  const int oc = plane % s.outC, b = plane / s.outC;
  const int H = s.H, W = s.W;
  const float *xs = x + (int64_t)b * s.inC * H * W;
  const float *wo = w + (int64_t)oc * s.inC * s.k * s.k;
  for (int pos = blockIdx.x * CT + threadIdx.x; pos < osz; pos += gridDim.x * CT) {
    const int oh = pos / s.oW, ow = pos - oh * s.oW;
    const int64_t idx = (int64_t)plane * osz + pos;
    float p = 0.0f;
    const bool fast = (s.k == 3 && s.stride == 1 && s.pad == 1);
    if (fast && oh >= 1 && oh < s.oH - 1) {
      if (ow >= 1 && ow < s.oW - 1) {
        for (int ic = 0; ic < s.inC; ++ic) {
          const float *wk = wo + ic * 9;
          const float *top = xs + ic * H * W + (oh - 1) * W + ow;
          const float *mid = top + W, *bot = mid + W;
          p += wk[0] * top[-1] + wk[1] * top[0] + wk[2] * top[1];
          p += wk[3] * mid[-1] + wk[4] * mid[0] + wk[5] * mid[1];
          p += wk[6] * bot[-1] + wk[7] * bot[0] + wk[8] * bot[1];
        }
      }  // else: Q7, the interior-row edge columns keep 0
    } else {
      for (int ic = 0; ic < s.inC; ++ic)
        for (int kh = 0; kh < s.k; ++kh) {
          const int ih = oh * s.stride + kh - s.pad;
          if (ih < 0 || ih >= H) continue;
          for (int kw = 0; kw < s.k; ++kw) {
            const int iw = ow * s.stride + kw - s.pad;
            if (iw < 0 || iw >= W) continue;
            p += wo[(ic * s.k + kh) * s.k + kw] * xs[(ic * H + ih) * W + iw];
          }
        }
    }
    out[idx] = act_fwd(p + bias[oc], fwd);
  }
}

__global__ __launch_bounds__(CT) void maxpool_fwd_kernel(const float *__restrict__ x,
                                                         float *__restrict__ out,
                                                         int32_t *__restrict__ argmax,
                                                         PoolShape s, int B) {
  const int osz = s.oH * s.oW;
  const int64_t total = (int64_t)B * s.C * osz;
  const int in_len = s.C * s.H * s.W;
  for (int64_t idx = (int64_t)blockIdx.x * CT + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * CT) {
    const int pos = (int)(idx % osz);
    const int c = (int)((idx / osz) % s.C);
    const int b = (int)(idx / ((int64_t)osz * s.C));
    const int oh = pos / s.oW, ow = pos % s.oW;
    const float *xs = x + (int64_t)b * in_len;
    float mv = -__builtin_inff();
    int mi = -1;
    for (int kh = 0; kh < s.k; ++kh)
      for (int kw = 0; kw < s.k; ++kw) {
        const int ih = oh * s.stride + kh - s.pad, iw = ow * s.stride + kw - s.pad;
        if (ih >= 0 && ih < s.H && iw >= 0 && iw < s.W) {
          const int i = (c * s.H + ih) * s.W + iw;
          const float v = xs[i];
          if (v > mv) {
            mv = v;
            mi = i;
          }
        }
      }
    out[idx] = mv;
    argmax[idx] = mi;
  }
}

// gin[b, i] = sum over output positions whose window holds input i and whose
// argmax == i, visited in increasing output position.  Block = one (sample,
// channel) plane, so a thread derives (ih, iw) with a single division.
__global__ __launch_bounds__(CT) void maxpool_bwd_kernel(const float *__restrict__ gout,
                                                         const int32_t *__restrict__ argmax,
                                                         float *__restrict__ gin, PoolShape s) {
  const int plane = blockIdx.x;  // b * C + c
  const int c = plane % s.C;
  const int hw = s.H * s.W, osz = s.oH * s.oW;
  const int64_t ob = (int64_t)plane * osz;
  const int ibase = c * hw;      // flat index of the plane inside its sample
  for (int e = threadIdx.x; e < hw; e += CT) {
    const int ih = e / s.W, iw = e - ih * s.W;
    const int i = ibase + e;
    // output rows/cols whose window covers (ih, iw)
    int oh0 = ih + s.pad - s.k + 1, oh1 = ih + s.pad;
    int ow0 = iw + s.pad - s.k + 1, ow1 = iw + s.pad;
    oh0 = oh0 <= 0 ? 0 : (oh0 + s.stride - 1) / s.stride;
    ow0 = ow0 <= 0 ? 0 : (ow0 + s.stride - 1) / s.stride;
    oh1 = min(oh1 / s.stride, s.oH - 1);
    ow1 = min(ow1 / s.stride, s.oW - 1);
    float g = 0.0f;
    for (int oh = oh0; oh <= oh1; ++oh)
      for (int ow = ow0; ow <= ow1; ++ow) {
        const int64_t o = ob + oh * s.oW + ow;
        if (argmax[o] == i) g += gout[o];
      }
    gin[(int64_t)plane * hw + e] = g;
  }
}

// Windows that tile the plane exactly (stride == k, no padding, H and W
// multiples of k): every input lies in one window, so a thread per window
// writes its k x k inputs: the window's gradient where the argmax points,
// 0 elsewhere (the same values as the gather above).
__global__ __launch_bounds__(CT) void maxpool_bwd_tiled_kernel(const float *__restrict__ gout,
                                                               const int32_t *__restrict__ argmax,
                                                               float *__restrict__ gin, PoolShape s,
                                                               int64_t n) {
  const int64_t o = (int64_t)blockIdx.x * CT + threadIdx.x;
  if (o >= n) return;
  const int osz = s.oH * s.oW;
  const int64_t plane = o / osz;  // b * C + c
  const int pos = (int)(o - plane * osz), oh = pos / s.oW, ow = pos - oh * s.oW;
  const int c = (int)(plane % s.C);
  const int am = argmax[o];
  const float g = gout[o];
  float *gp = gin + plane * s.H * s.W;
  for (int kh = 0; kh < s.k; ++kh) {
    const int ih = oh * s.k + kh;
    const int rowi = (c * s.H + ih) * s.W;  // flat index inside the sample
    if (s.k == 2) {
      const int iw = ow * 2;
      float2 v;
      v.x = am == rowi + iw ? g : 0.0f;
      v.y = am == rowi + iw + 1 ? g : 0.0f;
      *reinterpret_cast<float2 *>(gp + ih * s.W + iw) = v;
    } else {
      for (int kw = 0; kw < s.k; ++kw) {
        const int iw = ow * s.k + kw;
        gp[ih * s.W + iw] = am == rowi + iw ? g : 0.0f;
      }
    }
  }
}

// Conv2D weight + bias gradient partials.  Block (b, band): positions of one
// band of output rows of one sample; dz = gout * act'(out) is formed on the
// fly.  Output slot o < outC*inC*k*k is dW (oc, ic, kh, kw), the last outC
// slots are db.  part[block][slot] = sum over the band's positions.
__global__ __launch_bounds__(CT) void conv2d_wgrad_partial(const float *__restrict__ x,
                                                           const float *__restrict__ gout,
                                                           const float *__restrict__ out,
                                                           float *__restrict__ part, ConvShape s,
                                                           int band_rows, int deriv) {
  extern __shared__ float sm[];
  const int bands = (s.oH + band_rows - 1) / band_rows;
  const int b = blockIdx.x / bands, band = blockIdx.x % bands;
  const int oh0 = band * band_rows, oh1 = min(s.oH, oh0 + band_rows);
  const int rows = oh1 - oh0;
  const int P = rows * s.oW;
  const int osz = s.oH * s.oW;
  // dz tile [outC][P]
  float *dz = sm;
  for (int e = threadIdx.x; e < s.outC * P; e += CT) {
    const int oc = e / P, q = e % P;
    const int64_t gi = ((int64_t)b * s.outC + oc) * osz + oh0 * s.oW + q;
    dz[e] = gout[gi] * act_deriv(out[gi], deriv);
  }
  __syncthreads();
  const int nw = s.outC * s.inC * s.k * s.k;
  const int nslots = nw + s.outC;
  const float *xs = x + (int64_t)b * s.inC * s.H * s.W;
  for (int o = threadIdx.x; o < nslots; o += CT) {
    float acc = 0.0f;
    if (o < nw) {
      const int kw = o % s.k, kh = (o / s.k) % s.k, ic = (o / (s.k * s.k)) % s.inC,
                oc = o / (s.k * s.k * s.inC);
      const float *dzo = dz + oc * P;
      for (int r = 0; r < rows; ++r) {
        const int ih = (oh0 + r) * s.stride + kh - s.pad;
        if (ih < 0 || ih >= s.H) continue;
        const float *xr = xs + (ic * s.H + ih) * s.W;
        for (int ow = 0; ow < s.oW; ++ow) {
          const int iw = ow * s.stride + kw - s.pad;
          if (iw < 0 || iw >= s.W) continue;
          acc += dzo[r * s.oW + ow] * xr[iw];
        }
      }
    } else {
      const float *dzo = dz + (o - nw) * P;
      for (int q = 0; q < P; ++q) acc += dzo[q];
    }
    part[(int64_t)blockIdx.x * nslots + o] = acc;
  }
}

// The same partials on fp32 MFMA: per block an implicit GEMM
//   part[oc][tap] = sum_pos dz[oc][pos] * xcol[pos][tap],
// tap = (ic, kh, kw) plus one all-ones column that yields the bias gradient.
// dz and the block's input rows (zero padded by `pad` on every side) sit in
// LDS; each of the 4 waves takes a quarter of the positions and the waves'
// 16 x 32 results are added in LDS in wave order.
typedef float cfx16 __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(CT) void conv2d_wgrad_mfma(const float *__restrict__ x,
                                                        const float *__restrict__ gout,
                                                        const float *__restrict__ out,
                                                        float *__restrict__ part, ConvShape s,
                                                        int band_rows, int deriv) {
  extern __shared__ float sm[];
  const int bands = (s.oH + band_rows - 1) / band_rows;
  const int b = blockIdx.x / bands, band = blockIdx.x % bands;
  const int oh0 = band * band_rows, oh1 = min(s.oH, oh0 + band_rows);
  const int P = (oh1 - oh0) * s.oW;
  const int Pp = (P + 3) & ~3;  // whole 4-position MFMA steps
  const int osz = s.oH * s.oW;
  const int Rin = (band_rows - 1) * s.stride + s.k;  // input rows one band touches
  const int Wp = s.W + 2 * s.pad;
  // dz [Pp][ocs], ocs = outC rounded up to odd: the 32 lanes of an MFMA
  // operand read read consecutive channels of one position, and the staging
  // writes (consecutive positions) fall in distinct banks
  const int ocs = s.outC | 1;
  float *dz = sm;
  float *xb = dz + ocs * Pp;                         // [inC][Rin][Wp]
  int *poff = reinterpret_cast<int *>(xb + s.inC * Rin * Wp);  // [Pp] LDS offset of a position
  float *red = reinterpret_cast<float *>(poff + Pp);           // [4][32*32]
  // staged 8 elements per thread at a time, every load issued before the
  // first is used (a load per iteration waited out its own round trip)
  // (a thread per position, channels in groups: no index divisions)
  constexpr int SU = 8;
  for (int q = threadIdx.x; q < Pp; q += CT) {
    const bool qv = q < P;
    const int64_t base = (int64_t)b * s.outC * osz + oh0 * s.oW + q;
    for (int oc0 = 0; oc0 < s.outC; oc0 += SU) {
      float gv[SU], ov[SU];
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const bool ld = qv && oc0 + u < s.outC;
        const int64_t gi = base + (int64_t)(oc0 + u) * osz;
        gv[u] = ld ? gout[gi] : 0.f;
        ov[u] = ld ? out[gi] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < SU; ++u)
        if (oc0 + u < s.outC) dz[q * ocs + oc0 + u] = qv ? gv[u] * act_deriv(ov[u], deriv) : 0.f;
    }
  }
  const int ih0 = oh0 * s.stride - s.pad;
  const float *xs = x + (int64_t)b * s.inC * s.H * s.W;
  const int nxb = s.inC * Rin * Wp;
  for (int e0 = threadIdx.x; e0 < nxb; e0 += CT * SU) {
    float xv[SU];
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int e = e0 + u * CT;
      const int c = e % Wp, r = (e / Wp) % Rin, ic = e / (Wp * Rin);
      const int ih = ih0 + r, iw = c - s.pad;
      xv[u] = e < nxb && ih >= 0 && ih < s.H && iw >= 0 && iw < s.W ? xs[(ic * s.H + ih) * s.W + iw] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < SU; ++u)
      if (e0 + u * CT < nxb) xb[e0 + u * CT] = xv[u];
  }
  for (int q = threadIdx.x; q < Pp; q += CT)
    poff[q] = q < P ? (q / s.oW) * s.stride * Wp + (q % s.oW) * s.stride : 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ntap = s.inC * s.k * s.k;
  const int nw = s.outC * ntap, nslots = nw + s.outC;
  const int kq = ((Pp / 4 + 3) / 4) * 4;  // positions per wave (whole MFMA steps)
  const int kb = w * kq, ke = min(Pp, kb + kq);
  const int i16 = lane & 15, k4 = lane >> 4;
  // v_mfma_f32_16x16x4f32: A[i = l%16][k = l/16] (channel, position), B[k][j = l%16]
  // (position, tap; tap ntap is the all-ones bias column); result register r
  // of lane l is channel 4*(l/16) + r, tap l%16.  Two 16-wide tap tiles per
  // pass share the channel operand.
  for (int mt = 0; mt * 16 < s.outC; ++mt)
    for (int nt = 0; nt * 16 <= ntap; nt += 2) {
      const int oc = mt * 16 + i16;
      int toff[2];  // -1: zero column, -2: ones column (bias)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int tap = (nt + h) * 16 + i16;
        toff[h] = -1;
        if (tap < ntap) {
          const int kw = tap % s.k, kh = (tap / s.k) % s.k, ic = tap / (s.k * s.k);
          toff[h] = (ic * Rin + kh) * Wp + kw;
        } else if (tap == ntap) {
          toff[h] = -2;
        }
      }
      // 8 steps' operands read from LDS before their MFMAs, so the reads'
      // latencies overlap
      f4v acc0 = f4v{0.f, 0.f, 0.f, 0.f}, acc1 = f4v{0.f, 0.f, 0.f, 0.f};
      const int nst = (ke - kb) / 4;
      for (int s0 = 0; s0 < nst; s0 += 8) {
        float av[8], bv0[8], bv1[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool ok = s0 + u < nst;
          const int q = kb + 4 * (s0 + u) + k4;
          const int po = ok ? poff[q] : 0;
          av[u] = ok && oc < s.outC ? dz[q * ocs + oc] : 0.f;
          bv0[u] = !ok ? 0.f : toff[0] >= 0 ? xb[toff[0] + po] : (toff[0] == -2 && q < P ? 1.f : 0.f);
          bv1[u] = !ok ? 0.f : toff[1] >= 0 ? xb[toff[1] + po] : (toff[1] == -2 && q < P ? 1.f : 0.f);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv0[u], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv1[u], acc1, 0, 0, 0);
        }
      }
      // the 4 waves' 16 x 32 results added in LDS in wave order
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        red[w * 512 + (4 * k4 + r) * 32 + i16] = acc0[r];
        red[w * 512 + (4 * k4 + r) * 32 + 16 + i16] = acc1[r];
      }
      __syncthreads();
      for (int e = threadIdx.x; e < 512; e += CT) {
        const int o = mt * 16 + e / 32, t = nt * 16 + e % 32;
        const float v = (red[e] + red[512 + e]) + (red[1024 + e] + red[1536 + e]);
        if (o < s.outC && t < ntap) part[(int64_t)blockIdx.x * nslots + o * ntap + t] = v;
        else if (o < s.outC && t == ntap) part[(int64_t)blockIdx.x * nslots + nw + o] = v;
      }
      __syncthreads();
    }
}

// One wave per slot: lanes take the blocks, then a wave reduction.  With the
// step's update (ad.stride), each slot's gradient is updated by the lane that
// writes it, and blocks from nred on update ad.rest's ranges.
__global__ __launch_bounds__(CT) void conv2d_wgrad_reduce(const float *__restrict__ part,
                                                          int nblocks, int nslots, float scale,
                                                          float *__restrict__ grad, int nred,
                                                          AdamStep ad) {
  if ((int)blockIdx.x >= nred) {
    const int64_t step = (int64_t)(gridDim.x - nred) * CT;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float *g = ad.rest;
      for (int64_t i = ad.r0[r] + (int64_t)(blockIdx.x - nred) * CT + threadIdx.x; i < ad.r1[r]; i += step)
        adam_at(g + i, g[i], ad);
    }
    return;
  }
  const int lane = threadIdx.x & 63;
  const int o = blockIdx.x * (CT / 64) + (threadIdx.x >> 6);
  if (o >= nslots) return;
  float s = 0.f;
  for (int i = lane; i < nblocks; i += 8 * 64) {  // eight loads in flight, added in block order
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = i + 64 * u < nblocks ? part[(int64_t)(i + 64 * u) * nslots + o] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (i + 64 * u < nblocks) s += v[u];
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) s += __shfl_xor(s, d, 64);
  if (lane == 0) {  // grad = [dW | db], the Conv2D arena layout (conv2d.go:121-125)
    grad[o] = s * scale;
    if (ad.stride) adam_at(grad + o, s * scale, ad);
  }
}

// dX gather: gin[b, ic, ih, iw] = sum over (oc, kh, kw) of dz * w, dz formed
// from gout and the saved output.
__global__ __launch_bounds__(CT) void conv2d_dgrad_kernel(const float *__restrict__ gout,
                                                          const float *__restrict__ out,
                                                          const float *__restrict__ w,
                                                          float *__restrict__ gin, ConvShape s,
                                                          int B, int deriv) {
  const int in_len = s.inC * s.H * s.W;
  const int osz = s.oH * s.oW;
  const int64_t total = (int64_t)B * in_len;
  for (int64_t idx = (int64_t)blockIdx.x * CT + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * CT) {
    const int i = (int)(idx % in_len);
    const int b = (int)(idx / in_len);
    const int ic = i / (s.H * s.W), ih = (i / s.W) % s.H, iw = i % s.W;
    float g = 0.0f;
    for (int oc = 0; oc < s.outC; ++oc)
      for (int kh = 0; kh < s.k; ++kh) {
        const int t = ih + s.pad - kh;
        if (t < 0 || t % s.stride) continue;
        const int oh = t / s.stride;
        if (oh >= s.oH) continue;
        for (int kw = 0; kw < s.k; ++kw) {
          const int u = iw + s.pad - kw;
          if (u < 0 || u % s.stride) continue;
          const int ow = u / s.stride;
          if (ow >= s.oW) continue;
          const int64_t o = ((int64_t)b * s.outC + oc) * osz + oh * s.oW + ow;
          g += gout[o] * act_deriv(out[o], deriv) * w[((oc * s.inC + ic) * s.k + kh) * s.k + kw];
        }
      }
    gin[idx] = g;
  }
}

// Conv2D input gradient on fp32 MFMA for stride 1: an implicit GEMM per block
// (one sample, a band of input rows)
//   gin[ic][pos] = sum over tap = (oc, kh, kw) of W[oc][ic][kh][kw] * dzcol[tap][pos],
//   dzcol[(oc, kh, kw)][(ih, iw)] = dz[oc][ih + pad - kh][iw + pad - kw]
// (zero outside the output plane).  The band's dz rows with a k - 1 halo on
// each side (dz = gout * act'(out), zero padded) and W in tap-major order sit
// in LDS; each wave takes 32 x 32 (channel, position) tiles over the whole K,
// and the 32 lanes of a tile column store 32 consecutive positions of one
// input plane.
__global__ __launch_bounds__(CT) void conv2d_dgrad_mfma(const float *__restrict__ gout,
                                                        const float *__restrict__ out,
                                                        const float *__restrict__ w,
                                                        float *__restrict__ gin, ConvShape s,
                                                        int band_rows, int deriv) {
  extern __shared__ float sm[];
  const int bands = (s.H + band_rows - 1) / band_rows;
  const int b = blockIdx.x / bands, band = blockIdx.x % bands;
  const int ih0 = band * band_rows, R = min(s.H, ih0 + band_rows) - ih0;
  const int k = s.k, km = k - 1, kk = k * k;
  const int Rz = band_rows + km, Wz = s.W + km;
  const int ntap = s.outC * kk, ntp = (ntap + 7) & ~7;   // K padded with zero taps
  float *dzb = sm;                                         // [outC][Rz][Wz]
  float *wt = dzb + s.outC * Rz * Wz;                      // [ntp][inC]
  int *toff = reinterpret_cast<int *>(wt + ntp * s.inC);   // [ntp] LDS offset of a tap
  const int osz = s.oH * s.oW;
  const int oh0 = ih0 + s.pad - km, ow0 = s.pad - km;
  for (int e = threadIdx.x; e < s.outC * Rz * Wz; e += CT) {
    const int c = e % Wz, r = (e / Wz) % Rz, oc = e / (Wz * Rz);
    const int oh = oh0 + r, ow = ow0 + c;
    float v = 0.f;
    if (oh >= 0 && oh < s.oH && ow >= 0 && ow < s.oW) {
      const int64_t gi = ((int64_t)b * s.outC + oc) * osz + oh * s.oW + ow;
      v = gout[gi] * act_deriv(out[gi], deriv);
    }
    dzb[e] = v;
  }
  for (int e = threadIdx.x; e < ntp * s.inC; e += CT) {
    const int tap = e / s.inC, ic = e - tap * s.inC;
    float v = 0.f;
    if (tap < ntap) {
      const int oc = tap / kk, kh = (tap / k) % k, kw = tap % k;
      v = w[((oc * s.inC + ic) * k + kh) * k + kw];
    }
    wt[e] = v;
  }
  for (int t = threadIdx.x; t < ntp; t += CT) {
    int o = 0;
    if (t < ntap) {
      const int oc = t / kk, kh = (t / k) % k, kw = t % k;
      o = (oc * Rz + km - kh) * Wz + km - kw;
    }
    toff[t] = o;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int P = R * s.W;
  const int mtiles = (s.inC + 31) / 32, ntiles = (P + 31) / 32;
  const int64_t gbase = ((int64_t)b * s.inC * s.H + ih0) * s.W;  // (b, ic = 0, ih0, 0)
  for (int tile = wv; tile < mtiles * ntiles; tile += CT / 64) {
    const int mt = tile / ntiles, nt = tile - mt * ntiles;
    const int ic = mt * 32 + (lane & 31);
    const bool icv = ic < s.inC;
    const int pos = nt * 32 + (lane & 31);
    const int poff = pos < P ? (pos / s.W) * Wz + pos % s.W : 0;
    cfx16 acc = cfx16{};
    for (int q0 = 0; q0 < ntp; q0 += 8) {  // the operands of 4 MFMAs loaded ahead of them
      float a[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int q = q0 + 2 * u + (lane >> 5);
        a[u] = icv ? wt[q * s.inC + ic] : 0.f;
        bv[u] = dzb[toff[q] + poff];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u], bv[u], acc, 0, 0, 0);
    }
    if (pos < P) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < s.inC) gin[gbase + (int64_t)row * s.H * s.W + pos] = acc[r];
      }
    }
  }
}

// k3 s1 p1 with INC input channels (conv2D3x3Optimized): a thread per output
// position -- or per 2x2 quad of positions when a 2x2 / stride-2 MaxPool2D
// follows and tiles the plane -- and per group of OCG output channels.  The
// input window is read once into registers and serves every channel of the
// group; each output keeps conv2d_fwd_kernel's expressions, so the results
// are the same bit for bit.  With POOL the quad's four activations are
// scanned in (kh, kw) order with a strict '>' from -Inf (maxpool_fwd_kernel),
// writing the pooled value and its flat index inside the sample.
// the float64 activations out of line: inlined once per output they made
// the kernel ~12k instructions, fetched again by every wave
__device__ __noinline__ float act_fwd_call(float v, int kind) { return act_fwd(v, kind); }

template <int INC, int OCG, bool POOL>
__global__ __launch_bounds__(CT) void conv3_fwd_group_kernel(const float *__restrict__ x,
                                                             const float *__restrict__ w,
                                                             const float *__restrict__ bias,
                                                             float *__restrict__ out, ConvShape s, int B,
                                                             int fwd, float *__restrict__ pout,
                                                             int32_t *__restrict__ parg) {
  constexpr int Q = POOL ? 2 : 1;  // positions per side
  constexpr int R = Q + 2;         // window rows and columns
  const int H = s.H, W = s.W;      // = oH, oW
  const int qh = H / Q, qw = W / Q, per = qh * qw;
  const int groups = s.outC / OCG;
  // blockIdx.y = sample * groups + channel group: uniform, so the weights
  // and the bias come through scalar loads
  const int q = blockIdx.x * CT + threadIdx.x;
  if (q >= per) return;
  const int g = blockIdx.y % groups, b = blockIdx.y / groups;
  const int y0 = (q / qw) * Q, x0 = (q % qw) * Q;
  const float *xs = x + (int64_t)b * INC * H * W;
  // the window, zero outside the plane: clamped addresses and a select (no
  // branch around each load)
  float win[INC][R][R];
#pragma unroll
  for (int ic = 0; ic < INC; ++ic)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int c = 0; c < R; ++c) {
        const int ih = y0 - 1 + r, iw = x0 - 1 + c;
        const bool inb = ih >= 0 && ih < H && iw >= 0 && iw < W;
        const float v = xs[(ic * H + min(max(ih, 0), H - 1)) * W + min(max(iw, 0), W - 1)];
        win[ic][r][c] = inb ? v : 0.f;
      }
#pragma unroll 1
  for (int j = 0; j < OCG; ++j) {
    const int oc = g * OCG + j;
    const float *wk = w + oc * INC * 9;
    const float bo = bias[oc];
    float mv = -__builtin_inff();
    int mi = -1;
#pragma unroll
    for (int dy = 0; dy < Q; ++dy)
#pragma unroll
      for (int dx = 0; dx < Q; ++dx) {
        const int oh = y0 + dy, ow = x0 + dx;
        float p = 0.0f;
        if (oh >= 1 && oh < H - 1) {
#pragma unroll
          for (int ic = 0; ic < INC; ++ic) {
            const float *k9 = wk + ic * 9;
            p += k9[0] * win[ic][dy][dx] + k9[1] * win[ic][dy][dx + 1] + k9[2] * win[ic][dy][dx + 2];
            p += k9[3] * win[ic][dy + 1][dx] + k9[4] * win[ic][dy + 1][dx + 1] + k9[5] * win[ic][dy + 1][dx + 2];
            p += k9[6] * win[ic][dy + 2][dx] + k9[7] * win[ic][dy + 2][dx + 1] + k9[8] * win[ic][dy + 2][dx + 2];
          }
          if (ow < 1 || ow >= W - 1) p = 0.0f;  // Q7: the interior-row edge columns keep 0
        } else {  // first and last rows: taps in (ic, kh, kw) order, those outside skipped
#pragma unroll
          for (int ic = 0; ic < INC; ++ic)
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
              const int ih = oh + kh - 1;
#pragma unroll
              for (int kw = 0; kw < 3; ++kw) {
                const int iw = ow + kw - 1;
                const bool ok = ih >= 0 && ih < H && iw >= 0 && iw < W;
                const float t = p + wk[(ic * 3 + kh) * 3 + kw] * win[ic][dy + kh][dx + kw];
                p = ok ? t : p;
              }
            }
        }
        const float z = p + bo;
        const float v = fwd == F_RELU ? (z > 0.0f ? z : 0.0f) : fwd == F_IDENTITY ? z : act_fwd_call(z, fwd);
        const int e = (oc * H + oh) * W + ow;  // flat index inside the sample
        out[(int64_t)b * s.outC * H * W + e] = v;
        if (POOL && v > mv) {
          mv = v;
          mi = e;
        }
      }
    if (POOL) {
      const int64_t po = ((int64_t)b * s.outC + oc) * per + q;
      pout[po] = mv;
      parg[po] = mi;
    }
  }
}

template <int INC>
static hipError_t conv3_fwd_inc(const float *x, const float *w, const float *bias, float *out,
                                const ConvShape &s, int B, int fwd, float *pout, int32_t *parg,
                                hipStream_t st) {
  const bool pool = pout != nullptr;
  const int per = pool ? (s.H / 2) * (s.W / 2) : s.H * s.W;
  const int ocg = s.outC % 4 == 0 ? 4 : 1;
  const dim3 grid((per + CT - 1) / CT, B * (s.outC / ocg));
  if (pool && ocg == 4)
    hipLaunchKernelGGL((conv3_fwd_group_kernel<INC, 4, true>), dim3(grid), dim3(CT), 0, st, x, w, bias, out, s, B,
                       fwd, pout, parg);
  else if (pool)
    hipLaunchKernelGGL((conv3_fwd_group_kernel<INC, 1, true>), dim3(grid), dim3(CT), 0, st, x, w, bias, out, s, B,
                       fwd, pout, parg);
  else if (ocg == 4)
    hipLaunchKernelGGL((conv3_fwd_group_kernel<INC, 4, false>), dim3(grid), dim3(CT), 0, st, x, w, bias, out, s, B,
                       fwd, pout, parg);
  else
    hipLaunchKernelGGL((conv3_fwd_group_kernel<INC, 1, false>), dim3(grid), dim3(CT), 0, st, x, w, bias, out, s, B,
                       fwd, pout, parg);
  return hipGetLastError();
}

bool conv_fwd_pool_fusable(const ConvShape &s, const PoolShape &p, int B) {
  return (int64_t)B * s.outC <= 65535 && s.k == 3 && s.stride == 1 && s.pad == 1 && s.inC >= 1 && s.inC <= 4 && p.k == 2 && p.stride == 2 &&
         p.pad == 0 && p.C == s.outC && p.H == s.oH && p.W == s.oW && s.oH % 2 == 0 && s.oW % 2 == 0 &&
         p.oH == s.oH / 2 && p.oW == s.oW / 2 && (int64_t)s.outC * s.oH * s.oW < (1ll << 31);
}

static unsigned grid_for(int64_t n) {
  int64_t b = (n + CT - 1) / CT;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

hipError_t launch_conv_fwd(const float *x, const float *w, const float *bias, float *out,
                           const ConvShape &s, int B, int fwd, hipStream_t st, float *pool_out,
                           int32_t *pool_arg) {
  if (pool_out && !(pool_arg && s.k == 3 && s.stride == 1 && s.pad == 1 && s.inC <= 4 && s.oH % 2 == 0 &&
                    s.oW % 2 == 0))
    return hipErrorInvalidValue;
  if (s.k == 3 && s.stride == 1 && s.pad == 1 && s.inC >= 1 && s.inC <= 4 && s.oH == s.H && s.oW == s.W &&
      (int64_t)s.outC * s.oH * s.oW < (1ll << 31) && (int64_t)B * s.outC <= 65535) {
    switch (s.inC) {
      case 1: return conv3_fwd_inc<1>(x, w, bias, out, s, B, fwd, pool_out, pool_arg, st);
      case 2: return conv3_fwd_inc<2>(x, w, bias, out, s, B, fwd, pool_out, pool_arg, st);
      case 3: return conv3_fwd_inc<3>(x, w, bias, out, s, B, fwd, pool_out, pool_arg, st);
      default: return conv3_fwd_inc<4>(x, w, bias, out, s, B, fwd, pool_out, pool_arg, st);
    }
  }
  if (pool_out) return hipErrorInvalidValue;
  const int osz = s.oH * s.oW;
  const int gx = std::min((osz + CT - 1) / CT, 64);
  hipLaunchKernelGGL(conv2d_fwd_kernel, dim3(gx, B * s.outC), dim3(CT), 0, st, x, w, bias, out, s, B,
                     fwd);
  return hipGetLastError();
}

// AvgPool2D (avgpool2d.go:98-220, 401-474): count = in-bounds cells of the
// window (padding excluded), out = sum in (kh, kw) order * float32(1 / count).
__device__ __forceinline__ int avgpool_count(const PoolShape &s, int oh, int ow) {
  const int h0 = oh * s.stride - s.pad, w0 = ow * s.stride - s.pad;
  const int nh = min(h0 + s.k, s.H) - max(h0, 0), nw = min(w0 + s.k, s.W) - max(w0, 0);
  return (nh > 0 && nw > 0) ? nh * nw : 0;
}

__global__ __launch_bounds__(CT) void avgpool_fwd_kernel(const float *__restrict__ x,
                                                         float *__restrict__ out, PoolShape s,
                                                         int64_t n) {
  for (int64_t o = (int64_t)blockIdx.x * CT + threadIdx.x; o < n; o += (int64_t)gridDim.x * CT) {
    const int ow = (int)(o % s.oW), oh = (int)((o / s.oW) % s.oH);
    const int64_t plane = o / ((int64_t)s.oH * s.oW);  // b * C + c
    const float *xp = x + plane * s.H * s.W;
    const int count = avgpool_count(s, oh, ow);
    float v = 0.0f;
    if (count > 0) {
      float sum = 0.0f;
      for (int kh = 0; kh < s.k; ++kh) {
        const int ih = oh * s.stride + kh - s.pad;
        if (ih < 0 || ih >= s.H) continue;
        for (int kw = 0; kw < s.k; ++kw) {
          const int iw = ow * s.stride + kw - s.pad;
          if (iw >= 0 && iw < s.W) sum += xp[ih * s.W + iw];
        }
      }
      v = sum * (1.0f / (float)count);
    }
    out[o] = v;
  }
}

// Backward as a gather: input cell (ih, iw) adds g * float32(1 / count) of
// every window that holds it in increasing (oh, ow) order, the order in which
// the reference scatters them onto a zeroed gradient.  One block per plane.
__global__ __launch_bounds__(CT) void avgpool_bwd_kernel(const float *__restrict__ gout,
                                                         float *__restrict__ gin, PoolShape s) {
  const int64_t plane = blockIdx.x;
  const int hw = s.H * s.W, osz = s.oH * s.oW;
  const float *gp = gout + plane * osz;
  for (int e = threadIdx.x; e < hw; e += CT) {
    const int ih = e / s.W, iw = e - ih * s.W;
    int oh0 = ih + s.pad - s.k + 1, oh1 = ih + s.pad;
    int ow0 = iw + s.pad - s.k + 1, ow1 = iw + s.pad;
    oh0 = oh0 <= 0 ? 0 : (oh0 + s.stride - 1) / s.stride;
    ow0 = ow0 <= 0 ? 0 : (ow0 + s.stride - 1) / s.stride;
    oh1 = min(oh1 / s.stride, s.oH - 1);
    ow1 = min(ow1 / s.stride, s.oW - 1);
    float g = 0.0f;
    for (int oh = oh0; oh <= oh1; ++oh)
      for (int ow = ow0; ow <= ow1; ++ow) {
        const int count = avgpool_count(s, oh, ow);
        if (count > 0) g += gp[oh * s.oW + ow] * (1.0f / (float)count);
      }
    gin[plane * hw + e] = g;
  }
}

hipError_t launch_maxpool_fwd(const float *x, float *out, int32_t *argmax, const PoolShape &s,
                              int B, hipStream_t st) {
  const int64_t n = (int64_t)B * s.C * s.oH * s.oW;
  hipLaunchKernelGGL(maxpool_fwd_kernel, dim3(grid_for(n)), dim3(CT), 0, st, x, out, argmax, s, B);
  return hipGetLastError();
}

hipError_t launch_maxpool_bwd(const float *gout, const int32_t *argmax, float *gin,
                              const PoolShape &s, int B, hipStream_t st) {
  const bool tiled = s.stride == s.k && s.pad == 0 && s.H == s.oH * s.k && s.W == s.oW * s.k &&
                     (s.k != 2 || s.W % 2 == 0);
  if (tiled) {
    const int64_t n = (int64_t)B * s.C * s.oH * s.oW;
    hipLaunchKernelGGL(maxpool_bwd_tiled_kernel, dim3((unsigned)((n + CT - 1) / CT)), dim3(CT), 0, st,
                       gout, argmax, gin, s, n);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(maxpool_bwd_kernel, dim3(B * s.C), dim3(CT), 0, st, gout, argmax, gin, s);
  return hipGetLastError();
}

hipError_t launch_avgpool_fwd(const float *x, float *out, const PoolShape &s, int B, hipStream_t st) {
  const int64_t n = (int64_t)B * s.C * s.oH * s.oW;
  hipLaunchKernelGGL(avgpool_fwd_kernel, dim3(grid_for(n)), dim3(CT), 0, st, x, out, s, n);
  return hipGetLastError();
}

hipError_t launch_avgpool_bwd(const float *gout, float *gin, const PoolShape &s, int B, hipStream_t st) {
  hipLaunchKernelGGL(avgpool_bwd_kernel, dim3(B * s.C), dim3(CT), 0, st, gout, gin, s);
  return hipGetLastError();
}

hipError_t launch_conv_wgrad_reduce(const ConvWgradReduce &red, const AdamStep *upd, hipStream_t st) {
  AdamStep ad{};
  int extra = 0;
  if (upd) {
    ad = *upd;
    if (ad.stride <= 0) return hipErrorInvalidValue;
    int64_t n = 0;
    for (int r = 0; r < 2; ++r) {
      if (ad.r1[r] < ad.r0[r] || (ad.r1[r] > ad.r0[r] && !ad.rest)) return hipErrorInvalidValue;
      n += ad.r1[r] - ad.r0[r];
    }
    extra = (int)std::min<int64_t>((n + 4 * CT - 1) / (4 * CT), 1024);  // ~4 parameters per thread
  }
  const int nred = (red.nslots + 3) / 4;
  hipLaunchKernelGGL(conv2d_wgrad_reduce, dim3(nred + extra), dim3(CT), 0, st, red.ws, red.nblocks, red.nslots,
                     red.scale, red.grad, nred, ad);
  return hipGetLastError();
}

hipError_t launch_conv_wgrad(const float *x, const float *gout, const float *out, float *grad,
                             const ConvShape &s, int B, int deriv, float scale, float *ws,
                             size_t ws_cap, hipStream_t st, ConvWgradReduce *red) {
  const int nslots = s.outC * s.inC * s.k * s.k + s.outC;
  const int Wp = s.W + 2 * s.pad;
  // MFMA path: bands of output rows whose dz tile, input rows and tables fit
  // in 64 KiB of LDS
  auto mfma_lds = [&](int band) {
    const int P = band * s.oW, Pp = (P + 3) & ~3, Rin = (band - 1) * s.stride + s.k;
    return ((size_t)(s.outC | 1) * Pp + (size_t)s.inC * Rin * Wp + Pp + 4 * 1024) * sizeof(float);
  };
  int band = s.oH;
  while (band > 1 && mfma_lds(band) > 32768) band = (band + 1) / 2;
  if (mfma_lds(band) <= 65536) {
    const int bands = (s.oH + band - 1) / band;
    const int nblocks = B * bands;
    if ((size_t)nblocks * nslots > ws_cap) return hipErrorInvalidValue;
    hipLaunchKernelGGL(conv2d_wgrad_mfma, dim3(nblocks), dim3(CT), mfma_lds(band), st, x, gout, out,
                       ws, s, band, deriv);
    if (red) {
      *red = ConvWgradReduce{ws, nblocks, nslots, scale, grad};
      return hipGetLastError();
    }
    hipLaunchKernelGGL(conv2d_wgrad_reduce, dim3((nslots + 3) / 4), dim3(CT), 0, st, ws, nblocks,
                       nslots, scale, grad, (nslots + 3) / 4, AdamStep{});
    return hipGetLastError();
  }
  // scalar path for shapes whose input rows do not fit: dz tile <= 32 KiB
  band = s.oH;
  while (band > 1 && (size_t)s.outC * band * s.oW * sizeof(float) > 32768) band = (band + 1) / 2;
  const int bands = (s.oH + band - 1) / band;
  const int nblocks = B * bands;
  if ((size_t)nblocks * nslots > ws_cap) return hipErrorInvalidValue;
  const size_t shm = (size_t)s.outC * band * s.oW * sizeof(float);
  hipLaunchKernelGGL(conv2d_wgrad_partial, dim3(nblocks), dim3(CT), shm, st, x, gout, out, ws, s,
                     band, deriv);
  if (red) {
    *red = ConvWgradReduce{ws, nblocks, nslots, scale, grad};
    return hipGetLastError();
  }
  hipLaunchKernelGGL(conv2d_wgrad_reduce, dim3((nslots + 3) / 4), dim3(CT), 0, st, ws, nblocks,
                     nslots, scale, grad, (nslots + 3) / 4, AdamStep{});
  return hipGetLastError();
}

hipError_t launch_conv_dgrad(const float *gout, const float *out, const float *w, float *gin,
                             const ConvShape &s, int B, int deriv, hipStream_t st) {
  if (s.stride == 1) {  // MFMA implicit GEMM: bands of input rows, >= 4 blocks per CU
    const int km = s.k - 1, ntap = s.outC * s.k * s.k, ntp = (ntap + 7) & ~7;
    auto lds = [&](int band) {
      return ((size_t)s.outC * (band + km) * (s.W + km) + (size_t)ntp * s.inC + ntp) * sizeof(float);
    };
    int band = s.H;
    while (band > 1 && (lds(band) > 32768 || (int64_t)B * ((s.H + band - 1) / band) < 1024))
      band = (band + 1) / 2;
    if (lds(band) <= 65536) {
      const int64_t nblocks = (int64_t)B * ((s.H + band - 1) / band);
      if (nblocks > 0x7fffffff) return hipErrorInvalidValue;
      hipLaunchKernelGGL(conv2d_dgrad_mfma, dim3((unsigned)nblocks), dim3(CT), lds(band), st, gout, out,
                         w, gin, s, band, deriv);
      return hipGetLastError();
    }
  }
  // strided convolutions, and shapes whose band does not fit: per-element gather
  const int64_t n = (int64_t)B * s.inC * s.H * s.W;
  hipLaunchKernelGGL(conv2d_dgrad_kernel, dim3(grid_for(n)), dim3(CT), 0, st, gout, out, w, gin, s,
                     B, deriv);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// BatchNorm2D (batchnorm2d.go).  In the per-sample training path every
// Forward sees one sample, so the statistics of plane (b, f) are that
// sample's own: one wave per plane of HW values.  Forward: mean = sum *
// (1/HW), var = sum (x - mean)^2 * (1/HW), std = float32(sqrt(float64(var +
// eps))), y = gamma ((x - mean) * (1/std)) + beta (:320-400).  Backward
// (:611-660): dx = g gamma / std - sum(g) gamma / HW / std - (x - mean)
// sum(g (x - mean)) gamma / HW / std^3; per-plane partial sums of g (x -
// mean) / std and g for the gamma / beta column sums.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bn_wsum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__global__ __launch_bounds__(256) void bn_fwd_train_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ gb,
                                                           float *__restrict__ y,
                                                           float *__restrict__ st, int planes, int C,
                                                           int HW, float eps) {
  const int pl = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (pl >= planes) return;
  const int f = pl % C;
  const float *xr = x + (int64_t)pl * HW;
  const float invN = 1.0f / (float)HW;
  float s = 0.f;
  for (int i = lane; i < HW; i += 64) s += xr[i];
  const float mean = bn_wsum(s) * invN;
  float ss = 0.f;
  for (int i = lane; i < HW; i += 64) {
    const float d = xr[i] - mean;
    ss += d * d;
  }
  const float var = bn_wsum(ss) * invN;
  const float std = (float)sqrt((double)(var + eps)), istd = 1.0f / std;
  float *yr = y + (int64_t)pl * HW;
  if (gb) {
    const float g = gb[f], b = gb[C + f];
    for (int i = lane; i < HW; i += 64) yr[i] = g * ((xr[i] - mean) * istd) + b;
  } else {
    for (int i = lane; i < HW; i += 64) yr[i] = (xr[i] - mean) * istd;
  }
  if (lane == 0) {
    st[3 * pl] = mean;
    st[3 * pl + 1] = var;
    st[3 * pl + 2] = std;
  }
}

// running stats: one update per sample in sample order, r = (1 - m) r + m stat
// (batchnorm2d.go:337, 356), each product and sum rounded as in the reference
__global__ __launch_bounds__(256) void bn_running_kernel(const float *__restrict__ st,
                                                         float *__restrict__ rm,
                                                         float *__restrict__ rv, int B, int C,
                                                         float mom) {
  const int f = blockIdx.x * 256 + threadIdx.x;
  if (f >= C) return;
  const float om = 1.0f - mom;
  float m = rm[f], v = rv[f];
  for (int b = 0; b < B; ++b) {
    const float *p = st + 3 * ((int64_t)b * C + f);
    m = __fadd_rn(__fmul_rn(om, m), __fmul_rn(mom, p[0]));
    v = __fadd_rn(__fmul_rn(om, v), __fmul_rn(mom, p[1]));
  }
  rm[f] = m;
  rv[f] = v;
}

// inference (batchnorm2d.go:493-508): running stats, (x - mean) / std
__global__ __launch_bounds__(256) void bn_fwd_eval_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ gb,
                                                          const float *__restrict__ rm,
                                                          const float *__restrict__ rv,
                                                          float *__restrict__ y, int64_t total, int C,
                                                          int HW, float eps) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * 256) {
    const int f = (int)((e / HW) % C);
    const float std = (float)sqrt((double)(rv[f] + eps));
    const float norm = (x[e] - rm[f]) / std;
    y[e] = gb ? gb[f] * norm + gb[C + f] : norm;
  }
}

__global__ __launch_bounds__(256) void bn_bwd_kernel(const float *__restrict__ g,
                                                     const float *__restrict__ x,
                                                     const float *__restrict__ gb,
                                                     const float *__restrict__ st,
                                                     float *__restrict__ dx,
                                                     float *__restrict__ part, int planes, int C,
                                                     int HW) {
  const int pl = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (pl >= planes) return;
  const int f = pl % C;
  const float *gr = g + (int64_t)pl * HW, *xr = x + (int64_t)pl * HW;
  const float mean = st[3 * pl], std = st[3 * pl + 2];
  float sg = 0.f, sgx = 0.f;
  for (int i = lane; i < HW; i += 64) {
    sg += gr[i];
    sgx += gr[i] * (xr[i] - mean);
  }
  sg = bn_wsum(sg);
  sgx = bn_wsum(sgx);
  const float gm = gb ? gb[f] : 1.0f, m = (float)HW;
  const float t1 = (sg * gm) / m / std, den = std * std * std, sgxg = sgx * gm;
  float pg = 0.f;
  for (int i = lane; i < HW; i += 64) {
    const float diff = xr[i] - mean;
    if (dx) dx[(int64_t)pl * HW + i] = (gr[i] * gm) / std - t1 - diff * sgxg / m / den;
    pg += gr[i] * (diff / std);
  }
  pg = bn_wsum(pg);
  if (part && lane == 0) {
    part[pl] = pg;            // gamma: sum g (x - mean) / std
    part[planes + pl] = sg;   // beta: sum g
  }
}

hipError_t launch_bn_fwd(const float *x, const float *gb, float *y, float *st, float *rm, float *rv,
                         int B, int C, int HW, float eps, float mom, int training, hipStream_t s) {
  const int planes = B * C;
  if (planes <= 0) return hipSuccess;
  if (training) {
    hipLaunchKernelGGL(bn_fwd_train_kernel, dim3((planes + 3) / 4), dim3(256), 0, s, x, gb, y, st,
                       planes, C, HW, eps);
    hipLaunchKernelGGL(bn_running_kernel, dim3((C + 255) / 256), dim3(256), 0, s, st, rm, rv, B, C,
                       mom);
  } else {
    const int64_t total = (int64_t)planes * HW;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(bn_fwd_eval_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, gb, rm, rv, y,
                       total, C, HW, eps);
  }
  return hipGetLastError();
}

// inference-mode backward (batchnorm2d.go:525-551): dx = (g * gamma) / std of
// the running variance; the parameters get no gradient
__global__ __launch_bounds__(256) void bn_bwd_eval_kernel(const float *__restrict__ g,
                                                          const float *__restrict__ gb,
                                                          const float *__restrict__ rv,
                                                          float *__restrict__ dx, int64_t total,
                                                          int C, int HW, float eps) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * 256) {
    const int f = (int)((e / HW) % C);
    const float std = (float)sqrt((double)(rv[f] + eps));
    const float gg = gb ? g[e] * gb[f] : g[e];
    dx[e] = gg / std;
  }
}

hipError_t launch_bn_bwd_eval(const float *g, const float *gb, const float *rv, float *dx, int B,
                              int C, int HW, float eps, hipStream_t s) {
  const int64_t total = (int64_t)B * C * HW;
  if (total <= 0 || !dx) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(bn_bwd_eval_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, gb, rv, dx,
                     total, C, HW, eps);
  return hipGetLastError();
}

hipError_t launch_bn_bwd(const float *g, const float *x, const float *gb, const float *st, float *dx,
                         float *part, int B, int C, int HW, hipStream_t s) {
  const int planes = B * C;
  if (planes <= 0) return hipSuccess;
  hipLaunchKernelGGL(bn_bwd_kernel, dim3((planes + 3) / 4), dim3(256), 0, s, g, x, gb, st, dx, part,
                     planes, C, HW);
  return hipGetLastError();
}

}  // namespace gn
