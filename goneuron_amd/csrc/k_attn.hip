// Transformer-path kernels: Embedding gather / last-sample scatter,
// PositionalEncoding add, causal multi-head attention forward / backward,
// LayerNorm forward / backward, CLSPooling, per-sample token sums.
//
// Semantics follow the reference per sample (transformer.go, layernorm.go,
// embedding.go):
//  - scores s_ij = (q_i . k_j) / sqrt(hd), -1e9 where j > i under the causal
//    mask, row softmax (activations.go:161-183; exp in float32 here, see
//    attn_probs), o_i = sum_j p_ij v_j (transformer.go:466-503);
//  - backward dP_ij = gO_i . v_j, dS_ij = p_ij (dP_ij - sum_k dP_ik p_ik),
//    gradScore = dS / sqrt(hd), gQ += gradScore k, gK += gradScore q,
//    gV += p gO (transformer.go:583-648);
//  - LayerNorm y = gamma (x - mu)/std + beta, std = sqrt(var + eps) in float64;
//    backward dx = (gp - sum(gp)/N)/std - (x-mu) sum(gp (x-mu)) / (N std^2)
//    with gp = g gamma (layernorm.go:405-424; the exact gradient would have
//    std^3 in the last term);
//  - Embedding.Backward zeroes the whole gradient before scattering, so only
//    the last sample of each worker chunk contributes (embedding.go:152-154).
#include <algorithm>

#include "gn_common.h"

namespace gn {

constexpr int AT_T = 128;   // max sequence length held in LDS
constexpr int AT_HD = 32;   // max head dim held in LDS

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
// out[b, t, :] = E[floor(x[b, t]), :], ids[b, t] = that index; block row
// blockIdx.y is sample b.  An index outside [0, V) makes Embedding.Forward
// return an error (embedding.go:126-128), and the batch loop then skips the
// sample (net.go:738-741, 641-644): every block of the sample checks its T ids
// and block 0 records bad[b] (with bad_or, a later Embedding of the network,
// only sets it, so the flag covers every Embedding); such a sample's rows
// read E[0] and are masked out downstream.
__global__ __launch_bounds__(256) void embed_kernel(const float *__restrict__ x,
                                                    const float *__restrict__ E,
                                                    int32_t *__restrict__ ids,
                                                    float *__restrict__ out, int T, int V, int D,
                                                    int32_t *__restrict__ bad, int bad_or) {
  const int b = blockIdx.y;
  const float *xs = x + (int64_t)b * T;
  int any = 0;
  for (int t = threadIdx.x; t < T; t += 256) {
    const int idx = (int)floor((double)xs[t]);
    any |= (idx < 0 || idx >= V) ? 1 : 0;
  }
  any = __syncthreads_or(any);
  if (bad && blockIdx.x == 0 && threadIdx.x == 0 && (any || !bad_or)) bad[b] = any ? 1 : 0;
  const int64_t n = (int64_t)T * D;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int t = (int)(e / D), d = (int)(e - (int64_t)t * D);
    int idx = (int)floor((double)xs[t]);
    if (idx < 0 || idx >= V) idx = 0;
    if (d == 0) ids[(int64_t)b * T + t] = idx;
    out[(int64_t)b * n + e] = E[(int64_t)idx * D + d];
  }
}

// Embedding followed by PositionalEncoding in one pass: the embedding rows
// as embed_kernel writes them, and pe_out = those rows + P[t] (the
// PositionalEncoding output, pe_add_kernel's values).
__global__ __launch_bounds__(256) void embed_pe_kernel(const float *__restrict__ x,
                                                       const float *__restrict__ E,
                                                       const float *__restrict__ pe,
                                                       int32_t *__restrict__ ids,
                                                       float *__restrict__ out,
                                                       float *__restrict__ pe_out, int T, int V,
                                                       int D, int32_t *__restrict__ bad, int bad_or) {
  const int b = blockIdx.y;
  const float *xs = x + (int64_t)b * T;
  int any = 0;
  for (int t = threadIdx.x; t < T; t += 256) {
    const int idx = (int)floor((double)xs[t]);
    any |= (idx < 0 || idx >= V) ? 1 : 0;
  }
  any = __syncthreads_or(any);
  if (bad && blockIdx.x == 0 && threadIdx.x == 0 && (any || !bad_or)) bad[b] = any ? 1 : 0;
  const int64_t n = (int64_t)T * D;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int t = (int)(e / D), d = (int)(e - (int64_t)t * D);
    int idx = (int)floor((double)xs[t]);
    if (idx < 0 || idx >= V) idx = 0;
    if (d == 0) ids[(int64_t)b * T + t] = idx;
    const float v = E[(int64_t)idx * D + d];
    out[(int64_t)b * n + e] = v;
    pe_out[(int64_t)b * n + e] = v + pe[e];
  }
}

__global__ __launch_bounds__(256) void pe_add_kernel(const float *__restrict__ x,
                                                     const float *__restrict__ pe,
                                                     float *__restrict__ out, int64_t n, int TD) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256)
    out[e] = x[e] + pe[e % TD];
}

// grad[E] = 0 except the rows the scatter writes (zeroing blocks), and the
// token rows of each worker chunk's contributing sample scatter-added in
// (chunk, token) order.
// Embedding.Backward zeroes the gradient first (embedding.go:152-154), so the
// contributing sample is the last one whose backward ran: the chunk's last
// sample, or with skipped samples (bad[b]) the last valid one (sequential
// loop, net.go:738-741) or the one before the chunk's first bad sample (a
// worker returns at its first error, net.go:641-644); none if there is none.
// Block l takes contributing row l: if l is the first row carrying its id it
// sums, in order, every row with that id and writes the row of gradE; rows
// whose id appeared earlier write nothing, so all writes are to distinct rows.
constexpr int EG_MAXL = 2048;  // contributing rows held in LDS

// Blocks L.. zero the rows of gradE that no contributing row writes, EG_ZR
// rows each (the fill the reference's zeroing amounts to, without a launch of
// its own).
constexpr int EG_ZR = 32;
// Blocks past those (pe_grad not null): a PositionalEncoding's gradient below
// which this Embedding sits, pe_grad[e] = scale * sum over the B samples of
// g[b][e], b ascending (the same gradient rows; transformer.go:112-118), 256
// columns e of the T x D table per block.
// With the step's update (ad.stride; launch_embed_grad's upd): every
// gradient written here is updated by the thread that writes it (the zeroed
// rows too, with g = 0), and blocks past the PositionalEncoding's update the
// float4 groups of ad.rest's ranges (every other layer, whose gradients are
// final and whose parameters no later kernel of the step reads).
__device__ __forceinline__ void adam_g4(float4 *g4, float4 gv, const AdamStep &ad, float4 p, float4 m,
                                        float4 v) {
  adam1(p.x, gv.x, m.x, v.x, ad.efflr, ad.b1, ad.b2, ad.omb1, ad.omb2, ad.eps);
  adam1(p.y, gv.y, m.y, v.y, ad.efflr, ad.b1, ad.b2, ad.omb1, ad.omb2, ad.eps);
  adam1(p.z, gv.z, m.z, v.z, ad.efflr, ad.b1, ad.b2, ad.omb1, ad.omb2, ad.eps);
  adam1(p.w, gv.w, m.w, v.w, ad.efflr, ad.b1, ad.b2, ad.omb1, ad.omb2, ad.eps);
  const int64_t s4 = ad.stride >> 2;
  g4[-s4] = p;
  g4[s4] = m;
  g4[2 * s4] = v;
}

__global__ __launch_bounds__(256) void embed_grad_kernel(const float *__restrict__ g,
                                                         const int32_t *__restrict__ ids,
                                                         float *__restrict__ gradE, int B, int T,
                                                         int D, int chunk, int L, float scale,
                                                         const int32_t *__restrict__ bad, int par,
                                                         int V, float *__restrict__ pe_grad, AdamStep ad,
                                                         int pb) {
  __shared__ int sid[EG_MAXL];
  __shared__ int csamp[EG_MAXL];
  __shared__ int first;
  __shared__ int hit[EG_ZR];
  const int l = blockIdx.x, nch = L / T;
  const int zb = (V + EG_ZR - 1) / EG_ZR;
  if (l >= L + zb + pb) {  // update blocks: one float4 group of ad.rest's ranges per thread and pass
    const int nb = gridDim.x - (L + zb + pb), bi = l - (L + zb + pb);
    const int64_t s4 = ad.stride >> 2;
    for (int r = 0; r < 2; ++r) {
      float4 *g4 = reinterpret_cast<float4 *>(ad.rest);
      for (int64_t i = (ad.r0[r] >> 2) + (int64_t)bi * 256 + threadIdx.x; i < (ad.r1[r] >> 2);
           i += (int64_t)nb * 256) {
        const float4 gv = g4[i], p = g4[i - s4], m = g4[i + s4], v = g4[i + 2 * s4];
        adam_g4(g4 + i, gv, ad, p, m, v);
      }
    }
    return;
  }
  if (l >= L + zb) {  // PositionalEncoding block (uniform over the block)
    const int64_t n = (int64_t)T * D, e = (int64_t)(l - L - zb) * 256 + threadIdx.x;
    if (e >= n) return;
    float acc = 0.f;
    int b = 0;
    for (; b + 15 < B; b += 16) {  // sixteen rows in flight, added in order
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = g[(int64_t)(b + u) * n + e];
#pragma unroll
      for (int u = 0; u < 16; ++u) acc += v[u];
    }
    for (; b < B; ++b) acc += g[(int64_t)b * n + e];
    pe_grad[e] = acc * scale;
    if (ad.stride) adam_at(pe_grad + e, acc * scale, ad);
    return;
  }
  for (int w = threadIdx.x; w < nch; w += 256) {
    const int c0 = w * chunk, c1 = min(B, c0 + chunk);
    int sm = c1 - 1;
    if (bad) {
      if (par) {
        int f = c0;
        while (f < c1 && !bad[f]) ++f;
        sm = f - 1;
      } else {
        while (sm >= c0 && bad[sm]) --sm;
      }
      if (sm < c0) sm = -1;
    }
    csamp[w] = sm;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < L; e += 256) {
    const int sm = csamp[e / T];
    sid[e] = sm < 0 ? -1 : ids[(int64_t)sm * T + e % T];
  }
  if (threadIdx.x == 0) first = 1;
  if (l >= L) {  // zeroing block: rows [z0, z1) minus the contributing ids
    const int z0 = (l - L) * EG_ZR, z1 = min(V, z0 + EG_ZR);
    if (threadIdx.x < EG_ZR) hit[threadIdx.x] = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < L; e += 256) {
      const int id = sid[e];
      if (id >= z0 && id < z1) hit[id - z0] = 1;  // every writer stores 1
    }
    __syncthreads();
    float *base = gradE + (int64_t)z0 * D;
    if ((D & 3) == 0 && (reinterpret_cast<uintptr_t>(base) & 15) == 0) {
      // 16-byte stores, row and column from one 32-bit division per store
      const int D4 = D >> 2, n4 = (z1 - z0) * D4;
      float4 *b4 = reinterpret_cast<float4 *>(base);
      if (ad.stride) {  // zero gradients and their update; a thread's p, m, v loads go out together
        constexpr int ZG = EG_ZR * 256 / 4 / 256;  // float4 groups per thread at D <= 256
        const int64_t s4 = ad.stride >> 2;
        for (int e0 = threadIdx.x; e0 < n4; e0 += ZG * 256) {
          float4 p[ZG], m[ZG], v[ZG];
#pragma unroll
          for (int u = 0; u < ZG; ++u) {
            const int e = e0 + u * 256;
            if (e < n4 && !hit[e / D4]) {
              p[u] = b4[e - s4];
              m[u] = b4[e + s4];
              v[u] = b4[e + 2 * s4];
            }
          }
#pragma unroll
          for (int u = 0; u < ZG; ++u) {
            const int e = e0 + u * 256;
            if (e < n4 && !hit[e / D4]) {
              const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
              b4[e] = z;
              adam_g4(b4 + e, z, ad, p[u], m[u], v[u]);
            }
          }
        }
      } else {
        for (int e = threadIdx.x; e < n4; e += 256) {
          const int r = e / D4;
          if (!hit[r]) b4[e] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    } else {
      const int n = (z1 - z0) * D;
      for (int e = threadIdx.x; e < n; e += 256)
        if (!hit[e / D]) base[e] = 0.0f;
    }
    return;
  }
  __syncthreads();
  const int my = sid[l];
  if (my < 0) return;  // uniform over the block
  for (int e = threadIdx.x; e < l; e += 256)
    if (sid[e] == my) first = 0;  // benign race: every writer stores 0
  __syncthreads();
  if (!first) return;
  // wave 0 lists the rows e >= l with this id, in ascending order (ballots
  // over 64 rows at a time); every thread then sums only those rows
  __shared__ int lst[EG_MAXL];
  __shared__ int nl;
  if (threadIdx.x < 64) {
    int cnt = 0;
    for (int base = l; base < L; base += 64) {
      const int e = base + threadIdx.x;
      const bool m = e < L && sid[e] == my;
      const unsigned long long mask = __ballot(m);
      if (m) lst[cnt + __popcll(mask & ((1ull << threadIdx.x) - 1ull))] = e;
      cnt += __popcll(mask);
    }
    if (threadIdx.x == 0) nl = cnt;
  }
  __syncthreads();
  const int n = nl;
  for (int d = threadIdx.x; d < D; d += 256) {
    float acc = 0.f;
    for (int j = 0; j < n; ++j) {
      const int e = lst[j];
      acc += g[((int64_t)csamp[e / T] * T + e % T) * D + d];
    }
    gradE[(int64_t)my * D + d] = acc * scale;
    if (ad.stride) adam_at(gradE + (int64_t)my * D + d, acc * scale, ad);
  }
}

// More than EG_MAXL contributing rows: the same sums, with the contributing
// sample of every chunk and the id of every row in a global list that
// embed_grad_prep writes first, and each block's matching rows gathered into
// LDS EG_MAXL at a time (the running sum is kept in gradE between batches, so
// the additions keep their order).
__global__ __launch_bounds__(256) void embed_grad_prep(const int32_t *__restrict__ ids, int B, int T,
                                                       int chunk, int L, const int32_t *__restrict__ bad,
                                                       int par, int *__restrict__ sid) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= L) return;
  const int w = e / T, c0 = w * chunk, c1 = min(B, c0 + chunk);
  int sm = c1 - 1;
  if (bad) {
    if (par) {
      int f = c0;
      while (f < c1 && !bad[f]) ++f;
      sm = f - 1;
    } else {
      while (sm >= c0 && bad[sm]) --sm;
    }
    if (sm < c0) sm = -1;
  }
  sid[e] = sm < 0 ? -1 : ids[(int64_t)sm * T + e % T];
  sid[L + e] = sm;  // the row's sample (-1: none)
}

__global__ __launch_bounds__(256) void embed_grad_global_kernel(const float *__restrict__ g,
                                                                const int *__restrict__ sid,
                                                                float *__restrict__ gradE, int T, int D,
                                                                int L, float scale, int V) {
  __shared__ int first;
  __shared__ int hit[EG_ZR];
  __shared__ int lst[EG_MAXL];
  __shared__ int nl;
  const int l = blockIdx.x;
  const int *samp = sid + L;
  if (l >= L) {  // zeroing block
    const int z0 = (l - L) * EG_ZR, z1 = min(V, z0 + EG_ZR);
    if (threadIdx.x < EG_ZR) hit[threadIdx.x] = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < L; e += 256) {
      const int id = sid[e];
      if (id >= z0 && id < z1) hit[id - z0] = 1;
    }
    __syncthreads();
    float *base = gradE + (int64_t)z0 * D;
    const int n = (z1 - z0) * D;
    for (int e = threadIdx.x; e < n; e += 256)
      if (!hit[e / D]) base[e] = 0.0f;
    return;
  }
  const int my = sid[l];
  if (my < 0) return;  // uniform over the block
  if (threadIdx.x == 0) first = 1;
  __syncthreads();
  for (int e = threadIdx.x; e < l; e += 256)
    if (sid[e] == my) first = 0;
  __syncthreads();
  if (!first) return;
  float *row = gradE + (int64_t)my * D;
  bool started = false;
  for (int pos = l; pos < L;) {
    // wave 0 lists the next matching rows (ascending, at most EG_MAXL - 64
    // per batch so a ballot never overflows), every thread adds them
    if (threadIdx.x < 64) {
      int cnt = 0, base = pos;
      for (; base < L && cnt <= EG_MAXL - 64; base += 64) {
        const int e = base + threadIdx.x;
        const bool m = e < L && sid[e] == my;
        const unsigned long long mask = __ballot(m);
        if (m) lst[cnt + __popcll(mask & ((1ull << threadIdx.x) - 1ull))] = e;
        cnt += __popcll(mask);
      }
      if (threadIdx.x == 0) {
        nl = cnt;
        first = base;  // where the next batch starts
      }
    }
    __syncthreads();
    const int n = nl;
    const int next = first;
    for (int d = threadIdx.x; d < D; d += 256) {
      float acc = started ? row[d] : 0.f;
      for (int j = 0; j < n; ++j) {
        const int e = lst[j];
        acc += g[((int64_t)samp[e] * T + e % T) * D + d];
      }
      row[d] = next >= L ? acc * scale : acc;
    }
    started = true;
    pos = next;
    __syncthreads();
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
// Block = 64 columns x 16 token groups of sample blockIdx.y; partials added in LDS.
// blockIdx.z selects a member of a batched launch (X, S advanced by xs, ss).
__global__ __launch_bounds__(1024) void token_sum_kernel(const float *__restrict__ X,
                                                         float *__restrict__ S, int B, int T, int N,
                                                         int64_t xs, int64_t ss) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int64_t b = blockIdx.y;
  X += blockIdx.z * xs;
  S += blockIdx.z * ss;
  float s = 0.f;
  if (c < N) {
    const float *p = X + b * T * N + c;
    // eight tokens' loads in flight, added in token order
    int t = grp;
    for (; t + 7 * 16 < T; t += 8 * 16) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)(t + 16 * u) * N];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; t < T; t += 16) s += p[(int64_t)t * N];
  }
  red[grp][lane] = s;
  __syncthreads();
  if (grp == 0 && c < N) {
    float v = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) v += red[g][lane];
    S[b * N + c] = v;
  }
}

// Q10 weight and bias gradients of a Linear in the block from the per-sample
// token sums S [B][M] (pitch lds) and the last token's input rows X [B]
// (pitch ldx): dW[o][i] = scale * sum_b S[b][o] X[b][i] and db[o] = scale *
// sum_b S[b][o], b ascending (the K = B product and the column sum of one
// launch).  Block = 16 rows o x 64 columns i; per chunk of 64 samples every
// thread issues its S and X loads at once (one memory round trip), stages
// them in LDS, then thread (g, i) accumulates rows 4g..4g+3.  blockIdx.z
// selects the member.
constexpr int TD_O = 16, TD_I = 64, TD_CB = 64;
struct TdShared {
  float ss[TD_CB][TD_O];
  float xs[TD_CB][TD_I];
};
// One 16 x 64 block (by, bx) of a Q10 gradient.  The token sum of sample b
// is S[b * np * ps + o] when np = 1, or the np partial rows S[(b * np + j) *
// ps + o], j ascending, when the producer left per-row-block partials (a
// LayerNorm backward block of 16 token rows, np = T / 16).
__device__ __forceinline__ void tok_dw_block(TdShared &sh, const float *__restrict__ S, int np,
                                             int64_t ps, const float *__restrict__ X, int64_t ldx,
                                             float *__restrict__ dW, float *__restrict__ db, int B,
                                             int M, int N, float scale, int bx, int by) {
  const int tid = threadIdx.x, lane = tid & 63, g = tid >> 6;
  const int i0 = bx * TD_I, o0 = by * TD_O;
  const bool bias = bx == 0 && tid < TD_O;
  constexpr int NS = TD_CB * TD_O / 256, NX = TD_CB * TD_I / 256;  // 4 and 16 loads per thread
  float acc[4] = {0.f, 0.f, 0.f, 0.f}, bs = 0.f;
  for (int b0 = 0; b0 < B; b0 += TD_CB) {
    const int nb = min(TD_CB, B - b0);
    float sv[NS], xv[NX];
    const float *sp[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const int e = tid + 256 * q, bb = e / TD_O, oo = e % TD_O;
      sp[q] = bb < nb && o0 + oo < M ? S + (size_t)(b0 + bb) * np * ps + o0 + oo : nullptr;
      sv[q] = sp[q] ? sp[q][0] : 0.f;
    }
    // the further partials eight per element at a time, all elements' loads in
    // flight together, each element's partials added in order
    for (int j = 1; j < np; j += 8) {
      float u[NS][8];
#pragma unroll
      for (int q = 0; q < NS; ++q)
#pragma unroll
        for (int k = 0; k < 8; ++k) u[q][k] = sp[q] && j + k < np ? sp[q][(size_t)(j + k) * ps] : 0.f;
#pragma unroll
      for (int q = 0; q < NS; ++q)
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (j + k < np) sv[q] += u[q][k];
    }
#pragma unroll
    for (int q = 0; q < NX; ++q) {
      const int bb = (tid >> 6) + 4 * q;
      xv[q] = bb < nb && i0 + lane < N ? X[(size_t)(b0 + bb) * ldx + i0 + lane] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const int e = tid + 256 * q;
      sh.ss[e / TD_O][e % TD_O] = sv[q];
    }
#pragma unroll
    for (int q = 0; q < NX; ++q) sh.xs[(tid >> 6) + 4 * q][lane] = xv[q];
    __syncthreads();
    for (int bb = 0; bb < nb; ++bb) {
      const float x = sh.xs[bb][lane];
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[k] += sh.ss[bb][4 * g + k] * x;
    }
    if (bias)
      for (int bb = 0; bb < nb; ++bb) bs += sh.ss[bb][tid];
    __syncthreads();
  }
  const int i = i0 + lane;
  if (i < N) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int o = o0 + 4 * g + k;
      if (o < M) dW[(size_t)o * N + i] = acc[k] * scale;
    }
  }
  if (bias && o0 + tid < M) db[o0 + tid] = bs * scale;
}

__global__ __launch_bounds__(256) void tok_dw_kernel(TokDwSet set, int B, int M, int N, int lds,
                                                     int ldx, float scale) {
  __shared__ TdShared sh;
  const int z = blockIdx.z;
  tok_dw_block(sh, set.S[z], 1, lds, set.X[z], ldx, set.dW[z], set.db[z], B, M, N, scale, blockIdx.x,
               blockIdx.y);
}

// ---------------------------------------------------------------------------
// LayerNorm over rows of N (one wave64 per row)
// ---------------------------------------------------------------------------
// cls (may be null): rows r with r % clsT == 0 are also written to row r /
// clsT of cls (a CLSPooling above the LayerNorm, transformer.go:1679-1725).
__global__ __launch_bounds__(256) void ln_fwd_kernel(const float *__restrict__ x,
                                                     const float *__restrict__ gam,
                                                     const float *__restrict__ bet,
                                                     float *__restrict__ y,
                                                     float *__restrict__ stats, int rows, int N,
                                                     float eps, float *__restrict__ cls, int clsT) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float *xr = x + (int64_t)r * N;
  float *crow = cls && r % clsT == 0 ? cls + (int64_t)(r / clsT) * N : nullptr;
  constexpr int LF_C = 8;  // up to 512 columns held in registers
  if (N <= 64 * LF_C) {
    // the row in registers, read once (its loads in flight together); the
    // same sums in the same order as the loops below
    float v[LF_C], gv[LF_C], bv[LF_C];
#pragma unroll
    for (int c = 0; c < LF_C; ++c) {
      const int i = lane + 64 * c;
      v[c] = i < N ? xr[i] : 0.f;
      gv[c] = i < N ? gam[i] : 0.f;
      bv[c] = i < N ? bet[i] : 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < LF_C; ++c)
      if (lane + 64 * c < N) s += v[c];
    const float mean = wsum(s) / (float)N;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < LF_C; ++c)
      if (lane + 64 * c < N) {
        const float d = v[c] - mean;
        ss += d * d;
      }
    const float var = wsum(ss) / (float)N;
    const float std = (float)sqrt((double)(var + eps));
#pragma unroll
    for (int c = 0; c < LF_C; ++c) {
      const int i = lane + 64 * c;
      if (i < N) {
        const float o = gv[c] * ((v[c] - mean) / std) + bv[c];
        y[(int64_t)r * N + i] = o;
        if (crow) crow[i] = o;
      }
    }
    if (lane == 0) {
      stats[2 * r] = mean;
      stats[2 * r + 1] = std;
    }
    return;
  }
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
  for (int i = lane; i < N; i += 64) {
    const float o = gam[i] * ((xr[i] - mean) / std) + bet[i];
    y[(int64_t)r * N + i] = o;
    if (crow) crow[i] = o;
  }
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

// The same dx, and instead of the g * xhat matrix, the block's own column
// sums of g * xhat (gamma) and g (beta): block = 8 waves x 2 rows (two waves
// per SIMD: with 4 waves x 4 rows one wave per SIMD had waited out every
// load); a wave loads its rows' g and x into registers at once (lane i holds
// columns i, i + 64, ..., N <= 64 LN_MAXC), then finishes them row by row;
// the waves' sums are added in a fixed tree and written as one partial row
// pair part[block][0 .. 2N) for ln_param_final.
// gpool (may be null; then g is read): the gradient of a CLSPooling above,
// row r / poolT of gpool for rows r with r % poolT == 0 and zero for the rest
// (cls_bwd_kernel's rows, not materialised).  tsum (may be null): the
// block's column sums of dx, tsum[block][0 .. N), the per-row-block partials
// of the token sums that a Linear's Q10 gradient below needs.
// Blocks from nln on (ts.X not null): per-sample token sums of another
// matrix, ts.S[b][c] = sum_t ts.X[b][t][c] (a block per sample and 64
// columns, its 4 waves every 4th token with eight loads in flight, the wave
// sums added in wave order), work that would otherwise take a launch of its
// own.
struct LnTokSum {
  const float *X;
  float *S;
  int T, N;
};
constexpr int LN_RW = 2, LN_WV = 8, LN_MAXC = 8, LN_RPB = LN_WV * LN_RW, LN_NT = 64 * LN_WV;
__global__ __launch_bounds__(LN_NT) void ln_bwd_part_kernel(const float *__restrict__ g,
                                                          const float *__restrict__ gpool, int poolT,
                                                          const float *__restrict__ x,
                                                          const float *__restrict__ gam,
                                                          const float *__restrict__ stats,
                                                          float *__restrict__ dx,
                                                          float *__restrict__ part,
                                                          float *__restrict__ tsum, int rows, int N,
                                                          int nln, LnTokSum ts) {
  __shared__ float red[LN_WV][3][LN_MAXC * 64];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // the waves' partial sums v[0..7] added in a fixed tree
  auto tree8 = [](float v0, float v1, float v2, float v3, float v4, float v5, float v6, float v7) {
    return ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7));
  };
  if ((int)blockIdx.x >= nln) {  // token-sum block (uniform over the block)
    const int nc = (ts.N + 63) >> 6, tb = blockIdx.x - nln;
    const int b = tb / nc, c = (tb % nc) * 64 + lane;
    float acc = 0.f;
    if (c < ts.N) {
      const float *p = ts.X + (int64_t)b * ts.T * ts.N + c;
      int t = w;
      for (; t + 7 * LN_WV < ts.T; t += 8 * LN_WV) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)(t + LN_WV * u) * ts.N];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += v[u];
      }
      for (; t < ts.T; t += LN_WV) acc += p[(int64_t)t * ts.N];
    }
    red[w][0][lane] = acc;
    __syncthreads();
    if (w == 0 && c < ts.N)
      ts.S[(int64_t)b * ts.N + c] = tree8(red[0][0][lane], red[1][0][lane], red[2][0][lane], red[3][0][lane],
                                          red[4][0][lane], red[5][0][lane], red[6][0][lane], red[7][0][lane]);
    return;
  }
  const int rbase = blockIdx.x * LN_RPB + w * LN_RW;
  float gv[LN_RW][LN_MAXC], xv[LN_RW][LN_MAXC], gm[LN_MAXC], mean[LN_RW], sd[LN_RW];
#pragma unroll
  for (int j = 0; j < LN_MAXC; ++j) {
    const int i = lane + 64 * j;
    gm[j] = i < N ? gam[i] : 0.f;
  }
#pragma unroll
  for (int q = 0; q < LN_RW; ++q) {
    const int r = min(rbase + q, rows - 1);
    mean[q] = stats[2 * r];
    sd[q] = stats[2 * r + 1];
    const float *grow =
        gpool ? (r % poolT == 0 ? gpool + (int64_t)(r / poolT) * N : nullptr) : g + (int64_t)r * N;
#pragma unroll
    for (int j = 0; j < LN_MAXC; ++j) {
      const int i = lane + 64 * j;
      gv[q][j] = i < N && grow ? grow[i] : 0.f;
      xv[q][j] = i < N ? x[(int64_t)r * N + i] : 0.f;
    }
  }
  float pg[LN_MAXC], pb[LN_MAXC], pd[LN_MAXC];
#pragma unroll
  for (int j = 0; j < LN_MAXC; ++j) pg[j] = pb[j] = pd[j] = 0.f;
  const float nf = (float)N;
#pragma unroll
  for (int q = 0; q < LN_RW; ++q) {
    const int r = rbase + q;
    if (r >= rows) break;  // uniform over the wave
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int j = 0; j < LN_MAXC; ++j)
      if (lane + 64 * j < N) {
        const float gp = gv[q][j] * gm[j];
        sg += gp;
        sgx += gp * (xv[q][j] - mean[q]);
      }
    sg = wsum(sg);
    sgx = wsum(sgx);
    const float std = sd[q];
#pragma unroll
    for (int j = 0; j < LN_MAXC; ++j) {
      const int i = lane + 64 * j;
      if (i < N) {
        const float diff = xv[q][j] - mean[q];
        const float gi = gv[q][j], gp = gi * gm[j];
        float v = (gp - sg / nf) / std;
        v -= (diff * sgx) / (nf * std * std);
        dx[(int64_t)r * N + i] = v;
        pg[j] += gi * (diff / std);
        pb[j] += gi;
        pd[j] += v;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < LN_MAXC; ++j) {
    red[w][0][j * 64 + lane] = pg[j];
    red[w][1][j * 64 + lane] = pb[j];
    if (tsum) red[w][2][j * 64 + lane] = pd[j];
  }
  __syncthreads();
  float *pp = part + (size_t)blockIdx.x * 2 * N;
  for (int i = threadIdx.x; i < N; i += LN_NT) {
#define LN_RED(k) tree8(red[0][k][i], red[1][k][i], red[2][k][i], red[3][k][i], red[4][k][i], red[5][k][i], \
                        red[6][k][i], red[7][k][i])
    pp[i] = LN_RED(0);
    pp[N + i] = LN_RED(1);
    if (tsum) tsum[(size_t)blockIdx.x * N + i] = LN_RED(2);
#undef LN_RED
  }
}

// dgamma / dbeta: the blocks' partials summed per column of [gamma | beta]:
// a block takes 64 columns (one per lane), its 4 waves every 4th partial in
// block order, and the 4 sums are added in wave order, times scale.
__device__ __forceinline__ void ln_param_block(float (&red)[4][64], const float *__restrict__ part,
                                               int nblk, int N, float scale, float *__restrict__ dgam,
                                               float *__restrict__ dbet, int bx) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = bx * 64 + lane;
  float s = 0.f;
  if (c < 2 * N) {
    int b = w;
    // 32 or 16 partials in flight, added in the same order as below
    for (; b + 124 < nblk; b += 128) {
      float v[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) v[u] = part[(size_t)(b + 4 * u) * 2 * N + c];
#pragma unroll
      for (int u = 0; u < 32; ++u) s += v[u];
    }
    for (; b + 60 < nblk; b += 64) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = part[(size_t)(b + 4 * u) * 2 * N + c];
#pragma unroll
      for (int u = 0; u < 16; ++u) s += v[u];
    }
    for (; b + 12 < nblk; b += 16) {
      const float v0 = part[(size_t)b * 2 * N + c], v1 = part[(size_t)(b + 4) * 2 * N + c];
      const float v2 = part[(size_t)(b + 8) * 2 * N + c], v3 = part[(size_t)(b + 12) * 2 * N + c];
      s += v0;
      s += v1;
      s += v2;
      s += v3;
    }
    for (; b < nblk; b += 4) s += part[(size_t)b * 2 * N + c];
  }
  red[w][lane] = s;
  __syncthreads();
  if (w == 0 && c < 2 * N) {
    const float v = ((red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane])) * scale;
    if (c < N) dgam[c] = v;
    else dbet[c - N] = v;
  }
}

__global__ __launch_bounds__(256) void ln_param_final(const float *__restrict__ part, int nblk, int N,
                                                      float scale, float *__restrict__ dgam,
                                                      float *__restrict__ dbet) {
  __shared__ float red[4][64];
  ln_param_block(red, part, nblk, N, scale, dgam, dbet, blockIdx.x);
}

// A transformer block's parameter gradients in one launch: the blocks of
// every LayerNorm job (ln_param_block, the longest chains of loads, so they
// are dispatched first) and then of every Q10 Linear job (tok_dw_block), job
// j owning blocks [start[j], start[j + 1]).
__global__ __launch_bounds__(256) void tb_param_kernel(TbParamSet set, int B, float scale) {
  __shared__ union {
    TdShared td;
    float red[4][64];
  } sh;
  const int bid = blockIdx.x, nj = set.nlin + set.nln;
  int j = 0;
  while (j + 1 < nj && bid >= set.start[j + 1]) ++j;
  const int lb = bid - set.start[j];
  if (j < set.nln) {
    const TbLnJob &q = set.ln[j];
    ln_param_block(sh.red, q.part, q.nblk, q.N, scale, q.dgam, q.dbet, lb);
  } else {
    const TbParamJob &p = set.lin[j - set.nln];
    const int nbx = (p.N + TD_I - 1) / TD_I;
    tok_dw_block(sh.td, p.S, p.np, p.ps, p.X, p.ldx, p.dW, p.db, B, p.M, p.N, scale, lb % nbx, lb / nbx);
  }
}

// ---------------------------------------------------------------------------
// Rotary embeddings (applyRoPE, transformer.go:212-236): the pair (i, i+hd/2)
// of head h of the token at position t = row % T turns by the float32 angle
// tables (cos, sin)[t][i] built on the host as the reference computes them;
// products and sums are rounded one by one as in the reference (no fused
// multiply-add).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rope_kernel(float *__restrict__ x, const float *__restrict__ cs,
                                                   const float *__restrict__ sn, int64_t total,
                                                   int T, int NH, int hd, int conj) {
  const int half = hd >> 1;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / (NH * half);
    const int rem = (int)(e - r * (NH * half)), h = rem / half, i = rem - h * half;
    const int t = (int)(r % T);
    const float c = cs[t * half + i], s = conj ? -sn[t * half + i] : sn[t * half + i];
    float *p = x + r * NH * hd + h * hd;
    const float v1 = p[i], v2 = p[i + half];
    p[i] = __fsub_rn(__fmul_rn(v1, c), __fmul_rn(v2, s));
    p[i + half] = __fadd_rn(__fmul_rn(v1, s), __fmul_rn(v2, c));
  }
}

// ---------------------------------------------------------------------------
// RMSNorm over rows of N (rmsnorm.go:222-240, 301-329), one wave64 per row:
// rms = sqrt(sum x^2 / N + eps) rounded from float64, y = (x / rms) * gamma;
// dx = (gamma / rms) (g - x sum(g gamma x) / (N rms rms)); gx = g (x / rms)
// feeds the gamma column sums.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rms_fwd_kernel(const float *__restrict__ x,
                                                      const float *__restrict__ gam,
                                                      float *__restrict__ y, float *__restrict__ rmsv,
                                                      int rows, int N, float eps) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float *xr = x + (int64_t)r * N;
  float ss = 0.f;
  for (int i = lane; i < N; i += 64) ss += xr[i] * xr[i];
  ss = wsum(ss);
  const float rms = (float)sqrt((double)(ss / (float)N + eps));
  for (int i = lane; i < N; i += 64) y[(int64_t)r * N + i] = (xr[i] / rms) * gam[i];
  if (lane == 0) rmsv[r] = rms;
}

__global__ __launch_bounds__(256) void rms_bwd_kernel(const float *__restrict__ g,
                                                      const float *__restrict__ x,
                                                      const float *__restrict__ gam,
                                                      const float *__restrict__ rmsv,
                                                      float *__restrict__ dx,
                                                      float *__restrict__ gx, int rows, int N) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float *gr = g + (int64_t)r * N, *xr = x + (int64_t)r * N;
  const float rms = rmsv[r], inv = 1.0f / rms;
  float s = 0.f;
  for (int i = lane; i < N; i += 64) s += gr[i] * gam[i] * xr[i];
  s = wsum(s);
  const float factor = s / ((float)N * rms * rms);
  for (int i = lane; i < N; i += 64) {
    const float xi = xr[i], gi = gr[i];
    if (dx) dx[(int64_t)r * N + i] = (gam[i] * inv) * (gi - xi * factor);
    gx[(int64_t)r * N + i] = gi * (xi * inv);
  }
}

// ---------------------------------------------------------------------------
// Causal multi-head attention on fp32 MFMA, one workgroup per (sample,
// head).  Q/K/V/O are [B*T, D] with head h in columns [h*hd, (h+1)*hd);
// T <= 128 and hd <= 32 are held in LDS, staged [t][d] (zero padded to
// 128 x 32) at a 16-byte-aligned pitch (A16_HP, read as float4).  The tokens
// are cut into eight 16-token tiles, and each SIMD owns query tiles s and
// 7 - s (in the backward's key-side products key tiles s and 7 - s), so under
// the causal mask every SIMD works 9 of the 36 live tile pairs: with 8 waves
// per workgroup one tile per wave, two waves per SIMD (tile_of).  A wave per
// 32 queries, the first layout, gave one wave 4 of 10 tile pairs and another
// 1; balanced tiles took C4's forward 13.5 -> 10.6 us and backward 32.1 ->
// 23.6 us with 4 waves, and the second wave per SIMD to 9.3 and 19.2 us.
// The backward recomputes the probabilities from Q and K instead of storing
// B*NH*T*T.
// v_mfma_f32_16x16x4_f32: A[m = l%16][k = l/16], B[k = l/16][n = l%16],
// result register r of lane l is row 4*(l/16) + r, column l%16.
// Scores are formed transposed, S^T = K Q^T, so lane l holds query l%16 of
// its tile and keys 4*(l/16) + r; a product over keys (P V, dS K) then takes
// at step s of key tile kt key 16 kt + 4*(l/16) + s, i.e. the lane's own
// register s as its B operand, and the matching row of V (K) from LDS.
// ---------------------------------------------------------------------------
typedef float fx4 __attribute__((ext_vector_type(4)));
constexpr int A16_HP = 36;   // [t][d] pitch: rows 16-byte aligned, float4 reads conflict-free
constexpr int A16_SP = 132;  // [key][query] pitch of the P^T / dS^T matrix

__device__ __forceinline__ fx4 mfma16(float a, float b, const fx4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Rows [0, 128) x cols [0, 32) of head h of N matrices, zero padded, at
// pitch A16_HP; with hd, D and the pointers multiples of 4 floats every
// thread issues all its 16-byte loads (4 per matrix) before any store.
template <int N, int NT>
__device__ __forceinline__ void stage16(float *const (&dst)[N], const float *const (&src)[N], int b, int h,
                                        int T, int D, int hd) {
  constexpr int PQ = 1024 / NT;  // float4 per thread per matrix (128 rows x 8 float4)
  bool vec = (hd & 3) == 0 && (D & 3) == 0;
#pragma unroll
  for (int m = 0; m < N; ++m) vec = vec && (reinterpret_cast<uintptr_t>(src[m]) & 15) == 0;
  if (vec) {
    float4 v[N][PQ];
#pragma unroll
    for (int m = 0; m < N; ++m)
#pragma unroll
      for (int q = 0; q < PQ; ++q) {
        const int f = threadIdx.x + NT * q;
        const int t = f >> 3, d = (f & 7) << 2;
        v[m][q] = (t < T && d < hd)
                      ? *reinterpret_cast<const float4 *>(src[m] + ((int64_t)b * T + t) * D + h * hd + d)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
    for (int m = 0; m < N; ++m)
#pragma unroll
      for (int q = 0; q < PQ; ++q) {
        const int f = threadIdx.x + NT * q;
        *reinterpret_cast<float4 *>(dst[m] + (f >> 3) * A16_HP + ((f & 7) << 2)) = v[m][q];
      }
    return;
  }
  for (int m = 0; m < N; ++m)
    for (int e = threadIdx.x; e < AT_T * AT_HD; e += NT) {
      const int t = e / AT_HD, d = e % AT_HD;
      dst[m][t * A16_HP + d] = (t < T && d < hd) ? src[m][((int64_t)b * T + t) * D + h * hd + d] : 0.f;
    }
}

// The lane's 8 head-dim values of row `row` that the B operand of a 32-deep
// score product takes: d = 4*(l/16) + s (steps 0-3) and 16 + 4*(l/16) + s.
__device__ __forceinline__ void rows16(float4 (&r)[2], const float *s, int row, int lane) {
  const float4 *p = reinterpret_cast<const float4 *>(s + row * A16_HP + 4 * (lane >> 4));
  r[0] = p[0];
  r[1] = p[4];
}

// X^T tile: acc[r] = sum_d Y[16 yt + 4*(l/16) + r][d] * Z[row of zb][d] (Y rows
// from LDS, the lane's Z row in zb), k order d = 4*(l/16) + s, then + 16.
__device__ __forceinline__ fx4 tile_t(const float *sy, const float4 (&zb)[2], int yt, int lane) {
  float4 yb[2];
  rows16(yb, sy, 16 * yt + (lane & 15), lane);
  fx4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma16(yb[0].x, zb[0].x, acc);
  acc = mfma16(yb[0].y, zb[0].y, acc);
  acc = mfma16(yb[0].z, zb[0].z, acc);
  acc = mfma16(yb[0].w, zb[0].w, acc);
  acc = mfma16(yb[1].x, zb[1].x, acc);
  acc = mfma16(yb[1].y, zb[1].y, acc);
  acc = mfma16(yb[1].z, zb[1].z, acc);
  acc = mfma16(yb[1].w, zb[1].w, acc);
  return acc;
}

// o[half][r] += sum over the 16 keys of tile kt of Y[j][16 half + l%16] * Zt[j]
// (Zt the lane's transposed-score registers): the head-dim-major product
// O^T[d][i] = sum_j Y[j][d] Z[i][j].
__device__ __forceinline__ void keys_t(fx4 (&o)[2], const float *sy, const fx4 &zt, int kt, int lane) {
  const int j0 = 16 * kt + 4 * (lane >> 4), d = lane & 15;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    o[0] = mfma16(sy[(j0 + s) * A16_HP + d], zt[s], o[0]);
    o[1] = mfma16(sy[(j0 + s) * A16_HP + 16 + d], zt[s], o[1]);
  }
}

// Softmax of the scores of query i = 16 qt + l%16 over the key tiles kt <=
// klim (the rest are fully masked and contribute exact zeros): scores /
// sqrt(hd), -1e9 on causal-masked entries (as the reference), keys j >= T
// absent; float32 exp, products with the reciprocals of sqrt(hd) and of the
// row sum (attn_probs' arithmetic).
__device__ __forceinline__ void probs16(fx4 (&st)[8], int qt, int klim, int T, int causal,
                                        float inv_scale, int lane) {
  const int i = 16 * qt + (lane & 15);
  float mx = -__builtin_inff();
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) {
    if (kt > klim) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * kt + 4 * (lane >> 4) + r;
      float sc;
      if (j >= T) sc = -__builtin_inff();
      else if (causal && j > i) sc = -1e9f;
      else sc = st[kt][r] * inv_scale;
      st[kt][r] = sc;
      mx = fmaxf(mx, sc);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  float sum = 0.f;
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) {
    if (kt > klim) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * kt + 4 * (lane >> 4) + r;
      const float e = j < T ? expf(st[kt][r] - mx) : 0.f;
      st[kt][r] = e;
      sum += e;
    }
  }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  const float inv_sum = 1.0f / sum;
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) {
    if (kt > klim) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) st[kt][r] = st[kt][r] * inv_sum;
  }
}

// Store a head-dim-major accumulator pair (O^T[d][i]: lane l, register r is d
// = 4*(l/16) + r + 16 half, query i = l%16 of tile qt) as head-h columns of G.
__device__ __forceinline__ void store16_t(float *G, const fx4 (&v)[2], int b, int h, int T, int D, int hd,
                                          int qt, int lane) {
  const int i = 16 * qt + (lane & 15);
  if (i >= T) return;
  float *row = G + ((int64_t)b * T + i) * D + h * hd;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int d0 = 16 * half + 4 * (lane >> 4);
    if (d0 + 3 < hd && ((reinterpret_cast<uintptr_t>(row + d0) & 15) == 0)) {
      *reinterpret_cast<float4 *>(row + d0) = make_float4(v[half][0], v[half][1], v[half][2], v[half][3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (d0 + r < hd) row[d0 + r] = v[half][r];
    }
  }
}

// Query (key) tile u of wave w: with 4 waves tiles w and 7 - w; with 8 waves
// (two per SIMD, waves w and w + 4 on one SIMD) tile w for w < 4 and 11 - w
// after, so each SIMD again works tiles s and 7 - s.
template <int NW>
__device__ __forceinline__ int tile_of(int w, int u) {
  return NW == 4 ? (u ? 7 - w : w) : (w < 4 ? w : 11 - w);
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void attn16_fwd_kernel(const float *__restrict__ Q,
                                                             const float *__restrict__ K,
                                                             const float *__restrict__ V,
                                                             float *__restrict__ O, int T, int D, int NH,
                                                             int causal) {
  constexpr int NU = 8 / NW;
  __shared__ __align__(16) float sq[AT_T * A16_HP];
  __shared__ __align__(16) float sk[AT_T * A16_HP];
  __shared__ __align__(16) float sv[AT_T * A16_HP];
  const int b = blockIdx.x / NH, h = blockIdx.x % NH;
  const int hd = D / NH;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  {
    float *const dst[3] = {sq, sk, sv};
    const float *const src[3] = {Q, K, V};
    stage16<3, 64 * NW>(dst, src, b, h, T, D, hd);
  }
  __syncthreads();
  const float inv_scale = 1.0f / (float)sqrt((double)hd);
  const int nt = (T + 15) >> 4;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int qt = tile_of<NW>(w, u);
    if (qt >= nt) continue;
    const int klim = causal ? qt : nt - 1;
    float4 qb[2];
    rows16(qb, sq, 16 * qt + (lane & 15), lane);
    fx4 st[8];
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      if (kt <= klim) st[kt] = tile_t(sk, qb, kt, lane);
    probs16(st, qt, klim, T, causal, inv_scale, lane);
    // O^T[d][i] = sum_j V[j][d] P[i][j]
    fx4 o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      if (kt <= klim) keys_t(o, sv, st[kt], kt, lane);
    store16_t(O, o, b, h, T, D, hd, qt, lane);
  }
}

// Backward, same tiles: query side (wave w: query tiles w, 7 - w) recomputes
// P, forms dP^T = V gO^T, r_i = sum_j dP_ij p_ij and dS = (dP p - p r) /
// sqrt(hd), writes gQ = dS K and leaves P^T (then dS^T) in LDS as [j][i]; key
// side (wave w: key tiles w, 7 - w) sums gV_j = sum_i p_ij gO_i and gK_j =
// sum_i dS_ij q_i over the live query tiles.  TS (may be null): the
// per-sample token sums of gQ, gK and gV (member m at TS + m * tss, [B][D])
// for the Q10 gradients of the three projections: each wave's sums over its
// queries (keys) meet in LDS and are added in wave order.
template <int NW>
__global__ __launch_bounds__(64 * NW) void attn16_bwd_kernel(const float *__restrict__ Q,
                                                             const float *__restrict__ K,
                                                             const float *__restrict__ V,
                                                             const float *__restrict__ GO,
                                                             float *__restrict__ GQ,
                                                             float *__restrict__ GK,
                                                             float *__restrict__ GV, int T, int D,
                                                             int NH, int causal, float *__restrict__ TS,
                                                             int64_t tss) {
  constexpr int NU = 8 / NW;
  __shared__ __align__(16) float sq[AT_T * A16_HP];
  __shared__ __align__(16) float sk[AT_T * A16_HP];
  __shared__ __align__(16) float sv[AT_T * A16_HP];
  __shared__ __align__(16) float sg[AT_T * A16_HP];
  __shared__ __align__(16) float sp[AT_T * A16_SP];  // P^T, then dS^T, as [j][i]
  __shared__ float tred[3][NW][AT_HD];
  const int b = blockIdx.x / NH, h = blockIdx.x % NH;
  const int hd = D / NH;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  {
    float *const dst[4] = {sq, sk, sv, sg};
    const float *const src[4] = {Q, K, V, GO};
    stage16<4, 64 * NW>(dst, src, b, h, T, D, hd);
  }
  __syncthreads();
  const float inv_scale = 1.0f / (float)sqrt((double)hd);
  const int nt = (T + 15) >> 4;
  fx4 dsk[NU][8];  // dS^T of the wave's query tiles, kept for the gK pass
  float tq[8];    // gQ token-sum partials: value v = 4 half + r, d = 4*(l/16) + r + 16 half
#pragma unroll
  for (int v = 0; v < 8; ++v) tq[v] = 0.f;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int qt = tile_of<NW>(w, u);
    if (qt >= nt) continue;
    const int klim = causal ? qt : nt - 1;
    const int i = 16 * qt + (lane & 15);
    float4 qb[2], gb[2];
    rows16(qb, sq, i, lane);
    rows16(gb, sg, i, lane);
    fx4 pt[8];
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      if (kt <= klim) {
        pt[kt] = tile_t(sk, qb, kt, lane);
        dsk[u][kt] = tile_t(sv, gb, kt, lane);  // dP^T[j][i] = v_j . gO_i
      }
    probs16(pt, qt, klim, T, causal, inv_scale, lane);
    float rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      if (kt > klim) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * kt + 4 * (lane >> 4) + r;
        const bool live = j < T && !(causal && j > i);
        if (!live) dsk[u][kt][r] = 0.f;
        rs += dsk[u][kt][r] * pt[kt][r];
      }
    }
    rs += __shfl_xor(rs, 16, 64);
    rs += __shfl_xor(rs, 32, 64);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      if (kt > klim) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * kt + 4 * (lane >> 4) + r;
        const bool live = j < T && !(causal && j > i);
        const float p = pt[kt][r];
        dsk[u][kt][r] = live && i < T ? (dsk[u][kt][r] * p - p * rs) * inv_scale : 0.f;
        sp[j * A16_SP + i] = i < T ? p : 0.f;
      }
    }
    // gQ^T[d][i] = sum_j K[j][d] dS[i][j]
    fx4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      if (kt <= klim) keys_t(acc, sk, dsk[u][kt], kt, lane);
    store16_t(GQ, acc, b, h, T, D, hd, qt, lane);
    if (TS && i < T) {
#pragma unroll
      for (int v = 0; v < 8; ++v) tq[v] += acc[v >> 2][v & 3];
    }
  }
  if (TS) {
    // sum over the 16 queries of each lane group (lane bits 0-3): halving
    // butterfly, lane l ends with value ((l >> 1) & 7)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const bool up = (lane & 8) != 0;
      const float send = up ? tq[v] : tq[v + 4], keep = up ? tq[v + 4] : tq[v];
      tq[v] = keep + __shfl_xor(send, 8, 64);
    }
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const bool up = (lane & 4) != 0;
      const float send = up ? tq[v] : tq[v + 2], keep = up ? tq[v + 2] : tq[v];
      tq[v] = keep + __shfl_xor(send, 4, 64);
    }
    {
      const bool up = (lane & 2) != 0;
      const float send = up ? tq[0] : tq[1], keep = up ? tq[1] : tq[0];
      tq[0] = keep + __shfl_xor(send, 2, 64);
    }
    const float s = tq[0] + __shfl_xor(tq[0], 1, 64);
    const int v = (lane >> 1) & 7, d = 4 * (lane >> 4) + (v & 3) + 16 * (v >> 2);
    if ((lane & 1) == 0) tred[0][w][d] = s;
  }
  __syncthreads();
  // key side: wave w takes key tiles w and 7 - w; X[j][d] = sum_i Zt[j][i] Yq[i][d]
  // over the live query tiles (Zt[j][i] = 0 for i < j under the mask)
  auto keyside = [&](const float *Yq, float *G, int m) {
    float ts[2] = {0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int kt = tile_of<NW>(w, u);
      if (kt >= nt) continue;
      fx4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
      const float *zrow = sp + (16 * kt + (lane & 15)) * A16_SP + 4 * (lane >> 4);
      for (int qt = causal ? kt : 0; qt < nt; ++qt) {
        const float4 z = *reinterpret_cast<const float4 *>(zrow + 16 * qt);
        const float *y = Yq + (16 * qt + 4 * (lane >> 4)) * A16_HP + (lane & 15);
        acc[0] = mfma16(z.x, y[0], acc[0]);
        acc[1] = mfma16(z.x, y[16], acc[1]);
        acc[0] = mfma16(z.y, y[A16_HP], acc[0]);
        acc[1] = mfma16(z.y, y[A16_HP + 16], acc[1]);
        acc[0] = mfma16(z.z, y[2 * A16_HP], acc[0]);
        acc[1] = mfma16(z.z, y[2 * A16_HP + 16], acc[1]);
        acc[0] = mfma16(z.w, y[3 * A16_HP], acc[0]);
        acc[1] = mfma16(z.w, y[3 * A16_HP + 16], acc[1]);
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int d = 16 * half + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * kt + 4 * (lane >> 4) + r;
          if (j < T) {
            if (d < hd) G[((int64_t)b * T + j) * D + h * hd + d] = acc[half][r];
            ts[half] += acc[half][r];
          }
        }
      }
    }
    if (TS) {  // sum over the wave's keys of d = 16 half + l%16
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float s = ts[half];
        s += __shfl_xor(s, 16, 64);
        s += __shfl_xor(s, 32, 64);
        if (lane < 16) tred[m][w][16 * half + lane] = s;
      }
    }
  };
  keyside(sg, GV, 2);  // gV_j = sum_i p_ij gO_i
  __syncthreads();
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int qt = tile_of<NW>(w, u);
    if (qt >= nt) continue;
    const int klim = causal ? qt : nt - 1;
    const int i = 16 * qt + (lane & 15);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      if (kt > klim) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) sp[(16 * kt + 4 * (lane >> 4) + r) * A16_SP + i] = dsk[u][kt][r];
    }
  }
  __syncthreads();
  keyside(sq, GK, 1);  // gK_j = sum_i dS_ij q_i
  if (TS) {
    __syncthreads();
    const int m = threadIdx.x >> 5, d = threadIdx.x & 31;
    if (m < 3 && d < hd) {
      float v = tred[m][0][d];
#pragma unroll
      for (int q = 1; q < NW; ++q) v += tred[m][q][d];
      TS[m * tss + (int64_t)b * D + h * hd + d] = v;
    }
  }
}

constexpr int kAttnWaves = 8;  // waves per attention workgroup

static unsigned blocks_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 16384) b = 16384;
  return (unsigned)(b < 1 ? 1 : b);
}

hipError_t launch_embed(const float *x, const float *E, int32_t *ids, float *out, int B, int T, int V,
                        int D, int32_t *bad, hipStream_t s, bool bad_or) {
  if (B <= 0) return hipSuccess;
  const int64_t n = (int64_t)T * D;
  unsigned bx = (unsigned)std::min<int64_t>((n + 255) / 256, 64);
  hipLaunchKernelGGL(embed_kernel, dim3(bx, B), dim3(256), 0, s, x, E, ids, out, T, V, D, bad,
                     bad_or ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_embed_pe(const float *x, const float *E, const float *pe, int32_t *ids, float *out,
                           float *pe_out, int B, int T, int V, int D, int32_t *bad, hipStream_t s,
                           bool bad_or) {
  if (B <= 0) return hipSuccess;
  const int64_t n = (int64_t)T * D;
  unsigned bx = (unsigned)std::min<int64_t>((n + 255) / 256, 64);
  hipLaunchKernelGGL(embed_pe_kernel, dim3(bx, B), dim3(256), 0, s, x, E, pe, ids, out, pe_out, T, V, D, bad,
                     bad_or ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_pe_add(const float *x, const float *pe, float *out, int B, int TD, hipStream_t s) {
  const int64_t n = (int64_t)B * TD;
  hipLaunchKernelGGL(pe_add_kernel, dim3(blocks_for(n)), dim3(256), 0, s, x, pe, out, n, TD);
  return hipGetLastError();
}

static int embed_grad_rows(int B, int T, int W) {
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  const int chunk = (B + Wc - 1) / Wc;
  return ((B + chunk - 1) / chunk) * T;  // one contributing sample per chunk
}

bool embed_grad_takes_pe(int B, int T, int W) { return B > 0 && embed_grad_rows(B, T, W) <= EG_MAXL; }

bool embed_grad_upd_ok(int B, int T, int D, int W, const float *gradE, const float *rest, int64_t stride) {
  return B > 0 && embed_grad_rows(B, T, W) <= EG_MAXL && D % 4 == 0 && D <= 256 && stride > 0 &&
         stride % 4 == 0 && ((reinterpret_cast<uintptr_t>(gradE) | reinterpret_cast<uintptr_t>(rest)) & 15) == 0;
}

hipError_t launch_embed_grad(const float *g, const int32_t *ids, float *gradE, int V, int B, int T,
                             int D, int W, float scale, const int32_t *bad, hipStream_t s, float *ws,
                             size_t ws_floats, float *pe_grad, const AdamStep *upd) {
  const int Wc = W < 1 ? 1 : (W > B ? B : W);
  const int chunk = (B + Wc - 1) / Wc;
  const int L = embed_grad_rows(B, T, W);
  const int zb = (V + EG_ZR - 1) / EG_ZR;
  if (pe_grad && !embed_grad_takes_pe(B, T, W)) return hipErrorInvalidValue;
  AdamStep ad{};
  int nrest = 0;
  if (upd) {
    ad = *upd;
    if (!embed_grad_upd_ok(B, T, D, W, gradE, ad.rest, ad.stride)) return hipErrorInvalidValue;
    int64_t n4 = 0;
    for (int r = 0; r < 2; ++r) {
      if (ad.r1[r] < ad.r0[r] || ((ad.r0[r] | ad.r1[r]) & 3)) return hipErrorInvalidValue;
      n4 += (ad.r1[r] - ad.r0[r]) >> 2;
    }
    nrest = (int)std::min<int64_t>((n4 + 255) / 256, 16384);
  }
  if (L > EG_MAXL) {
    // the row lists in the caller's workspace: 2 L ints
    if (!ws || ws_floats < (size_t)2 * L) return hipErrorInvalidValue;
    int *sid = reinterpret_cast<int *>(ws);
    hipLaunchKernelGGL(embed_grad_prep, dim3((L + 255) / 256), dim3(256), 0, s, ids, B, T, chunk, L, bad,
                       W > 1 ? 1 : 0, sid);
    hipLaunchKernelGGL(embed_grad_global_kernel, dim3(L + zb), dim3(256), 0, s, g, sid, gradE, T, D, L,
                       scale, V);
    return hipGetLastError();
  }
  const int pb = pe_grad ? (int)(((int64_t)T * D + 255) / 256) : 0;
  hipLaunchKernelGGL(embed_grad_kernel, dim3(L + zb + pb + nrest), dim3(256), 0, s, g, ids, gradE, B, T, D, chunk,
                     L, scale, bad, W > 1 ? 1 : 0, V, pe_grad, ad, pb);
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
  return launch_token_sum_multi(X, S, B, T, N, 1, 0, 0, s);
}

hipError_t launch_token_sum_multi(const float *X, float *S, int B, int T, int N, int nmem,
                                  int64_t xstride, int64_t sstride, hipStream_t s) {
  if (B <= 0 || nmem <= 0) return hipSuccess;
  hipLaunchKernelGGL(token_sum_kernel, dim3((N + 63) / 64, B, nmem), dim3(1024), 0, s, X, S, B, T, N,
                     xstride, sstride);
  return hipGetLastError();
}

hipError_t launch_tok_dw(const TokDwSet &set, int nmem, int B, int M, int N, int lds, int ldx,
                         float scale, hipStream_t s) {
  if (nmem < 1 || nmem > 3) return hipErrorInvalidValue;
  if (M <= 0 || N <= 0) return hipSuccess;
  hipLaunchKernelGGL(tok_dw_kernel, dim3((N + TD_I - 1) / TD_I, (M + TD_O - 1) / TD_O, nmem), dim3(256), 0,
                     s, set, B, M, N, lds, ldx, scale);
  return hipGetLastError();
}

hipError_t launch_ln_fwd(const float *x, const float *gam, const float *bet, float *y, float *stats,
                         int rows, int N, float eps, hipStream_t s, float *cls, int clsT) {
  if (cls && clsT < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(ln_fwd_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, gam, bet, y, stats,
                     rows, N, eps, cls, clsT);
  return hipGetLastError();
}

// dx plus the gamma / beta gradients (scaled) through per-block partials in
// ws; hipErrorNotSupported when N or the partials do not fit.
hipError_t launch_ln_bwd_params(const float *g, const float *x, const float *gam, const float *stats,
                                float *dx, float *dgam, float *dbet, int rows, int N, float scale,
                                float *ws, size_t ws_cap, hipStream_t s) {
  const int nblk = (rows + LN_RPB - 1) / LN_RPB;
  if (N > 64 * LN_MAXC || (size_t)nblk * 2 * N > ws_cap) return hipErrorNotSupported;
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(ln_bwd_part_kernel, dim3(nblk), dim3(LN_NT), 0, s, g, nullptr, 1, x, gam, stats, dx, ws,
                     nullptr, rows, N, nblk, LnTokSum{});
  hipLaunchKernelGGL(ln_param_final, dim3((2 * N + 63) / 64), dim3(256), 0, s, ws, nblk, N, scale, dgam,
                     dbet);
  return hipGetLastError();
}

int ln_bwd_blocks(int rows) { return (rows + LN_RPB - 1) / LN_RPB; }
int ln_bwd_rows_per_block() { return LN_RPB; }
bool ln_bwd_part_supported(int N) { return N >= 1 && N <= 64 * LN_MAXC; }

hipError_t launch_ln_bwd_part(const float *g, const float *gpool, int poolT, const float *x,
                              const float *gam, const float *stats, float *dx, float *part, float *tsum,
                              int rows, int N, hipStream_t s, const float *tsx, float *tss, int tsB, int tsT,
                              int tsN) {
  if (!ln_bwd_part_supported(N) || (!g && !gpool) || (gpool && poolT < 1) || !part)
    return hipErrorInvalidValue;
  if (tsx && (!tss || tsB < 0 || tsT < 1 || tsN < 1)) return hipErrorInvalidValue;
  if (rows <= 0) return hipSuccess;
  const int nln = ln_bwd_blocks(rows);
  const int nts = tsx ? tsB * ((tsN + 63) / 64) : 0;
  hipLaunchKernelGGL(ln_bwd_part_kernel, dim3(nln + nts), dim3(LN_NT), 0, s, g, gpool, gpool ? poolT : 1, x, gam,
                     stats, dx, part, tsum, rows, N, nln, LnTokSum{tsx, tss, tsT, tsN});
  return hipGetLastError();
}

hipError_t launch_tb_params(TbParamSet &set, int B, float scale, hipStream_t s) {
  if (set.nlin < 0 || set.nlin > TBP_MAXLIN || set.nln < 0 || set.nln > TBP_MAXLN)
    return hipErrorInvalidValue;
  int n = 0, j = 0;
  for (int k = 0; k < set.nln; ++k, ++j) {
    const TbLnJob &q = set.ln[k];
    if (q.N < 0 || q.nblk < 1 || !q.part || !q.dgam || !q.dbet) return hipErrorInvalidValue;
    set.start[j] = n;
    n += (2 * q.N + 63) / 64;
  }
  for (int k = 0; k < set.nlin; ++k, ++j) {
    const TbParamJob &p = set.lin[k];
    if (p.M < 0 || p.N < 0 || p.np < 1 || !p.S || !p.X || !p.dW || !p.db) return hipErrorInvalidValue;
    set.start[j] = n;
    n += ((p.N + TD_I - 1) / TD_I) * ((p.M + TD_O - 1) / TD_O);
  }
  set.start[j] = n;
  if (n == 0 || B <= 0) return hipSuccess;
  hipLaunchKernelGGL(tb_param_kernel, dim3(n), dim3(256), 0, s, set, B, scale);
  return hipGetLastError();
}

hipError_t launch_ln_bwd(const float *g, const float *x, const float *gam, const float *stats,
                         float *dx, float *gx, int rows, int N, hipStream_t s) {
  hipLaunchKernelGGL(ln_bwd_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, g, x, gam, stats, dx, gx,
                     rows, N);
  return hipGetLastError();
}

hipError_t launch_rope(float *x, const float *cs, const float *sn, int rows, int T, int NH, int hd,
                       int conj, hipStream_t s) {
  const int64_t total = (int64_t)rows * NH * (hd / 2);
  if (total <= 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, cs, sn, total, T, NH, hd,
                     conj);
  return hipGetLastError();
}

hipError_t launch_rms_fwd(const float *x, const float *gam, float *y, float *rms, int rows, int N,
                          float eps, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(rms_fwd_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, gam, y, rms, rows, N,
                     eps);
  return hipGetLastError();
}

hipError_t launch_rms_bwd(const float *g, const float *x, const float *gam, const float *rms,
                          float *dx, float *gx, int rows, int N, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(rms_bwd_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, g, x, gam, rms, dx, gx,
                     rows, N);
  return hipGetLastError();
}

bool attn_supported(int T, int D, int NH) {
  return NH > 0 && D % NH == 0 && T >= 1 && T <= AT_T && D / NH <= AT_HD;
}

// ---------------------------------------------------------------------------
// Attention of any sequence length and head size (the fused kernels above
// hold T <= 128 keys and 32-wide heads in LDS).  The scores of every (sample,
// head) pair are materialised: S = Q_h K_h^T by one batched MFMA GEMM over
// the B x NH pairs (each a T x hd slice of the [B*T, D] matrices), a row
// kernel applies the mask, the scale and the reference's row softmax, and a
// second batched GEMM forms O_h = P V_h.  The backward recomputes P, forms
// dP = gO_h V_h^T, turns it into gradScore = P (dP - sum_k dP_k P_k) / sqrt(hd)
// in a row kernel (masked entries 0, transformer.go:583-630), and takes
// gQ = G K_h, gK = G^T Q_h, gV = P^T gO_h as three batched GEMMs.
// ---------------------------------------------------------------------------

// Row r of S (member r / T, query i = r % T): masked keys j > i take -1e9,
// the rest s / sqrt(hd) (transformer.go:466-477); then activations.go:161-183:
// row max, exp of (x - max) in float64 rounded to float32, float32 sum, divide.
__global__ __launch_bounds__(256) void attn_softmax_rows(float *__restrict__ S, int64_t rows, int T,
                                                         int causal, float scale) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const int i = (int)(r % T);
  float *row = S + r * T;
  float mx = -__builtin_inff();
  for (int j = lane; j < T; j += 64) {
    const float v = (causal && j > i) ? -1e9f : row[j] / scale;
    row[j] = v;
    mx = fmaxf(mx, v);
  }
  mx = wmax(mx);
  float sum = 0.f;
  for (int j = lane; j < T; j += 64) {
    const float e = (float)exp((double)(row[j] - mx));
    row[j] = e;
    sum += e;
  }
  sum = wsum(sum);
  for (int j = lane; j < T; j += 64) row[j] = row[j] / sum;
}

// G (holding dP) <- P (dP - sum_k dP_k P_k) / sqrt(hd) on unmasked keys, 0 on
// masked ones (their gradRow entries are never formed, transformer.go:595-606)
__global__ __launch_bounds__(256) void attn_dscore_rows(const float *__restrict__ P, float *__restrict__ G,
                                                        int64_t rows, int T, int causal, float scale) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const int i = (int)(r % T);
  const float *p = P + r * T;
  float *g = G + r * T;
  float d = 0.f;
  for (int j = lane; j < T; j += 64)
    if (!(causal && j > i)) d += g[j] * p[j];
  d = wsum(d);
  for (int j = lane; j < T; j += 64) g[j] = (causal && j > i) ? 0.f : (p[j] * (g[j] - d)) / scale;
}

size_t attn_gemm_floats(int B, int T, int NH) { return 2 * (size_t)B * NH * T * T; }

namespace {
// One batched GEMM over the (sample, head) pairs.  Operands are either a
// head slice of a [B*T, D] matrix (sample stride T*D, head stride hd, row
// pitch D) or a T x T block of the score buffer (stride T*T per pair).
struct HeadOp {
  const float *p;
  bool scores;
};
hipError_t pair_gemm(char ta, char tb, int M, int N, int K, HeadOp A, HeadOp Bm, float *C, bool c_scores,
                     int B, int T, int D, int NH, hipStream_t s) {
  const int hd = D / NH;
  const int64_t TT = (int64_t)T * T;
  GemmArgs a{};
  a.M = M;
  a.N = N;
  a.K = K;
  a.alpha = 1.f;
  a.nbatch = B * NH;
  a.nbatch_in = NH;
  auto set = [&](HeadOp o, const float *&ptr, int &ld, int64_t &bs, int64_t &is) {
    ptr = o.p;
    ld = o.scores ? T : D;
    bs = o.scores ? NH * TT : (int64_t)T * D;
    is = o.scores ? TT : hd;
  };
  set(A, a.A, a.lda, a.bstride_A, a.istride_A);
  set(Bm, a.B, a.ldb, a.bstride_B, a.istride_B);
  const float *cp = nullptr;
  set(HeadOp{C, c_scores}, cp, a.ldc, a.bstride_C, a.istride_C);
  a.C = C;
  // the batch index is the grid's z dimension (at most 65535): samples in
  // chunks whose (sample, head) pairs fit it, each chunk's operands advanced
  // by whole samples
  const int per = std::max(1, 65535 / NH);
  for (int b0 = 0; b0 < B; b0 += per) {
    const int nb = std::min(per, B - b0);
    GemmArgs c = a;
    c.nbatch = nb * NH;
    c.A = a.A + (int64_t)b0 * a.bstride_A;
    c.B = a.B + (int64_t)b0 * a.bstride_B;
    c.C = a.C + (int64_t)b0 * a.bstride_C;
    const hipError_t e = launch_gemm(ta, tb, EPI_SCALE, c, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}
hipError_t softmax_scores(float *S, int B, int T, int NH, int hd, int causal, hipStream_t s) {
  const int64_t rows = (int64_t)B * NH * T;
  hipLaunchKernelGGL(attn_softmax_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, S, rows, T, causal,
                     (float)sqrt((double)hd));
  return hipGetLastError();
}
}  // namespace

hipError_t launch_attn_fwd_gemm(const float *Q, const float *K, const float *V, float *O, int B, int T,
                                int D, int NH, int causal, float *S, hipStream_t s) {
  const int hd = D / NH;
  hipError_t e = pair_gemm('N', 'T', T, T, hd, {Q, false}, {K, false}, S, true, B, T, D, NH, s);
  if (e == hipSuccess) e = softmax_scores(S, B, T, NH, hd, causal, s);
  if (e == hipSuccess) e = pair_gemm('N', 'N', T, hd, T, {S, true}, {V, false}, O, false, B, T, D, NH, s);
  return e;
}

hipError_t launch_attn_bwd_gemm(const float *Q, const float *K, const float *V, const float *GO,
                                float *GQ, float *GK, float *GV, int B, int T, int D, int NH, int causal,
                                float *S, hipStream_t s) {
  const int hd = D / NH;
  float *P = S, *G = S + (size_t)B * NH * T * T;
  hipError_t e = pair_gemm('N', 'T', T, T, hd, {Q, false}, {K, false}, P, true, B, T, D, NH, s);
  if (e == hipSuccess) e = softmax_scores(P, B, T, NH, hd, causal, s);
  if (e == hipSuccess) e = pair_gemm('N', 'T', T, T, hd, {GO, false}, {V, false}, G, true, B, T, D, NH, s);
  if (e == hipSuccess) {
    const int64_t rows = (int64_t)B * NH * T;
    hipLaunchKernelGGL(attn_dscore_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, P, G, rows, T,
                       causal, (float)sqrt((double)hd));
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = pair_gemm('N', 'N', T, hd, T, {G, true}, {K, false}, GQ, false, B, T, D, NH, s);
  if (e == hipSuccess) e = pair_gemm('T', 'N', T, hd, T, {G, true}, {Q, false}, GK, false, B, T, D, NH, s);
  if (e == hipSuccess) e = pair_gemm('T', 'N', T, hd, T, {P, true}, {GO, false}, GV, false, B, T, D, NH, s);
  return e;
}

// GlobalAveragePooling1D (transformer.go:1541-1600): out[b][i] = (sum over
// s of x[b][s][i], in increasing s, float32) / float32(T); the backward
// gives every position g[b][i] / float32(T).
__global__ __launch_bounds__(256) void gap1d_fwd_kernel(const float *__restrict__ x, float *__restrict__ out,
                                                        int64_t BD, int T, int D) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= BD) return;
  const int64_t b = e / D, i = e - b * D;
  const float *p = x + b * T * D + i;
  float sum = 0.f;
  int s = 0;
  for (; s + 4 <= T; s += 4) {  // four loads in flight, added in order
    const float v0 = p[(int64_t)s * D], v1 = p[(int64_t)(s + 1) * D], v2 = p[(int64_t)(s + 2) * D],
                v3 = p[(int64_t)(s + 3) * D];
    sum += v0;
    sum += v1;
    sum += v2;
    sum += v3;
  }
  for (; s < T; ++s) sum += p[(int64_t)s * D];
  out[e] = sum / (float)T;
}

__global__ __launch_bounds__(256) void gap1d_bwd_kernel(const float *__restrict__ g, float *__restrict__ gin,
                                                        int64_t n, int T, int D) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t TD = (int64_t)T * D, b = e / TD, i = e % D;
  gin[e] = g[b * D + i] / (float)T;
}

hipError_t launch_gap1d_fwd(const float *x, float *out, int B, int T, int D, hipStream_t s) {
  const int64_t BD = (int64_t)B * D;
  hipLaunchKernelGGL(gap1d_fwd_kernel, dim3((unsigned)((BD + 255) / 256)), dim3(256), 0, s, x, out, BD, T, D);
  return hipGetLastError();
}

hipError_t launch_gap1d_bwd(const float *g, float *gin, int B, int T, int D, hipStream_t s) {
  const int64_t n = (int64_t)B * T * D;
  hipLaunchKernelGGL(gap1d_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, gin, n, T, D);
  return hipGetLastError();
}

hipError_t launch_attn_fwd(const float *Q, const float *K, const float *V, float *O, int B, int T,
                           int D, int NH, int causal, hipStream_t s) {
  if (!attn_supported(T, D, NH)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attn16_fwd_kernel<kAttnWaves>, dim3(B * NH), dim3(64 * kAttnWaves), 0, s, Q, K, V, O, T, D,
                     NH, causal);
  return hipGetLastError();
}

hipError_t launch_attn_bwd(const float *Q, const float *K, const float *V, const float *GO,
                           float *GQ, float *GK, float *GV, int B, int T, int D, int NH, int causal,
                           hipStream_t s, float *TS, int64_t tss) {
  if (!attn_supported(T, D, NH)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attn16_bwd_kernel<kAttnWaves>, dim3(B * NH), dim3(64 * kAttnWaves), 0, s, Q, K, V, GO, GQ,
                     GK, GV, T, D, NH, causal, TS, tss);
  return hipGetLastError();
}

}  // namespace gn
