// fp32 MFMA GEMM family for gfx950 (CDNA4).
//
// C[M,N] = epilogue( sum_k opA[m,k] * opB[k,n] ) with both operands staged
// through LDS in a K-contiguous, padded layout so every lane fetches its MFMA
// operands with ds_read_b128.
//
// Tiling: 128x128 block tile, BK = 32, 256 threads = 4 wave64s in a 2x2 grid,
// each wave owns a 64x64 sub-tile = 2x2 v_mfma_f32_32x32x2_f32 accumulators
// (64 fp32 accumulators per lane).  Within a K tile, lane half h (lanes 32-63)
// feeds k = 16h + s at MFMA step s, so each lane's 16 operand values per tile
// row are contiguous in LDS.  Two LDS stages: global loads for tile k+1 are
// issued into registers before the MFMAs of tile k and written to the other
// stage afterwards, one barrier per K tile.
//
// Used by Dense forward (NT: X[B,in] * W[out,in]^T, fused bias + activation),
// Dense dX (NN: dZ[B,out] * W[out,in], fused activation derivative of the layer
// below) and Dense dW (TN: dZ^T X scaled by 1/B), the batched replacements of
// the per-sample mat-vecs in layer.go:406, :591-663.
#include "gn_common.h"

namespace gn {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 32;
constexpr int PITCH = BK + 4;  // floats; 16 B pad keeps b128 row reads conflict-free
constexpr int NT = 256;

__device__ __forceinline__ float apply_fwd(float v, int kind) {
  switch (kind) {
    case F_RELU: return v > 0.0f ? v : 0.0f;
    case F_SIGMOID: return 1.0f / (1.0f + (float)exp((double)(-v)));
    case F_TANH: return (float)tanh((double)v);
    case F_NAN: return __builtin_nanf("");
    default: return v;
  }
}

__device__ __forceinline__ float apply_deriv(float out, int kind) {
  switch (kind) {
    case D_RELU: return out > 0.0f ? 1.0f : 0.0f;
    case D_SIGMOID: return out * (1.0f - out);
    case D_TANH: return 1.0f - out * out;
    case D_NAN: return __builtin_nanf("");
    default: return 1.0f;
  }
}

// Global -> register staging of one operand tile.  KC: the operand's K index
// is contiguous in memory (rows x K, row pitch ld); otherwise it is stored
// K x rows.  VEC: float4 accesses are legal (16 B aligned, sizes % 4 == 0).
template <bool KC, bool VEC>
__device__ __forceinline__ void load_tile(const float *__restrict__ base, int ld, int rows, int K,
                                          int r0, int k0, float4 (&reg)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = t + NT * j;
    if (KC) {
      const int r = f >> 3, k4 = (f & 7) << 2;
      const int gr = r0 + r, gk = k0 + k4;
      if (VEC) {
        if (gr < rows && gk < K)
          reg[j] = *reinterpret_cast<const float4 *>(base + (size_t)gr * ld + gk);
        else
          reg[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float *p = base + (size_t)gr * ld + gk;
        const bool ok = gr < rows;
        reg[j].x = (ok && gk + 0 < K) ? p[0] : 0.f;
        reg[j].y = (ok && gk + 1 < K) ? p[1] : 0.f;
        reg[j].z = (ok && gk + 2 < K) ? p[2] : 0.f;
        reg[j].w = (ok && gk + 3 < K) ? p[3] : 0.f;
      }
    } else {
      const int k = f >> 5, r4 = (f & 31) << 2;
      const int gk = k0 + k, gr = r0 + r4;
      if (VEC) {
        if (gk < K && gr < rows)
          reg[j] = *reinterpret_cast<const float4 *>(base + (size_t)gk * ld + gr);
        else
          reg[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float *p = base + (size_t)gk * ld + gr;
        const bool ok = gk < K;
        reg[j].x = (ok && gr + 0 < rows) ? p[0] : 0.f;
        reg[j].y = (ok && gr + 1 < rows) ? p[1] : 0.f;
        reg[j].z = (ok && gr + 2 < rows) ? p[2] : 0.f;
        reg[j].w = (ok && gr + 3 < rows) ? p[3] : 0.f;
      }
    }
  }
}

template <bool KC>
__device__ __forceinline__ void store_tile(float (*S)[PITCH], const float4 (&reg)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = t + NT * j;
    if (KC) {
      const int r = f >> 3, k4 = (f & 7) << 2;
      *reinterpret_cast<float4 *>(&S[r][k4]) = reg[j];
    } else {
      const int k = f >> 5, r4 = (f & 31) << 2;
      S[r4 + 0][k] = reg[j].x;
      S[r4 + 1][k] = reg[j].y;
      S[r4 + 2][k] = reg[j].z;
      S[r4 + 3][k] = reg[j].w;
    }
  }
}

// Block -> tile mapping.  Workgroups are dispatched round-robin over the 8
// XCDs (each with its own L2), so consecutive block ids land on different
// XCDs.  Remap so that each XCD receives a contiguous range of tile ids, and
// walk tiles in groups of GROUP_M tile rows so that neighbouring blocks on one
// XCD share A rows and B columns in that XCD's L2.
__device__ __forceinline__ void tile_of_block(int tiles_m, int tiles_n, int &tm, int &tn) {
  const int nblk = tiles_m * tiles_n;
  int pid = blockIdx.x;
  constexpr int NXCD = 8;
  if (nblk >= NXCD * 4 && nblk % NXCD == 0) {
    const int per = nblk / NXCD;
    pid = (pid % NXCD) * per + pid / NXCD;
  }
  constexpr int GROUP_M = 4;
  const int width = GROUP_M * tiles_n;
  const int group = pid / width;
  const int first_m = group * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  tm = first_m + (pid % width) % gsz;
  tn = (pid % width) / gsz;
}

template <bool AK, bool BKC, bool VEC, int EPI>
__global__ __launch_bounds__(NT) void gemm_f32_mfma(GemmArgs p, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(16))) float As[2][BM][PITCH];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN][PITCH];

  int tm, tn;
  tile_of_block(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int half = lane >> 5, l32 = lane & 31;
  const int M = p.M, N = p.N, K = p.K;
  const int nk = (K + BK - 1) / BK;

  float4 ra[4], rb[4];
  load_tile<AK, VEC>(p.A, p.lda, M, K, m0, 0, ra);
  load_tile<BKC, VEC>(p.B, p.ldb, N, K, n0, 0, rb);
  store_tile<AK>(As[0], ra);
  store_tile<BKC>(Bs[0], rb);
  __syncthreads();

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      load_tile<AK, VEC>(p.A, p.lda, M, K, m0, (kt + 1) * BK, ra);
      load_tile<BKC, VEC>(p.B, p.ldb, N, K, n0, (kt + 1) * BK, rb);
    }
    float a[2][16], b[2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float *src = &As[cur][wm * 64 + i * 32 + l32][half * 16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 x = *reinterpret_cast<const float4 *>(src + 4 * q);
        a[i][4 * q + 0] = x.x;
        a[i][4 * q + 1] = x.y;
        a[i][4 * q + 2] = x.z;
        a[i][4 * q + 3] = x.w;
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float *src = &Bs[cur][wn * 64 + j * 32 + l32][half * 16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 x = *reinterpret_cast<const float4 *>(src + 4 * q);
        b[j][4 * q + 0] = x.x;
        b[j][4 * q + 1] = x.y;
        b[j][4 * q + 2] = x.z;
        b[j][4 * q + 3] = x.w;
      }
    }
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
    if (more) {
      store_tile<AK>(As[cur ^ 1], ra);
      store_tile<BKC>(Bs[cur ^ 1], rb);
    }
    __syncthreads();
  }

  // Epilogue.  v_mfma_f32_32x32x2_f32 result layout: lane l, accumulator r
  // holds row 8*(r/4) + 4*(l/32) + r%4, column l%32 of the 32x32 tile.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + l32;
      if (col >= N) continue;
      float bias = 0.f;
      if (EPI == EPI_BIAS_ACT && p.bias) bias = p.bias[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
        if (row >= M) continue;
        float v = acc[i][j][r];
        if (EPI == EPI_SCALE) {
          v *= p.alpha;
        } else if (EPI == EPI_BIAS_ACT) {
          v = apply_fwd(v + bias, p.act);
        } else {
          v *= apply_deriv(p.aux[(size_t)row * p.ldaux + col], p.act);
        }
        p.C[(size_t)row * p.ldc + col] = v;
      }
    }
}

template <bool AK, bool BKC, int EPI>
static hipError_t launch_t(bool vec, const GemmArgs &a, hipStream_t s) {
  const int tm = (a.M + BM - 1) / BM, tn = (a.N + BN - 1) / BN;
  dim3 grid(tm * tn), block(NT);
  if (vec)
    hipLaunchKernelGGL((gemm_f32_mfma<AK, BKC, true, EPI>), grid, block, 0, s, a, tm, tn);
  else
    hipLaunchKernelGGL((gemm_f32_mfma<AK, BKC, false, EPI>), grid, block, 0, s, a, tm, tn);
  return hipGetLastError();
}

template <int EPI>
static hipError_t launch_e(char ta, char tb, bool vec, const GemmArgs &a, hipStream_t s) {
  // op(A) 'N' -> A is M x K, K contiguous.  op(B) 'T' -> B is N x K, K contiguous.
  const bool ak = (ta == 'N');
  const bool bk = (tb == 'T');
  if (ak && bk) return launch_t<true, true, EPI>(vec, a, s);
  if (ak && !bk) return launch_t<true, false, EPI>(vec, a, s);
  if (!ak && bk) return launch_t<false, true, EPI>(vec, a, s);
  return launch_t<false, false, EPI>(vec, a, s);
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

hipError_t launch_gemm(char ta, char tb, int epi, const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  // float4 staging needs 16 B aligned rows and the contiguous extent % 4 == 0
  const bool ak = (ta == 'N'), bk = (tb == 'T');
  bool vec = aligned16(a.A) && aligned16(a.B) && (a.lda % 4 == 0) && (a.ldb % 4 == 0);
  vec = vec && (ak ? (a.K % 4 == 0) : (a.M % 4 == 0));
  vec = vec && (bk ? (a.K % 4 == 0) : (a.N % 4 == 0));
  if (epi == EPI_BIAS_ACT) return launch_e<EPI_BIAS_ACT>(ta, tb, vec, a, s);
  if (epi == EPI_DACT) return launch_e<EPI_DACT>(ta, tb, vec, a, s);
  return launch_e<EPI_SCALE>(ta, tb, vec, a, s);
}

}  // namespace gn
