// fp32 MFMA GEMM family for gfx950 (CDNA4).
//
// C[M,N] = epilogue( sum_k opA[m,k] * opB[k,n] ) with both operands staged
// through LDS.  A K-contiguous operand is stored [row][k] (padded) and each lane
// fetches its 16 MFMA operands per K tile with 4 ds_read_b128; an M/N-contiguous
// operand keeps its global layout in LDS (no transposing scalar stores) and is
// read with ds_read_b32 by consecutive lanes.
//
// Tiling: R x R block tile (R = 128, or 64 for grids that 128-wide tiles
// cannot fill), 64-wide K stages, 512 threads = 8 wave64s in two K-groups.
// Group g owns k in [32g, 32g+32) of every stage; inside a group the 4 waves
// tile the block 2x2, each wave an (R/2)x(R/2) sub-tile of
// v_mfma_f32_32x32x2_f32 accumulators (2x2 of them, 64 fp32 per lane, at
// R = 128).  The two groups' partial sums are added through LDS before the
// epilogue.  With a
// 1024-row batch a 4096-wide layer has exactly 256 tiles (one per CU): the
// K-groups give every SIMD two waves to hide LDS and barrier latency.  Lane
// half h feeds k = 16h + s at MFMA step s, so each lane's 16 operand values per
// slab are contiguous for a K-contiguous operand.  Two LDS stages, one
// barrier per stage.  When every tile and K stage lies inside the matrices the
// main loop is software-pipelined (the barrier sits before the last quarter
// of a stage's MFMAs, fragment halves are double-buffered in registers, global
// loads are issued about one stage before their LDS writes, and
// __builtin_amdgcn_sched_group_barrier fixes the interleave); otherwise a
// bounds-checked loop prefetches one stage into registers.  When the tile
// grid cannot fill the 256 CUs the K range is split across blocks; the partial
// sums are added in split order by a second kernel that also applies the
// epilogue.
//
// 128-wide tiles whose K ranges are whole stages run a four-wave variant
// instead (gemm_f32_mfma_w4): one wave per 64 x 64 sub-tile over the whole K
// range, operands fetched with direct global -> LDS loads (no staging
// registers, no LDS store instructions), fragment reads and loads issued one
// per MFMA.  With at least two tiles per CU it uses 32-deep stages so that two
// blocks share a CU and one block's prologue, barriers and epilogue overlap
// the other's MFMAs.
//
// Used by Dense forward (NT: X[B,in] * W[out,in]^T, fused bias + activation),
// Dense dX (NN: dZ[B,out] * W[out,in], fused activation derivative of the layer
// below) and Dense dW (TN: dZ^T X scaled by 1/B), the batched replacements of
// the per-sample mat-vecs in layer.go:406, :591-663.
#include "gn_common.h"

#include <algorithm>

namespace gn {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;          // K staged per iteration (two 32-wide halves)
constexpr int PITCH = BK + 4;   // floats; 16 B pad keeps b128 row reads conflict-free
constexpr int NT = 512;         // 8 wave64s: 2 K-groups x (2 x 2) waves

// Per-tile-size constants: R rows (and columns) per block tile.
template <int R>
struct Tile {
  static constexpr int T = R / 64;            // 32x32 MFMA tiles per wave per dimension
  static constexpr int RP = R + 4;            // pitch of an M/N-contiguous operand in LDS
  static constexpr int STAGE = (R * PITCH > BK * RP) ? R * PITCH : BK * RP;  // floats
  static constexpr int NLD = R / 32;          // float4 loads per thread per operand tile
  static constexpr int QPL = T * T * 4;       // float4 accumulator groups per lane
};

__device__ __forceinline__ float apply_fwd(float v, int kind) {
  switch (kind) {
    case F_RELU: return v > 0.0f ? v : 0.0f;
    case F_SIGMOID: return 1.0f / (1.0f + (float)exp((double)(-v)));
    case F_TANH: return (float)tanh((double)v);
    case F_NAN: return __builtin_nanf("");
    case F_LEAKY: return v > 0.0f ? v : 0.1f * v;
    default: return v;
  }
}

__device__ __forceinline__ float apply_deriv(float out, int kind) {
  switch (kind) {
    case D_RELU: return out > 0.0f ? 1.0f : 0.0f;
    case D_SIGMOID: return out * (1.0f - out);
    case D_TANH: return 1.0f - out * out;
    case D_NAN: return __builtin_nanf("");
    case D_GELU: return gelu_deriv(out);
    default: return 1.0f;
  }
}

// Global -> register staging of one R-row operand tile.  KC: the operand's K
// index is contiguous in memory (rows x K, row pitch ld); otherwise it is
// stored K x rows.  VEC: float4 accesses are legal (16 B aligned, sizes % 4 ==
// 0).  Only k in [k0, kend) is read; everything else is zero-filled.
template <int R, bool KC, bool VEC>
__device__ __forceinline__ void load_tile(const float *__restrict__ base, int ld, int rows, int kend,
                                          int r0, int k0, float4 (&reg)[Tile<R>::NLD]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < Tile<R>::NLD; ++j) {
    const int f = t + NT * j;
    if (KC) {
      const int r = f >> 4, k4 = (f & 15) << 2;
      const int gr = r0 + r, gk = k0 + k4;
      if (VEC) {
        if (gr < rows && gk < kend)
          reg[j] = *reinterpret_cast<const float4 *>(base + (size_t)gr * ld + gk);
        else
          reg[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float *p = base + (size_t)gr * ld + gk;
        const bool ok = gr < rows;
        reg[j].x = (ok && gk + 0 < kend) ? p[0] : 0.f;
        reg[j].y = (ok && gk + 1 < kend) ? p[1] : 0.f;
        reg[j].z = (ok && gk + 2 < kend) ? p[2] : 0.f;
        reg[j].w = (ok && gk + 3 < kend) ? p[3] : 0.f;
      }
    } else {
      const int k = f / (R / 4), r4 = (f % (R / 4)) << 2;
      const int gk = k0 + k, gr = r0 + r4;
      if (VEC) {
        if (gk < kend && gr < rows)
          reg[j] = *reinterpret_cast<const float4 *>(base + (size_t)gk * ld + gr);
        else
          reg[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float *p = base + (size_t)gk * ld + gr;
        const bool ok = gk < kend;
        reg[j].x = (ok && gr + 0 < rows) ? p[0] : 0.f;
        reg[j].y = (ok && gr + 1 < rows) ? p[1] : 0.f;
        reg[j].z = (ok && gr + 2 < rows) ? p[2] : 0.f;
        reg[j].w = (ok && gr + 3 < rows) ? p[3] : 0.f;
      }
    }
  }
}

// LDS layouts.  K-contiguous operands: [R rows][68] (k fastest, 16 B pad),
// read as 4 x ds_read_b128 per lane.  M/N-contiguous operands keep their
// global layout, [64 k][R + 4] (row fastest), written with ds_write_b128 and
// read as 16 x ds_read_b32 per lane (consecutive lanes, consecutive rows).
template <int R, bool KC>
__device__ __forceinline__ void store_tile(float *S, const float4 (&reg)[Tile<R>::NLD]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < Tile<R>::NLD; ++j) {
    const int f = t + NT * j;
    if (KC) {
      const int r = f >> 4, k4 = (f & 15) << 2;
      *reinterpret_cast<float4 *>(S + r * PITCH + k4) = reg[j];
    } else {
      const int k = f / (R / 4), r4 = (f % (R / 4)) << 2;
      *reinterpret_cast<float4 *>(S + k * Tile<R>::RP + r4) = reg[j];
    }
  }
}

// MFMA operand fragment of one 32-row slab for K-group g: lane half h
// supplies k = 32g + 16h + s at step s (s = 0..15), row = rowbase + lane % 32.
template <int R, bool KC>
__device__ __forceinline__ void read_frag(const float *S, int rowbase, int koff, int l32,
                                          float (&a)[16]) {
  if (KC) {
    const float *src = S + (rowbase + l32) * PITCH + koff;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 x = *reinterpret_cast<const float4 *>(src + 4 * q);
      a[4 * q + 0] = x.x;
      a[4 * q + 1] = x.y;
      a[4 * q + 2] = x.z;
      a[4 * q + 3] = x.w;
    }
  } else {
    const float *src = S + koff * Tile<R>::RP + rowbase + l32;
#pragma unroll
    for (int s = 0; s < 16; ++s) a[s] = src[s * Tile<R>::RP];
  }
}

// Staging for the pipelined loop, in native vector types (a float4 struct
// copy through a register array can leave the array in scratch memory).
// Rows past the matrix edge re-read its last valid row or float4 (their
// results are never stored).  With KT, k past kend reads a valid address and
// the store replaces it by zeros (the select waits at the store, where the
// load has to be complete anyway), which adds exact zeros to every sum like
// the checked loop.  Needs the float4 legality of the checked loop's VEC case
// (16 B aligned rows, contiguous extent % 4 == 0).
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int R, bool KC, bool KT>
__device__ __forceinline__ void load_tile_pipe(const float *__restrict__ base, int ld, int rows,
                                               int kend, int r0, int k0,
                                               floatx4 (&reg)[Tile<R>::NLD]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < Tile<R>::NLD; ++j) {
    const int f = t + NT * j;
    if (KC) {
      const int r = f >> 4, k4 = (f & 15) << 2;
      const int gr = min(r0 + r, rows - 1), gk = KT ? min(k0 + k4, kend - 4) : k0 + k4;
      reg[j] = *reinterpret_cast<const floatx4 *>(base + (size_t)gr * ld + gk);
    } else {
      const int k = f / (R / 4), r4 = (f % (R / 4)) << 2;
      const int gr = min(r0 + r4, rows - 4), gk = KT ? min(k0 + k, kend - 1) : k0 + k;
      reg[j] = *reinterpret_cast<const floatx4 *>(base + (size_t)gk * ld + gr);
    }
  }
}

template <int R, bool KC, bool KT>
__device__ __forceinline__ void store_tile_pipe(float *S, const floatx4 (&reg)[Tile<R>::NLD], int k0,
                                                int kend) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < Tile<R>::NLD; ++j) {
    const int f = t + NT * j;
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    if (KC) {
      const int r = f >> 4, k4 = (f & 15) << 2;
      *reinterpret_cast<floatx4 *>(S + r * PITCH + k4) = (!KT || k0 + k4 < kend) ? reg[j] : zero;
    } else {
      const int k = f / (R / 4), r4 = (f % (R / 4)) << 2;
      *reinterpret_cast<floatx4 *>(S + k * Tile<R>::RP + r4) = (!KT || k0 + k < kend) ? reg[j] : zero;
    }
  }
}

// Half a fragment: MFMA steps s = 8h .. 8h+7 of read_frag (koff advanced by 8h).
template <int R, bool KC>
__device__ __forceinline__ void read_frag_half(const float *S, int rowbase, int koff, int l32,
                                               float (&a)[8]) {
  if (KC) {
    const float *src = S + (rowbase + l32) * PITCH + koff;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const floatx4 x = *reinterpret_cast<const floatx4 *>(src + 4 * q);
      a[4 * q + 0] = x[0];
      a[4 * q + 1] = x[1];
      a[4 * q + 2] = x[2];
      a[4 * q + 3] = x[3];
    }
  } else {
    const float *src = S + koff * Tile<R>::RP + rowbase + l32;
#pragma unroll
    for (int s = 0; s < 8; ++s) a[s] = src[s * Tile<R>::RP];
  }
}

// Both fragment halves' slabs of a wave (T slabs).  With T = 2 an
// M/N-contiguous operand is read pairwise: lane l takes rows 2*(l%32) and
// 2*(l%32)+1 with one ds_read_b64, the even row feeding slab 0 and the odd row
// slab 1, so a slab holds every other row of the wave's 64 (the epilogue maps
// rows back; each output's K order is unchanged).
template <int R, bool KC>
__device__ __forceinline__ void read_frags(const float *S, int rowbase, int koff, int l32,
                                           float (&a)[Tile<R>::T][8]) {
  constexpr int T = Tile<R>::T;
  if (KC || T != 2) {
#pragma unroll
    for (int i = 0; i < T; ++i) read_frag_half<R, KC>(S, rowbase + i * 32, koff, l32, a[i]);
  } else {
    const float *src = S + koff * Tile<R>::RP + rowbase + 2 * l32;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float2 x = *reinterpret_cast<const float2 *>(src + s * Tile<R>::RP);
      a[0][s] = x.x;
      a[T - 1][s] = x.y;
    }
  }
}

// Direct global -> LDS staging (gfx950 global_load_lds_dwordx4).  One wave
// instruction writes its 64 lanes' 16 B contiguously from an LDS base held in
// M0, so the LDS layout follows the lane order and is chosen through the
// global address each lane fetches: float4 slot f = t + NT*j of a stage lands
// at LDS float 4f.  No staging registers and no LDS store instructions; the
// data is in LDS once the wave's vmcnt has drained past the load.
//   K-contiguous operand: [R rows][64 k], unpadded; the 16 float4 chunks of
//   row r are XOR-swizzled by r & 15 (slot f is row f >> 4, physical chunk
//   f & 15, holding logical chunk (f & 15) ^ (r & 15)), so the b128 fragment
//   reads of 16 consecutive rows hit 16 different bank groups.
//   M/N-contiguous operand: [64 k][R rows], unpadded (its global layout).
// Tile edges re-read the last valid row, as in load_tile_pipe (full K stages
// only).
typedef __attribute__((address_space(3))) void *lds_void_ptr;

// XOR swizzle of the float4 chunks of K-contiguous row r (CH chunks per row):
// any 8 consecutive rows (and any 16 when CH = 16) map a logical chunk to
// distinct physical chunks, and with CH = 8 two rows 8 apart also differ, so
// 16 consecutive rows of b128 reads cover all banks whether the LDS serves 8
// or 16 lanes per pass.
template <int CH>
__device__ __forceinline__ int chunk_swz(int r) {
  return CH == 16 ? (r & 15) : ((r & 7) ^ ((r >> 3) & 1));
}

template <int R, bool KC, int NTH = NT, int BKW = BK>
__device__ __forceinline__ void load_tile_direct(const float *__restrict__ base, int ld, int rows,
                                                 int r0, int k0, float *S) {
  constexpr int CH = BKW / 4;  // float4 chunks per K-contiguous row
  const int t = threadIdx.x;
  const int wslot = __builtin_amdgcn_readfirstlane((t >> 6) * 64);  // the wave's first slot
#pragma unroll
  for (int j = 0; j < R * CH / NTH; ++j) {
    const int f = t + NTH * j;
    const float *src;
    if (KC) {
      const int r = f / CH, c = (f % CH) ^ chunk_swz<CH>(r);
      src = base + (size_t)min(r0 + r, rows - 1) * ld + k0 + 4 * c;
    } else {
      const int k = f / (R / 4), r4 = (f % (R / 4)) << 2;
      src = base + (size_t)(k0 + k) * ld + min(r0 + r4, rows - 4);
    }
    __builtin_amdgcn_global_load_lds(src, (lds_void_ptr)(S + 4 * (NTH * j + wslot)), 16, 0, 0);
  }
}

// Fragment halves (MFMA steps koff .. koff+7 of each of the wave's T slabs)
// from the direct layouts; pairwise rows for an M/N-contiguous operand at
// T = 2, as in read_frags.
template <int R, bool KC, int BKW = BK>
__device__ __forceinline__ void read_frags_direct(const float *S, int rowbase, int koff, int l32,
                                                  float (&a)[Tile<R>::T][8]) {
  constexpr int T = Tile<R>::T, CH = BKW / 4;
  if (KC) {
    const int c0 = koff >> 2, sw = chunk_swz<CH>(l32);  // rowbase is a multiple of 16
#pragma unroll
    for (int i = 0; i < T; ++i) {
      const float *src = S + (rowbase + i * 32 + l32) * BKW;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const floatx4 x = *reinterpret_cast<const floatx4 *>(src + 4 * ((c0 + q) ^ sw));
        a[i][4 * q + 0] = x[0];
        a[i][4 * q + 1] = x[1];
        a[i][4 * q + 2] = x[2];
        a[i][4 * q + 3] = x[3];
      }
    }
  } else if (T == 2) {
    const float *src = S + koff * R + rowbase + 2 * l32;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float2 x = *reinterpret_cast<const float2 *>(src + s * R);
      a[0][s] = x.x;
      a[T - 1][s] = x.y;
    }
  } else {
    const float *src = S + koff * R + rowbase + l32;
#pragma unroll
    for (int s = 0; s < 8; ++s) a[0][s] = src[s * R];
  }
}

// s_waitcnt immediate (gfx9 encoding) waiting for vmcnt <= n only.
#define GN_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x3F70 | ((n) & 15) | (((n) >> 4) << 14))

// Batched launches (gridDim.z > 1): the z-th GEMM's A, B, bias and C.
__device__ __forceinline__ void batch_offsets(GemmArgs &p) {
  if (gridDim.z > 1) {
    int64_t z = blockIdx.z, zi = 0;
    if (p.nbatch_in > 1) {
      zi = z % p.nbatch_in;
      z /= p.nbatch_in;
    }
    p.A += z * p.bstride_A + zi * p.istride_A;
    p.B += z * p.bstride_B + zi * p.istride_B;
    if (p.bias) p.bias += z * p.bstride_bias;
    p.C += z * p.bstride_C + zi * p.istride_C;
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

// Out-of-line activation for the GEMM epilogue's rare kinds.
__device__ __noinline__ float apply_fwd_call(float v, int kind) { return apply_fwd(v, kind); }
__device__ __noinline__ float apply_deriv_call(float out, int kind) { return apply_deriv(out, kind); }

__device__ __forceinline__ float epilogue(float v, int epi, const GemmArgs &p, int row, int col) {
  if (epi == EPI_SCALE) return v * p.alpha;
  if (epi == EPI_BIAS_ACT) return apply_fwd(v + (p.bias ? p.bias[col] : 0.f), p.act);
  if (epi == EPI_BIAS_ADD)
    return v * p.alpha + (p.bias ? p.bias[col] : 0.f) + p.aux[(size_t)row * p.ldaux + col];
  const int ar = p.aux_div > 1 ? (row / p.aux_div) * p.aux_div + p.aux_div - 1 : row;
  if (p.colscale) v = v * p.colscale[col];
  if (p.act == D_ONE) return v * 1.0f;
  return v * apply_deriv(p.aux[(size_t)ar * p.ldaux + col], p.act);
}

// EPI_PARTIAL: split-K partial sums to the workspace (epilogue applied later).
constexpr int EPI_PARTIAL = 3;

// Epilogue of a block tile: accumulators -> C (or the split-K workspace).
// v_mfma_f32_32x32x2_f32 result layout: lane l, accumulator r holds row
// 8*(r/4) + 4*(l/32) + r%4, column l%32 of the 32x32 tile; with PAIR_A /
// PAIR_B the slabs of that operand hold every other row (read pairwise).
template <int RM, int RN, int EPI, bool PAIR_A, bool PAIR_B>
__device__ __forceinline__ void gemm_store(const GemmArgs &p,
                                           const floatx16 (&acc)[Tile<RM>::T][Tile<RN>::T],
                                           int m0, int n0, int wm, int wn, int half, int l32) {
  constexpr int TM = Tile<RM>::T, TN = Tile<RN>::T;
  const int M = p.M, N = p.N;
  auto col_of = [&](int j) { return n0 + wn * (RN / 2) + (PAIR_B ? 2 * l32 + j : j * 32 + l32); };
  auto row_of = [&](int i, int r) {
    const int rr = (r >> 2) * 8 + half * 4 + (r & 3);
    return m0 + wm * (RM / 2) + (PAIR_A ? 2 * rr + i : i * 32 + rr);
  };
  // Every value the epilogue reads (bias, saved activations, residual rows)
  // is loaded before the first store: the compiler cannot tell a store from
  // an alias of them, so a load placed between stores would wait out its own
  // round trip to L2, 64 times per lane.
  float bcol[TN];
  float av[TM][TN][16];
#pragma unroll
  for (int j = 0; j < TN; ++j) bcol[j] = 0.f;
  if constexpr (EPI == EPI_BIAS_ACT || EPI == EPI_BIAS_ADD) {
    if (p.bias) {
#pragma unroll
      for (int j = 0; j < TN; ++j) bcol[j] = col_of(j) < N ? p.bias[col_of(j)] : 0.f;
    }
  }
  const bool cscale = EPI == EPI_DACT && p.colscale;
  if (cscale) {
#pragma unroll
    for (int j = 0; j < TN; ++j) bcol[j] = col_of(j) < N ? p.colscale[col_of(j)] : 0.f;
  }
  const bool use_aux = (EPI == EPI_BIAS_ADD) || (EPI == EPI_DACT && p.act != D_ONE);
  if (use_aux) {
    // aux row of an output row: itself, or for EPI_DACT the last row of its
    // group of aux_div rows (Q10), found with a multiply-high by
    // ceil(2^32 / d), exact while rows * d < 2^32 (else the division).
    const unsigned d = EPI == EPI_DACT && p.aux_div > 1 ? (unsigned)p.aux_div : 1u;
    const bool magic_ok = (unsigned long long)M * d < (1ull << 32);
    const unsigned magic = d > 1 ? (unsigned)(0xFFFFFFFFull / d + 1) : 0u;
    const int mlast = min(m0 + RM, M) - 1;
    if (d > 1 && (unsigned)m0 / d == (unsigned)mlast / d) {
      // the block's rows share one aux row (a tile inside one sample's
      // tokens): one load per column instead of one per element
      const size_t ar = (size_t)((unsigned)m0 / d * d + d - 1);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = col_of(j);
        const float a = col < N ? p.aux[ar * p.ldaux + col] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) av[i][j][r] = a;
      }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = row_of(i, r), col = col_of(j);
            int ar = row;
            if (d > 1) {
              const unsigned q = magic_ok ? __umulhi((unsigned)row, magic) : (unsigned)row / d;
              ar = (int)(q * d + d - 1);
            }
            av[i][j][r] = (row < M && col < N) ? p.aux[(size_t)ar * p.ldaux + col] : 0.f;
          }
    }
  }
  float *ws = EPI == EPI_PARTIAL ? p.ws + (size_t)blockIdx.y * M * N : nullptr;
  auto store_all = [&](auto f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = col_of(j);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row_of(i, r);
          if (row >= M) continue;
          if (EPI == EPI_PARTIAL)
            ws[(size_t)row * N + col] = acc[i][j][r];
          else
            p.C[(size_t)row * p.ldc + col] = f(acc[i][j][r], i, j, r);
        }
      }
  };
  // The activation is chosen once per block: identity and ReLU inline, the
  // rest through an out-of-line call, so the 64-value-per-lane epilogue stays
  // small (inlining the float64 sigmoid / tanh into it blew the code past the
  // instruction cache).
  if constexpr (EPI == EPI_BIAS_ACT) {
    if (p.act == F_IDENTITY)
      store_all([&](float v, int, int j, int) { return v + bcol[j]; });
    else if (p.act == F_RELU)
      store_all([&](float v, int, int j, int) {
        const float z = v + bcol[j];
        return z > 0.0f ? z : 0.0f;
      });
    else
      store_all([&](float v, int, int j, int) { return apply_fwd_call(v + bcol[j], p.act); });
  } else if constexpr (EPI == EPI_DACT) {
    if (cscale) {  // a Dropout between two Dense layers (dropout.go:283-290): its factor first
      if (p.act == D_ONE)
        store_all([&](float v, int, int j, int) { return (v * bcol[j]) * 1.0f; });
      else if (p.act == D_RELU)
        store_all([&](float v, int i, int j, int r) { return (v * bcol[j]) * (av[i][j][r] > 0.0f ? 1.0f : 0.0f); });
      else
        store_all([&](float v, int i, int j, int r) { return (v * bcol[j]) * apply_deriv_call(av[i][j][r], p.act); });
    } else if (p.act == D_ONE)
      store_all([&](float v, int, int, int) { return v * 1.0f; });
    else if (p.act == D_RELU)
      store_all([&](float v, int i, int j, int r) { return v * (av[i][j][r] > 0.0f ? 1.0f : 0.0f); });
    else
      store_all([&](float v, int i, int j, int r) { return v * apply_deriv_call(av[i][j][r], p.act); });
  } else if constexpr (EPI == EPI_BIAS_ADD) {
    store_all([&](float v, int i, int j, int r) { return v * p.alpha + bcol[j] + av[i][j][r]; });
  } else {
    store_all([&](float v, int, int, int) { return v * p.alpha; });
  }
}

// R = 128 runs one block per CU (139 KB of LDS), so two waves per SIMD and
// the full 256-register budget; R = 64 fits two blocks per CU.
// PIPE: 0 = bounds-checked loop, 1 = pipelined loop (K range a multiple of
// BK), 2 = pipelined loop with a partial last K stage.
template <int R, bool AK, bool BKC, bool VEC, int EPI, int PIPE>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, R == 128 ? 2 : 4)))
void gemm_f32_mfma(GemmArgs p, int tiles_m, int tiles_n, int kchunk) {
  using TL = Tile<R>;
  constexpr int T = TL::T;
  __shared__ __attribute__((aligned(16))) float As[2][TL::STAGE];
  __shared__ __attribute__((aligned(16))) float Bs[2][TL::STAGE];

  batch_offsets(p);
  int tm, tn;
  tile_of_block(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * R, n0 = tn * R;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  // waves 0-3 take k in [0,32) of every stage, waves 4-7 take [32,64); within
  // a group the 4 waves tile the R x R block as 2x2 sub-tiles of R/2 x R/2.
  const int g = w >> 2, w4 = w & 3;
  const int wm = w4 >> 1, wn = w4 & 1;
  const int half = lane >> 5, l32 = lane & 31;
  const int koff = g * 32 + half * 16;
  const int M = p.M, N = p.N;
  const int kbeg = blockIdx.y * kchunk;
  const int kend = min(p.K, kbeg + kchunk);
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  // operand bases of the K stage starting at k (segmented K: the stage's segment)
  auto opA = [&](int k) -> const float * { return p.kseg ? p.A + (int64_t)(k / p.kseg) * p.kseg_dA : p.A; };
  auto opB = [&](int k) -> const float * { return p.kseg ? p.B + (int64_t)(k / p.kseg) * p.kseg_dB : p.B; };

  floatx16 acc[T][T];
#pragma unroll
  for (int i = 0; i < T; ++i)
#pragma unroll
    for (int j = 0; j < T; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if constexpr (PIPE != 0) {
    // Operands are float4-legal and nk >= 1; tile edges are clamped (see
    // load_tile_pipe).  Software
    // pipeline, one barrier per stage, each stage's 16 MFMA steps in halves
    // f0 (s < 8) and f1 (s >= 8):
    //   f1 fragment reads | MFMAs s = 0..7 | MFMAs s = 8..11 with the LDS
    //   writes of the next stage | barrier | next stage's f0 fragment reads
    //   and the global loads of the stage after next | MFMAs s = 12..15.
    // The barrier sits before the stage's last quarter of MFMAs, so the
    // fragment reads after it are covered by MFMAs on registers; global loads
    // are issued about one stage before their LDS writes.  Loads and writes
    // beyond the last stage re-read it into the idle buffer.
    constexpr bool KT = PIPE == 2;
    const int mrow = wm * (R / 2), ncol = wn * (R / 2);
    floatx4 ra[TL::NLD], rb[TL::NLD];
    load_tile_pipe<R, AK, KT>(opA(kbeg), p.lda, M, kend, m0, kbeg, ra);
    load_tile_pipe<R, BKC, KT>(opB(kbeg), p.ldb, N, kend, n0, kbeg, rb);
    store_tile_pipe<R, AK, KT>(As[0], ra, kbeg, kend);
    store_tile_pipe<R, BKC, KT>(Bs[0], rb, kbeg, kend);
    {
      const int k1 = kbeg + min(1, nk - 1) * BK;
      load_tile_pipe<R, AK, KT>(opA(k1), p.lda, M, kend, m0, k1, ra);
      load_tile_pipe<R, BKC, KT>(opB(k1), p.ldb, N, kend, n0, k1, rb);
    }
    __syncthreads();
    float f0a[T][8], f0b[T][8];
    read_frags<R, AK>(As[0], mrow, koff, l32, f0a);
    read_frags<R, BKC>(Bs[0], ncol, koff, l32, f0b);
    // fragment reads per half stage: 2 b128 per slab (K-contiguous), else 8
    // (b64 pairs at T = 2, b32 at T = 1)
    constexpr int DSRH = (AK ? 2 * T : 8) + (BKC ? 2 * T : 8);
    constexpr int NW = 2 * TL::NLD;                            // loads (= LDS writes) per stage
    constexpr int MQ = 4 * T * T;                              // MFMAs per quarter stage
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      float f1a[T][8], f1b[T][8];
      read_frags<R, AK>(As[cur], mrow, koff + 8, l32, f1a);
      read_frags<R, BKC>(Bs[cur], ncol, koff + 8, l32, f1b);
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
          for (int j = 0; j < T; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f0a[i][s], f0b[j][s], acc[i][j], 0, 0, 0);
      {
        const int k1 = kbeg + min(kt + 1, nk - 1) * BK;  // the stage ra, rb hold
        store_tile_pipe<R, AK, KT>(As[cur ^ 1], ra, k1, kend);
        store_tile_pipe<R, BKC, KT>(Bs[cur ^ 1], rb, k1, kend);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
          for (int j = 0; j < T; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f1a[i][s], f1b[j][s], acc[i][j], 0, 0, 0);
      // group masks: 0x008 MFMA, 0x020 global load, 0x100 LDS read, 0x200 LDS write
      __builtin_amdgcn_sched_group_barrier(0x100, DSRH, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * MQ, 0);
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, MQ / NW, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
      __syncthreads();
      read_frags<R, AK>(As[cur ^ 1], mrow, koff, l32, f0a);
      read_frags<R, BKC>(Bs[cur ^ 1], ncol, koff, l32, f0b);
      {
        const int k2 = kbeg + min(kt + 2, nk - 1) * BK;
        load_tile_pipe<R, AK, KT>(opA(k2), p.lda, M, kend, m0, k2, ra);
        load_tile_pipe<R, BKC, KT>(opB(k2), p.ldb, N, kend, n0, k2, rb);
      }
#pragma unroll
      for (int s = 4; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
          for (int j = 0; j < T; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f1a[i][s], f1b[j][s], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, DSRH, 0);
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, MQ / NW, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
    }
    // the last iteration's fragment reads target LDS the reduction reuses
    __syncthreads();
  } else {
    float4 ra[TL::NLD], rb[TL::NLD];
    load_tile<R, AK, VEC>(opA(kbeg), p.lda, M, kend, m0, kbeg, ra);
    load_tile<R, BKC, VEC>(opB(kbeg), p.ldb, N, kend, n0, kbeg, rb);
    store_tile<R, AK>(As[0], ra);
    store_tile<R, BKC>(Bs[0], rb);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < nk;
      if (more) {
        load_tile<R, AK, VEC>(opA(kbeg + (kt + 1) * BK), p.lda, M, kend, m0, kbeg + (kt + 1) * BK, ra);
        load_tile<R, BKC, VEC>(opB(kbeg + (kt + 1) * BK), p.ldb, N, kend, n0, kbeg + (kt + 1) * BK, rb);
      }
      float a[T][16], b[T][16];
#pragma unroll
      for (int i = 0; i < T; ++i) read_frag<R, AK>(As[cur], wm * (R / 2) + i * 32, koff, l32, a[i]);
#pragma unroll
      for (int j = 0; j < T; ++j) read_frag<R, BKC>(Bs[cur], wn * (R / 2) + j * 32, koff, l32, b[j]);
#pragma unroll
      for (int s = 0; s < 16; ++s)
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
          for (int j = 0; j < T; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
      if (more) {
        store_tile<R, AK>(As[cur ^ 1], ra);
        store_tile<R, BKC>(Bs[cur ^ 1], rb);
      }
      __syncthreads();
    }
  }

  // K-group 1 hands its accumulators to group 0 through LDS (the operand
  // stages are free after the last barrier): 4 waves x 64 lanes x T*T*16 floats.
  float *red = &As[0][0];
  static_assert(4 * 64 * TL::QPL * 4 <= 2 * TL::STAGE, "reduction buffer");
  if (g == 1) {
#pragma unroll
    for (int q = 0; q < TL::QPL; ++q) {
      const int ij = q >> 2, r4 = (q & 3) << 2;
      const floatx16 &v = acc[ij / T][ij % T];
      *reinterpret_cast<float4 *>(red + ((w4 * TL::QPL + q) * 64 + lane) * 4) =
          make_float4(v[r4], v[r4 + 1], v[r4 + 2], v[r4 + 3]);
    }
  }
  __syncthreads();
  if (g == 1) return;
#pragma unroll
  for (int q = 0; q < TL::QPL; ++q) {
    const int ij = q >> 2, r4 = (q & 3) << 2;
    const float4 o = *reinterpret_cast<const float4 *>(red + ((w4 * TL::QPL + q) * 64 + lane) * 4);
    floatx16 &v = acc[ij / T][ij % T];
    v[r4] += o.x;
    v[r4 + 1] += o.y;
    v[r4 + 2] += o.z;
    v[r4 + 3] += o.w;
  }

  gemm_store<R, R, EPI, PIPE != 0 && !AK && T == 2, PIPE != 0 && !BKC && T == 2>(p, acc, m0, n0, wm,
                                                                                  wn, half, l32);
}

// Four-wave variant for full K stages and R = 128: each wave owns a 64 x 64
// sub-tile over the block's whole K range (no in-block K split, no
// reduction), operands staged by direct global -> LDS loads two stages deep.
// BKW = 32 keeps a block at 64 KB of LDS so two blocks share a CU: the two
// waves on a SIMD then belong to different blocks and one block's MFMAs run
// while the other waits at its barrier (one 8-wave block stalls both waves of
// every SIMD at each barrier).  Lane half h feeds k = (BKW/2)h + s at MFMA
// step s of a stage; the steps run in quarters of 8 whose fragments
// alternate between two register sets; all quarters but the last run before
// the stage's barrier:
//   MFMAs q0 (reads q1) | ... | wait for the next stage's loads | barrier |
//   next stage's q0 reads and the loads of the stage after next into the
//   buffer just released | MFMAs of the last quarter.
constexpr int NT4 = 256;

template <int BKW, int NS, int RN, bool AK, bool BKC, int EPI>
__global__ __launch_bounds__(NT4)
__attribute__((amdgpu_waves_per_eu(NS * BKW * (128 + RN) <= 16384 ? 2 : 1,
                                   NS * BKW * (128 + RN) <= 16384 ? 2 : 1)))
void gemm_f32_mfma_w4(GemmArgs p, int tiles_m, int tiles_n, int kchunk) {
  constexpr int RM = 128, TM = 2, TN = RN / 64;
  constexpr int NLA = RM * BKW / 4 / NT4, NLB = RN * BKW / 4 / NT4;  // direct loads per thread
  constexpr int QN = BKW / 16;  // quarters of 8 MFMA steps per stage
  static_assert(QN == 2 || QN == 4, "stage depth");
  static_assert(RN == 128 || RN == 64, "tile width");
  __shared__ __attribute__((aligned(16))) float As[NS][RM * BKW];
  __shared__ __attribute__((aligned(16))) float Bs[NS][RN * BKW];

  batch_offsets(p);
  int tm, tn;
  tile_of_block(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * RM, n0 = tn * RN;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int half = lane >> 5, l32 = lane & 31;
  const int koff = half * (BKW / 2);
  const int M = p.M, N = p.N;
  const int kbeg = blockIdx.y * kchunk;
  const int kend = min(p.K, kbeg + kchunk);
  const int nk = (kend - kbeg) / BKW;  // >= 1, full stages (checked by the launcher)
  const int mrow = wm * (RM / 2), ncol = wn * (RN / 2);

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int k1 = kbeg + min(st, nk - 1) * BKW;
    load_tile_direct<RM, AK, NT4, BKW>(p.A, p.lda, M, m0, k1, As[st]);
    load_tile_direct<RN, BKC, NT4, BKW>(p.B, p.ldb, N, n0, k1, Bs[st]);
  }
  constexpr int NW = NLA + NLB;  // direct loads per thread per stage
  GN_WAIT_VMCNT(NW * (NS - 1));  // stage 0 has landed; later ones may be in flight
  __syncthreads();
  float fa[TM][8], fb[TN][8];
  read_frags_direct<RM, AK, BKW>(As[0], mrow, koff, l32, fa);
  read_frags_direct<RN, BKC, BKW>(Bs[0], ncol, koff, l32, fb);
  constexpr int DSRH = (AK ? 2 * TM : 8) + (BKC ? 2 * TN : 8);
  constexpr int MQ = 8 * TM * TN;  // MFMAs per quarter stage
  static_assert(DSRH <= MQ, "one read per MFMA");
  auto mfma8 = [&](const float (&a)[TM][8], const float (&b)[TN][8]) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
  };
  int cur = 0;  // buffer of stage kt; stage kt + j sits in (cur + j) % NS
  for (int kt = 0; kt < nk; ++kt) {
    const int nxt = cur + 1 == NS ? 0 : cur + 1;
    float ga[TM][8], gb[TN][8];
    read_frags_direct<RM, AK, BKW>(As[cur], mrow, koff + 8, l32, ga);
    read_frags_direct<RN, BKC, BKW>(Bs[cur], ncol, koff + 8, l32, gb);
    mfma8(fa, fb);
    if constexpr (QN == 4) {
      read_frags_direct<RM, AK, BKW>(As[cur], mrow, koff + 16, l32, fa);
      read_frags_direct<RN, BKC, BKW>(Bs[cur], ncol, koff + 16, l32, fb);
      mfma8(ga, gb);
      read_frags_direct<RM, AK, BKW>(As[cur], mrow, koff + 24, l32, ga);
      read_frags_direct<RN, BKC, BKW>(Bs[cur], ncol, koff + 24, l32, gb);
      mfma8(fa, fb);
    }
    // group masks: 0x008 MFMA, 0x020 global load, 0x100 LDS read.  Each
    // quarter's fragment reads go out one per MFMA among the first MFMAs of
    // the quarter before (a single wave per SIMD issues in order: a run of
    // reads leaves the matrix pipe idle), at most DSRH outstanding where a
    // wait is needed (lgkmcnt counts to 15).
#pragma unroll
    for (int q = 0; q < QN - 1; ++q) {
#pragma unroll
      for (int r = 0; r < DSRH; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, MQ - DSRH, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the MFMAs above the barrier
    // this wave's loads of stage kt+1 are in LDS (those of kt+2 .. kt+NS-1
    // may still be in flight)
    GN_WAIT_VMCNT(NW * (NS - 2));
    __syncthreads();
    read_frags_direct<RM, AK, BKW>(As[nxt], mrow, koff, l32, fa);
    read_frags_direct<RN, BKC, BKW>(Bs[nxt], ncol, koff, l32, fb);
    {
      // stage kt+NS into stage kt's buffer, which every wave finished
      // reading before this barrier
      const int k2 = kbeg + min(kt + NS, nk - 1) * BKW;
      load_tile_direct<RM, AK, NT4, BKW>(p.A, p.lda, M, m0, k2, As[cur]);
      load_tile_direct<RN, BKC, NT4, BKW>(p.B, p.ldb, N, n0, k2, Bs[cur]);
    }
    cur = nxt;
    mfma8(ga, gb);
    // reads and loads one per MFMA while MFMAs last, the remaining loads after
    constexpr int NWM = NW < MQ - DSRH ? NW : MQ - DSRH;
#pragma unroll
    for (int r = 0; r < DSRH; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int q = 0; q < NWM; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    if constexpr (NW > NWM) __builtin_amdgcn_sched_group_barrier(0x020, NW - NWM, 0);
    if constexpr (MQ > DSRH + NWM) __builtin_amdgcn_sched_group_barrier(0x008, MQ - DSRH - NWM, 0);
  }
  GN_WAIT_VMCNT(0);  // nothing may land after the block ends
  gemm_store<RM, RN, EPI, !AK, !BKC && TN == 2>(p, acc, m0, n0, wm, wn, half, l32);
}

// Split-K reduction: partials summed in split order, then the epilogue.
// Blocks from nred on (p.cs_src set): the column sums cs_dst[c] = cs_scale *
// sum_r cs_src[r][c], rows in order with eight loads in flight, one thread
// per column (a bias gradient that would otherwise take a launch).
__device__ __forceinline__ void reduce_side_colsum(const GemmArgs &p, int cb) {
  const int c = cb * NT + threadIdx.x;
  if (c >= p.cs_cols) return;
  const float *src = p.cs_src + c;
  float v = 0.f;
  int r = 0;
  for (; r + 7 < p.cs_rows; r += 8) {
    float u8[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) u8[u] = src[(size_t)(r + u) * p.cs_cols];
#pragma unroll
    for (int u = 0; u < 8; ++u) v += u8[u];
  }
  for (; r < p.cs_rows; ++r) v += src[(size_t)r * p.cs_cols];
  p.cs_dst[c] = v * p.cs_scale;
}

__global__ __launch_bounds__(NT) void gemm_splitk_reduce(GemmArgs p, int splits, int epi, int nred) {
  if ((int)blockIdx.x >= nred) {
    reduce_side_colsum(p, blockIdx.x - nred);
    return;
  }
  const size_t MN = (size_t)p.M * p.N;
  for (size_t idx = (size_t)blockIdx.x * NT + threadIdx.x; idx < MN; idx += (size_t)nred * NT) {
    float v = p.ws[idx];
    for (int s = 1; s < splits; s += 8) {  // eight loads in flight, added in split order
      float u8[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) u8[u] = s + u < splits ? p.ws[(s + u) * MN + idx] : 0.f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s + u < splits) v += u8[u];
    }
    const int row = (int)(idx / p.N), col = (int)(idx % p.N);
    const float y = epilogue(v, epi, p, row, col);
    p.C[(size_t)row * p.ldc + col] = y;
    if (p.drop_out) p.drop_out[(size_t)row * p.ldc + col] = p.drop_mask[col] > 0.f ? y * p.drop_scale : 0.0f;
  }
}

// Small outputs with many splits: one wave per element, lanes over the splits
// (a fixed tree order), so the sum is not a chain of `splits` dependent loads.
__global__ __launch_bounds__(NT) void gemm_splitk_reduce_wave(GemmArgs p, int splits, int epi, int nred) {
  if ((int)blockIdx.x >= nred) {
    reduce_side_colsum(p, blockIdx.x - nred);
    return;
  }
  const size_t MN = (size_t)p.M * p.N;
  const size_t idx = (size_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (idx >= MN) return;
  float v = 0.f;
  for (int s = lane; s < splits; s += 64) v += p.ws[s * MN + idx];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if (lane == 0) {
    const int row = (int)(idx / p.N), col = (int)(idx % p.N);
    const float y = epilogue(v, epi, p, row, col);
    p.C[(size_t)row * p.ldc + col] = y;
    if (p.drop_out) p.drop_out[(size_t)row * p.ldc + col] = p.drop_mask[col] > 0.f ? y * p.drop_scale : 0.0f;
  }
}

template <int R, bool AK, bool BKC, int EPI>
static hipError_t launch_t(bool vec, bool ktail, const GemmArgs &a, int tm, int tn, int splits,
                          int kchunk, hipStream_t s) {
  dim3 grid(tm * tn, splits, a.nbatch > 1 ? a.nbatch : 1), block(NT);
  if (R == 128 && vec && !ktail) {
    // Four-wave kernels: 32-deep stages (64 KB of LDS) when there are at
    // least two tiles per CU (two blocks share a CU) or the K range is at most
    // four 64-deep stages (the transformer's K = 256 projections: +0.7 % on
    // its step; at K = 1024 the C3 step lost 3 %); else 64-deep stages, one
    // block per CU.
    if (tm * tn * splits >= 512 || kchunk <= 256)
      hipLaunchKernelGGL((gemm_f32_mfma_w4<32, 2, 128, AK, BKC, EPI>), grid, dim3(NT4), 0, s, a, tm, tn,
                         kchunk);
    else
      hipLaunchKernelGGL((gemm_f32_mfma_w4<64, 2, 128, AK, BKC, EPI>), grid, dim3(NT4), 0, s, a, tm, tn,
                         kchunk);
  } else if (vec && !ktail)
    hipLaunchKernelGGL((gemm_f32_mfma<R, AK, BKC, true, EPI, 1>), grid, block, 0, s, a, tm, tn,
                       kchunk);
  else if (vec)
    hipLaunchKernelGGL((gemm_f32_mfma<R, AK, BKC, true, EPI, 2>), grid, block, 0, s, a, tm, tn,
                       kchunk);
  else
    hipLaunchKernelGGL((gemm_f32_mfma<R, AK, BKC, false, EPI, 0>), grid, block, 0, s, a, tm, tn,
                       kchunk);
  return hipGetLastError();
}

template <int R, int EPI>
static hipError_t launch_e(char ta, char tb, bool vec, bool ktail, const GemmArgs &a, int tm, int tn,
                           int splits, int kchunk, hipStream_t s) {
  // op(A) 'N' -> A is M x K, K contiguous.  op(B) 'T' -> B is N x K, K contiguous.
  const bool ak = (ta == 'N');
  const bool bk = (tb == 'T');
  if (ak && bk) return launch_t<R, true, true, EPI>(vec, ktail, a, tm, tn, splits, kchunk, s);
  if (ak && !bk) return launch_t<R, true, false, EPI>(vec, ktail, a, tm, tn, splits, kchunk, s);
  if (!ak && bk) return launch_t<R, false, true, EPI>(vec, ktail, a, tm, tn, splits, kchunk, s);
  return launch_t<R, false, false, EPI>(vec, ktail, a, tm, tn, splits, kchunk, s);
}

template <int R>
static hipError_t launch_r(char ta, char tb, int epi, bool vec, const GemmArgs &a, int splits,
                           int kchunk, hipStream_t s) {
  const int tm = (a.M + R - 1) / R, tn = (a.N + R - 1) / R;
  // float4-legal operands take the pipelined loop; it checks k only when the
  // last K stage is partial
  const bool ktail = a.K % BK != 0;
  if (splits > 1) return launch_e<R, EPI_PARTIAL>(ta, tb, vec, ktail, a, tm, tn, splits, kchunk, s);
  if (epi == EPI_BIAS_ACT)
    return launch_e<R, EPI_BIAS_ACT>(ta, tb, vec, ktail, a, tm, tn, 1, kchunk, s);
  if (epi == EPI_DACT) return launch_e<R, EPI_DACT>(ta, tb, vec, ktail, a, tm, tn, 1, kchunk, s);
  if (epi == EPI_BIAS_ADD)
    return launch_e<R, EPI_BIAS_ADD>(ta, tb, vec, ktail, a, tm, tn, 1, kchunk, s);
  return launch_e<R, EPI_SCALE>(ta, tb, vec, ktail, a, tm, tn, 1, kchunk, s);
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The tile plan of launch_gemm takes 128-wide tiles (four-wave kernels,
// which load whole K ranges) when they fill the chip; a segmented K needs the
// 64-wide plan.
static bool plan_big(const GemmArgs &a) {
  const int64_t nmem = (a.nbatch > 1 && a.nbatch_in > 1) ? a.nbatch : 1;
  const int64_t t128 = ((a.M + 127) / 128) * (int64_t)((a.N + 127) / 128) * nmem;
  const int64_t t64 = ((a.M + 63) / 64) * (int64_t)((a.N + 63) / 64) * nmem;
  return t128 >= 160 && !(a.K <= 256 && t64 >= 1024);
}

bool gemm_segments_ok(const GemmArgs &a) {
  return a.kseg > 0 && a.kseg % BK == 0 && a.nbatch <= 1 && !a.defer_splits && !a.drop_out && !plan_big(a);
}

hipError_t launch_gemm(char ta, char tb, int epi, const GemmArgs &a0, hipStream_t s) {
  if (a0.M <= 0 || a0.N <= 0) return hipSuccess;
  GemmArgs a = a0;
  if (a.kseg > 0) {
    // the stage loaders of the eight-wave kernel step to segment k / kseg
    if (!gemm_segments_ok(a)) return hipErrorNotSupported;
    a.kseg_dA = a.seg_A - (ta == 'N' ? (int64_t)a.kseg : (int64_t)a.kseg * a.lda);
    a.kseg_dB = a.seg_B - (tb == 'T' ? (int64_t)a.kseg : (int64_t)a.kseg * a.ldb);
  } else {
    a.kseg = 0;
  }
  if (a.drop_out && (epi != EPI_BIAS_ACT || a.nbatch > 1 || !a.drop_mask)) return hipErrorInvalidValue;
  // float4 staging needs 16 B aligned rows and the contiguous extent % 4 == 0
  const bool ak = (ta == 'N'), bk = (tb == 'T');
  bool vec = aligned16(a.A) && aligned16(a.B) && (a.lda % 4 == 0) && (a.ldb % 4 == 0) &&
             ((a.seg_A | a.seg_B) & 3) == 0;
  vec = vec && (ak ? (a.K % 4 == 0) : (a.M % 4 == 0));
  vec = vec && (bk ? (a.K % 4 == 0) : (a.N % 4 == 0));
  vec = vec && a.K > 0;  // the pipelined loop assumes at least one K stage
  // 128-wide tiles when they fill the 256 CUs, else 64-wide tiles; when even
  // those cannot fill the chip and K has at least 8 stages, split K (down to
  // one K stage per split: a lone tile runs at 1/256 of the chip).  Partials
  // go to the workspace and are summed in split order.  Below 8 stages a tile
  // is short and the reduce launch would cost more than the split saves.
  // two-level batches (many small members) count the tiles of all members
  const int64_t nmem = (a.nbatch > 1 && a.nbatch_in > 1) ? a.nbatch : 1;
  const int64_t t128 = ((a.M + 127) / 128) * (int64_t)((a.N + 127) / 128) * nmem;
  const int64_t t64 = ((a.M + 63) / 64) * (int64_t)((a.N + 63) / 64) * nmem;
  // short K (at most four 64-deep stages) with four 64-wide tiles per CU:
  // 64-wide tiles, whose blocks cover each other's prologue and epilogue
  const bool big = plan_big(a);
  if (a.kseg > 0 && big) return hipErrorNotSupported;  // the four-wave kernels load whole K ranges
  const int tiles = (int)std::min<int64_t>(big ? t128 : t64, 1 << 30);
  int splits = 1;
  if (tiles < 160 && a.K >= 8 * BK && a.ws) {
    splits = std::min((256 + tiles - 1) / tiles, a.K / BK);
    while (splits > 1 && (size_t)splits * a.M * a.N > a.ws_cap) --splits;
  }
  int kchunk = a.K > 0 ? a.K : 1;
  if (splits > 1) {
    kchunk = ((a.K + splits - 1) / splits + BK - 1) / BK * BK;
    splits = (a.K + kchunk - 1) / kchunk;
  }
  const bool two = a.nbatch_in > 1;
  const bool stride16 = ((a.bstride_A | a.bstride_B | (two ? a.istride_A | a.istride_B : 0)) & 3) == 0;
  if (a.defer_splits && a.nbatch > 1) return hipErrorInvalidValue;
  if (a.nbatch > 1 && (splits > 1 || !stride16)) {
    // split-K partials share one workspace, and float4 legality is judged on
    // the first member: one launch per GEMM of the batch
    for (int z = 0; z < a.nbatch; ++z) {
      const int64_t zo = two ? z / a.nbatch_in : z, zi = two ? z % a.nbatch_in : 0;
      GemmArgs az = a;
      az.nbatch = 1;
      az.nbatch_in = 0;
      az.A += zo * a.bstride_A + zi * a.istride_A;
      az.B += zo * a.bstride_B + zi * a.istride_B;
      if (az.bias) az.bias += zo * a.bstride_bias;
      az.C += zo * a.bstride_C + zi * a.istride_C;
      const hipError_t ez = launch_gemm(ta, tb, epi, az, s);
      if (ez != hipSuccess) return ez;
    }
    return hipSuccess;
  }
  hipError_t e = big ? launch_r<128>(ta, tb, epi, vec, a, splits, kchunk, s)
                     : launch_r<64>(ta, tb, epi, vec, a, splits, kchunk, s);
  if (e != hipSuccess) return e;
  if (a.defer_splits) {
    *a.defer_splits = splits;
    if (splits > 1) return hipGetLastError();  // partials only: the caller reduces
  }
  if (splits <= 1) {
    if (!a.drop_out) return e;
    if (a.ldc != a.N) return hipErrorInvalidValue;
    return launch_dropout(a.C, a.drop_mask, a.drop_scale, a.drop_out, a.M, a.N, s);
  }
  const size_t MN = (size_t)a.M * a.N;
  const unsigned csb = a.cs_src && a.cs_dst && a.cs_cols > 0 ? (unsigned)((a.cs_cols + NT - 1) / NT) : 0u;
  if (splits >= 16 && MN <= 65536) {
    const unsigned blocks = (unsigned)((MN + NT / 64 - 1) / (NT / 64));
    hipLaunchKernelGGL(gemm_splitk_reduce_wave, dim3(blocks + csb), dim3(NT), 0, s, a, splits, epi, (int)blocks);
  } else {
    const unsigned blocks = (unsigned)std::min<size_t>((MN + NT - 1) / NT, 4096);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(blocks + csb), dim3(NT), 0, s, a, splits, epi, (int)blocks);
  }
  if (a.cs_done) *a.cs_done = csb > 0 ? 1 : 0;
  return hipGetLastError();
}

}  // namespace gn
