// fp32 GEMM family on gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
// One kernel template covers the three forms of the reference:
//   A@B   (GemmKernel, src/gpu/matmul.rs:21-120)            A k-contiguous, B n-contiguous
//   A@Bᵀ  (GemmTransposeBKernel, src/gpu/matmul.rs:122-219)  A k-contiguous, B k-contiguous
//   dest += dYᵀ·X  (OuterProductAccumKernel, src/gpu/reduce.rs:15-115)
//                                                           A m-contiguous, B n-contiguous
// Operands are copied global→LDS exactly as they lie in memory (float4 loads,
// no transposition); the fragment read adapts instead:
//   * a k-contiguous operand is read as one float4 along k per lane, and the
//     four values feed four consecutive MFMAs;
//   * a k-strided operand is read as four b32 values at rows k, k+1, k+2, k+3.
// Both operands use the same k permutation inside a 16-wide k chunk: MFMA s
// (0..3) takes k = 16c + 4·(lane/16) + s, so Σ over s and the MFMA's own
// 4-wide reduction covers the chunk exactly once.
//
// Work split: a 256-thread block (4 waves in 2×2) owns a BM×BN tile; each
// wave owns (BM/2)×(BN/2) as a grid of 16×16 MFMA tiles.  Global→LDS is
// double-buffered with one barrier per BK step.  Long-K/small-output shapes
// (the weight-gradient accumulate) split K over blockIdx.z into fp32 partial
// tiles that a second kernel reduces in fixed split order — deterministic,
// no atomics — and adds into the destination.
#include "common.hpp"

#include <map>
#include <mutex>

#include <algorithm>
#include <type_traits>
#include <cstdlib>

namespace {

constexpr int kThreads = 256;

struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  float* P;  // split-K partials [splits][M][N]
  int M, N, K;
  int lda, ldb, ldc;
  int k_chunk;  // K range per blockIdx.z (multiple of BK)
  int split;    // 1: write partial tiles to P[z] (epilogue runs in splitk_reduce)
  int tiles_m, tiles_n;
  aur::Epilogue epi;
  // Strided batch (gridDim.y > 1): problem z uses A + z·sA, B + z·sB, C + z·sC.
  long long sA, sB, sC;
};

// Points the operands at problem blockIdx.y of a strided batch.
__device__ __forceinline__ void select_batch(GemmArgs& g) {
  if (gridDim.y > 1) {
    const long long z = blockIdx.y;
    g.A += z * g.sA;
    g.B += z * g.sB;
    g.C += z * g.sC;
  }
}

// Fused epilogue on one output element v = (A·B)(row, col), stored at C[i]
// with i = row*ldc + col (R, X, C2 share C's layout).
// GELU, tanh form (src/linalg.rs:72-87): gelu(x) = 0.5·x·(1 + tanh(u)),
// u = √(2/π)·(x + 0.044715·x³).  With σ(t) = 1/(1 + e^(−t)) the identities
// 1 + tanh(u) = 2σ(2u) and sech²(u) = 4σ(2u)(1 − σ(2u)) give both the value
// and the derivative from one exp2 and one reciprocal, with no cancellation:
//   gelu(x)  = x·σ(2u)
//   gelu'(x) = σ(2u) + 2x·σ(2u)(1 − σ(2u))·√(2/π)·(1 + 3·0.044715·x²)
// (1 − σ(2u) = e^(−2u)·σ(2u) where σ is near 1).  The tanhf form spends
// most of the FFN GEMM epilogues in VALU work.
__device__ __forceinline__ float gelu_sigma(float x, float& one_minus) {
  const float k = 0.7978845608028654f, log2e = 1.4426950408889634f;
  const float u = k * (x + 0.044715f * x * x * x);
  const float e = __builtin_amdgcn_exp2f(-2.0f * log2e * u);  // e^(−2u)
  const float sig = __builtin_amdgcn_rcpf(1.0f + e);
  one_minus = e < 1.0f ? e * sig : 1.0f - sig;
  return sig;
}

__device__ __forceinline__ float gelu_tanh(float x) {
  float om;
  return x * gelu_sigma(x, om);
}

__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float k = 0.7978845608028654f;
  float om;
  const float sig = gelu_sigma(x, om);
  return sig + 2.0f * x * sig * om * (k * (1.0f + 3.0f * 0.044715f * x * x));
}

__device__ __forceinline__ void apply_epilogue(const aur::Epilogue& e, float* __restrict__ C, size_t i,
                                               float v) {
  switch (e.mode) {
    case aur::EPI_ACCUM: C[i] = C[i] + v; break;
    case aur::EPI_RESID: C[i] = e.R[i] + v; break;
    case aur::EPI_GELU:
      C[i] = v;
      e.C2[i] = gelu_tanh(v);
      break;
    case aur::EPI_GELU_BWD: C[i] = v * gelu_tanh_grad(e.X[i]); break;
    default: C[i] = v; break;
  }
}

// Writes a wave's TM×TN grid of 16×16 accumulator tiles (lane holds rows
// 4·g16 + e, column l16 of each) with the epilogue mode fixed at compile
// time, so the store loops carry no per-element branch.  MODE −1: split-K
// partial tile into P[z].  `full`: every row and column is in range.
template <int MODE, int TM, int TN>
__device__ __forceinline__ void write_tile(const GemmArgs& g, const floatx4 (&acc)[TM][TN], int r0, int c0,
                                           int g16, int l16, bool full) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = c0 + j * 16 + l16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + i * 16 + 4 * g16 + e;
        if (!full && (row >= g.M || col >= g.N)) continue;
        const float v = acc[i][j][e];
        if constexpr (MODE < 0) {
          g.P[((size_t)blockIdx.z * g.M + row) * g.N + col] = v;
        } else {
          const size_t idx = (size_t)row * g.ldc + col;
          if constexpr (MODE == aur::EPI_ACCUM) g.C[idx] = g.C[idx] + v;
          else if constexpr (MODE == aur::EPI_RESID) g.C[idx] = g.epi.R[idx] + v;
          else if constexpr (MODE == aur::EPI_GELU) {
            g.C[idx] = v;
            g.epi.C2[idx] = gelu_tanh(v);
          } else if constexpr (MODE == aur::EPI_GELU_BWD) g.C[idx] = v * gelu_tanh_grad(g.epi.X[idx]);
          else g.C[idx] = v;
        }
      }
    }
}

template <int TM, int TN>
__device__ __forceinline__ void write_tiles(const GemmArgs& g, const floatx4 (&acc)[TM][TN], int r0, int c0,
                                            int g16, int l16, bool full) {
  if (g.split) {
    write_tile<-1>(g, acc, r0, c0, g16, l16, full);
    return;
  }
  switch (g.epi.mode) {
    case aur::EPI_ACCUM: write_tile<aur::EPI_ACCUM>(g, acc, r0, c0, g16, l16, full); break;
    case aur::EPI_RESID: write_tile<aur::EPI_RESID>(g, acc, r0, c0, g16, l16, full); break;
    case aur::EPI_GELU: write_tile<aur::EPI_GELU>(g, acc, r0, c0, g16, l16, full); break;
    case aur::EPI_GELU_BWD: write_tile<aur::EPI_GELU_BWD>(g, acc, r0, c0, g16, l16, full); break;
    default: write_tile<aur::EPI_STORE>(g, acc, r0, c0, g16, l16, full); break;
  }
}

// The epilogue operand (R or X, laid out like C) of a wave's TM×TN tiles,
// in the accumulator layout: pre[i][j][e] = S[r0 + 16i + 4·g16 + e][c0 + 16j + l16].
template <int TM, int TN>
__device__ __forceinline__ void load_epi_operand(const GemmArgs& g, floatx4 (&pre)[TM][TN], int r0, int c0,
                                                 int g16, int l16, int mode) {
  const float* src = mode == aur::EPI_RESID ? g.epi.R : g.epi.X;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pre[i][j][e] = src[(size_t)(r0 + i * 16 + 4 * g16 + e) * g.ldc + c0 + j * 16 + l16];
}

// write_tile for whole tiles whose epilogue operand was prefetched.
template <int MODE, int TM, int TN>
__device__ __forceinline__ void write_tile_pre(const GemmArgs& g, const floatx4 (&acc)[TM][TN],
                                               const floatx4 (&pre)[TM][TN], int r0, int c0, int g16,
                                               int l16) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const size_t idx = (size_t)(r0 + i * 16 + 4 * g16 + e) * g.ldc + c0 + j * 16 + l16;
        if constexpr (MODE == aur::EPI_RESID)
          g.C[idx] = pre[i][j][e] + acc[i][j][e];
        else
          g.C[idx] = acc[i][j][e] * gelu_tanh_grad(pre[i][j][e]);
      }
}

template <int BM, int BN, int BK, bool AK, bool BKC>
struct Smem {
  // k-contiguous operand: [rows][BK+4]; k-strided operand: [BK][cols+4].
  static constexpr int A_ELEMS = AK ? BM * (BK + 4) : BK * (BM + 4);
  static constexpr int B_ELEMS = BKC ? BN * (BK + 4) : BK * (BN + 4);
  static constexpr int STAGE = A_ELEMS + B_ELEMS;
  static constexpr int BYTES = 2 * STAGE * 4;
};

// Loads the (rows × BK) tile of a k-contiguous operand X(r,k)=x[r*ld+k], or
// the (BK × cols) tile of a k-strided operand X(r,k)=x[k*ld+r], into registers.
template <int ROWS, int BK, bool KCONTIG, bool VEC>
struct TileLoader {
  static constexpr int NV = ROWS * BK / 4 / kThreads;  // float4 per thread
  static_assert(NV >= 1 && ROWS * BK % (4 * kThreads) == 0, "tile/threads mismatch");
  floatx4 v[NV];

  __device__ __forceinline__ void load(const float* __restrict__ x, int ld, int r0, int rmax,
                                       int k0, int kmax, int tid) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = tid + i * kThreads;
      int r, k;
      if (KCONTIG) {
        r = f / (BK / 4);
        k = (f % (BK / 4)) * 4;
      } else {
        k = f / (ROWS / 4);
        r = (f % (ROWS / 4)) * 4;
      }
      const int gr = r0 + r, gk = k0 + k;
      floatx4 val = {0.f, 0.f, 0.f, 0.f};
      if (KCONTIG) {
        if (gr < rmax) {
          const float* p = x + (size_t)gr * ld + gk;
          if (VEC) {
            if (gk < kmax) val = *reinterpret_cast<const floatx4*>(p);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (gk + e < kmax) val[e] = p[e];
          }
        }
      } else {
        if (gk < kmax) {
          const float* p = x + (size_t)gk * ld + gr;
          if (VEC) {
            if (gr < rmax) val = *reinterpret_cast<const floatx4*>(p);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (gr + e < rmax) val[e] = p[e];
          }
        }
      }
      v[i] = val;
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ s, int tid) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = tid + i * kThreads;
      int off;
      if (KCONTIG) {
        off = (f / (BK / 4)) * (BK + 4) + (f % (BK / 4)) * 4;
      } else {
        off = (f / (ROWS / 4)) * (ROWS + 4) + (f % (ROWS / 4)) * 4;
      }
      *reinterpret_cast<floatx4*>(s + off) = v[i];
    }
  }
};

// Fragment of one 16-row slice for k chunk c: f[s] is this lane's operand of
// MFMA s, i.e. X(row0 + lane%16, 16c + 4·(lane/16) + s).
template <int ROWS, int BK, bool KCONTIG>
__device__ __forceinline__ floatx4 read_frag(const float* __restrict__ s, int row, int c, int g) {
  floatx4 f;
  if (KCONTIG) {
    f = *reinterpret_cast<const floatx4*>(s + row * (BK + 4) + 16 * c + 4 * g);
  } else {
    const float* p = s + (16 * c + 4 * g) * (ROWS + 4) + row;
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = p[e * (ROWS + 4)];
  }
  return f;
}

template <int BM, int BN, int BK, bool AK, bool BKC, bool VEC>
__global__ void __launch_bounds__(kThreads) gemm_f32_mfma(GemmArgs g) {
  select_batch(g);
  using S = Smem<BM, BN, BK, AK, BKC>;
  constexpr int WM = BM / 2, WN = BN / 2;  // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;
  __shared__ __attribute__((aligned(16))) float smem[2 * S::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int g16 = lane >> 4, l16 = lane & 15;

  // XCD-aware tile order: consecutive workgroups are dispatched round-robin
  // over the 8 XCDs; give each XCD a contiguous run of tiles, and walk that
  // run in groups of GM tile rows, column by column, so the ~64 tiles an
  // XCD runs at once form a GM × 8 block: each A and B panel slice is
  // fetched into that XCD's L2 once for 8 tiles instead of once per tile
  // (row-major order would stream every B panel through L2 per tile row).
  constexpr int GM = 8;
  const int ntiles = g.tiles_m * g.tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int per_group = GM * g.tiles_n;
  const int first_m = (pid / per_group) * GM;
  const int gsz = min(g.tiles_m - first_m, GM);
  const int tm = first_m + (pid % per_group) % gsz, tn = (pid % per_group) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;

  const int kbeg = blockIdx.z * g.k_chunk;
  const int kend = min(g.K, kbeg + g.k_chunk);
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

  TileLoader<BM, BK, AK, VEC> la;
  TileLoader<BN, BK, BKC, VEC> lb;

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  if (nk > 0) {
    la.load(g.A, g.lda, m0, g.M, kbeg, kend, tid);
    lb.load(g.B, g.ldb, n0, g.N, kbeg, kend, tid);
    la.store(smem, tid);
    lb.store(smem + S::A_ELEMS, tid);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      const int k0 = kbeg + (kt + 1) * BK;
      la.load(g.A, g.lda, m0, g.M, k0, kend, tid);
      lb.load(g.B, g.ldb, n0, g.N, k0, kend, tid);
    }
    const float* sa = smem + cur * S::STAGE;
    const float* sb = sa + S::A_ELEMS;
#pragma unroll
    for (int c = 0; c < BK / 16; ++c) {
      floatx4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = read_frag<BM, BK, AK>(sa, wm * WM + i * 16 + l16, c, g16);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = read_frag<BN, BK, BKC>(sb, wn * WN + j * 16 + l16, c, g16);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x4(fa[i][s], fb[j][s], acc[i][j]);
    }
    if (more) {
      float* na = smem + (cur ^ 1) * S::STAGE;
      la.store(na, tid);
      lb.store(na + S::A_ELEMS, tid);
    }
    __syncthreads();
  }

  // Epilogue: lane holds D[4·g16 + e][l16] of each 16×16 tile.
  write_tiles(g, acc, m0 + wm * WM, n0 + wn * WN, g16, l16, m0 + BM <= g.M && n0 + BN <= g.N);
}

// ------------------------------------------------ direct global→LDS path
// Whole-tile shapes (M, N multiples of the tile, every K range a multiple of
// 32, 16-byte aligned operands) load their tiles with global_load_lds_dwordx4:
// the data goes from memory straight into LDS, with no register round trip
// and no ds_write, so the waves spend their issue slots on fragment reads and
// MFMAs (measured on MI355X at NT 8192×8192×512: 106 → 133 TFLOP/s).  A wave
// load instruction fills 1 KB of consecutive LDS, so tiles are unpadded and
// bank conflicts are avoided by an XOR swizzle of 16-byte granules:
//   k-contiguous operand, [ROWS][32]: granule q of row r at q ^ ((r >> 1) & 7)
//     (a b128 fragment read of rows r..r+15 at one k hits 16 distinct bank
//     groups: row parity × the 8 swizzle values); [ROWS][16] (BK = 16, 64-byte
//     rows): q ^ ((r >> 2) & 3) (r mod 4 picks the bank quarter, r >> 2 the
//     granule within it);
//   k-strided operand, [BK][ROWS]: granule q of k-row k at q ^ (((k >> 2) & 3) << 2)
//     (the four k-rows 4g + s of a b32 fragment read land in 4 different
//     granule groups); rows of 8 granules (32-row tiles) use q ^ (((k >> 2) & 1) << 2),
//     two groups, so every granule stays in its row.
// The swizzle is an involution, so the same function maps physical → logical
// on the load side.
template <int ROWS, bool KCONTIG, int BK = 32, int NWV = 4>
struct DirectTile {
  static_assert(BK == 32 || BK == 16, "BK is 16 or 32");
  static constexpr int ELEMS = ROWS * BK;
  static constexpr int GPR = KCONTIG ? BK / 4 : ROWS / 4;  // 16-byte granules per LDS row
  static constexpr int RPI = 64 / GPR;                     // LDS rows per wave instruction
  static constexpr int NIW = (KCONTIG ? ROWS : BK) / RPI / NWV;  // instructions per wave
  static_assert(NIW >= 1 && (KCONTIG ? ROWS : BK) % (RPI * NWV) == 0, "tile too small for the waves");

  static_assert(KCONTIG || GPR >= 8, "the k-strided swizzle needs at least 8 granules per LDS row");
  __device__ static __forceinline__ int phys(int lrow, int q) {
    if (KCONTIG) return BK == 32 ? q ^ ((lrow >> 1) & 7) : q ^ ((lrow >> 2) & 3);
    // k-strided rows of 32 floats (8 granules, 32-row tiles) XOR with 0 or 4
    // only: the wider XOR of 16-granule rows would leave the row (and the
    // tile: past the end of the operand at its last column tile).
    return q ^ (((lrow >> 2) & (GPR >= 16 ? 3 : 1)) << 2);
  }
  // This wave's share of the tile at (row origin r0, k origin k0).
  __device__ static __forceinline__ void issue(const float* __restrict__ x, int ld, int r0, int k0,
                                               float* lds, int w, int lane) {
#pragma unroll
    for (int j = 0; j < NIW; ++j) {
      const int L0 = RPI * (NIW * w + j);
      const int lrow = L0 + lane / GPR, q = phys(lrow, lane % GPR);
      const float* src = KCONTIG ? x + (size_t)(r0 + lrow) * ld + k0 + 4 * q
                                 : x + (size_t)(k0 + lrow) * ld + r0 + 4 * q;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds + L0 * GPR * 4), 16,
                                       0, 0);
    }
  }
  // f[s] = X(row, 16c + 4g + s), the same k permutation as read_frag.
  __device__ static __forceinline__ floatx4 frag(const float* __restrict__ lds, int row, int c, int g) {
    floatx4 f;
    if (KCONTIG) {
      f = *reinterpret_cast<const floatx4*>(lds + row * BK + 4 * phys(row, 4 * c + g));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = 16 * c + 4 * g + e;
        f[e] = lds[k * ROWS + 4 * phys(k, row >> 2) + (row & 3)];
      }
    }
    return f;
  }
};

// PRE (epilogue operand prefetch, whole output tiles without split-K): the
// residual R (EPI_RESID) or the activation X (EPI_GELU_BWD) of this wave's
// tile is loaded into registers with the last K step, so its HBM latency
// hides under the final MFMAs instead of stalling the store.
//
// BK: K per LDS stage.  The 256×128 tile uses BK = 16 (48 KB of LDS for both
// stages, so two blocks share a CU) and its 128 accumulators per lane must fit
// beside the fragments in the 256 registers of two waves per SIMD.  Its waves
// each own 128×64 outputs: 6 load instructions per 128 MFMAs instead of 8,
// and 12 fragment reads per 32 MFMAs instead of 8 per 16.
template <int BM, int BN, bool AK, bool BKC, int PRE = 0, int BK = 32, int NW = 4>
__global__ void __launch_bounds__(64 * NW, (BM == 256 || NW == 8 ? 2 : 1)) gemm_f32_mfma_direct(GemmArgs g) {
  select_batch(g);
  using TA = DirectTile<BM, AK, BK, NW>;
  using TB = DirectTile<BN, BKC, BK, NW>;
  constexpr int ST = TA::ELEMS + TB::ELEMS;
  constexpr int WGN = NW / 2;  // waves along N (two along M)
  constexpr int WM = BM / 2, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
  __shared__ __attribute__((aligned(1024))) float smem[2 * ST];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int g16 = lane >> 4, l16 = lane & 15;
  // Tile order: as gemm_f32_mfma (contiguous run per XCD, 8-row groups).
  constexpr int GM = 8;
  const int ntiles = g.tiles_m * g.tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int per_group = GM * g.tiles_n;
  const int first_m = (pid / per_group) * GM;
  const int gsz = min(g.tiles_m - first_m, GM);
  const int m0 = (first_m + (pid % per_group) % gsz) * BM, n0 = ((pid % per_group) / gsz) * BN;
  const int kbeg = blockIdx.z * g.k_chunk;
  const int nk = (min(g.K, kbeg + g.k_chunk) - kbeg) / BK;

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 pre[PRE != 0 ? TM : 1][PRE != 0 ? TN : 1];

  if (nk > 0) {
    TA::issue(g.A, g.lda, m0, kbeg, smem, wave, lane);
    TB::issue(g.B, g.ldb, n0, kbeg, smem + TA::ELEMS, wave, lane);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // Software pipeline over K stages (two LDS stages, one barrier per stage).
  // A stage's MFMAs are split into two halves around the barrier: the first
  // half carries the LDS fragment reads the second half needs; the barrier
  // (after this wave's loads of the next stage landed) releases the stage
  // just read, so the second half carries the global→LDS loads of the stage
  // after next and the first-half fragment reads of the next stage.  The
  // loads and reads are spread one per MFMA (sched_group_barrier), so the
  // MFMA pipe is not left idle while a burst of them issues — which with one
  // or two waves per SIMD nothing else covers (measured on MI355X, C1 sweep
  // 126.5-126.8 → 128.4-129.1 TFLOP/s, 8192×512×2048 A@Bᵀ 124.9 → 129.4).
  // The last two stages are peeled (no loads past the end), so the loop body
  // has no branch and the interleave spans it.
  //   BK = 32: the halves are the two 16-wide k chunks of the stage.
  //   BK = 16 (the 256×128 tile): the halves are the rows i < TM/2 and
  //   i ≥ TM/2 of A; B's fragments are double-buffered.
  // Instruction classes for sched_group_barrier: 0x008 MFMA, 0x020 VMEM
  // read, 0x100 DS read.
  constexpr int NLD = TA::NIW + TB::NIW;  // global→LDS loads per stage and wave
  if constexpr (BK == 16) {
    static_assert(TM % 2 == 0, "row halves");
    constexpr int H = TM / 2;
    constexpr int NRA = H * (AK ? 1 : 4), NRB = TN * (BKC ? 1 : 4);  // DS reads
    constexpr int NMF = 4 * H * TN;  // MFMAs per half
    constexpr int R1 = NRA < NMF ? NRA : NMF;
    constexpr int L2 = NLD < NMF ? NLD : NMF;
    constexpr int R2 = NRA + NRB < NMF - L2 ? NRA + NRB : NMF - L2;
    floatx4 fa[TM], fb[TN], fbn[TN];
    if (nk > 1) {
      TA::issue(g.A, g.lda, m0, kbeg + BK, smem + ST, wave, lane);
      TB::issue(g.B, g.ldb, n0, kbeg + BK, smem + ST + TA::ELEMS, wave, lane);
    }
#pragma unroll
    for (int i = 0; i < H; ++i) fa[i] = TA::frag(smem, wm * WM + i * 16 + l16, 0, g16);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[j] = TB::frag(smem + TA::ELEMS, wn * WN + j * 16 + l16, 0, g16);
    // One stage.  MODE 0: loads the stage after next; 1 (the second-to-last
    // stage): loads nothing; 2 (the last): no barrier or next-stage reads
    // either, and fetches the epilogue operand instead.
    auto step = [&](int kt, auto mode) {
      constexpr int MODE = decltype(mode)::value;
      constexpr bool LAST = MODE == 2;
      if constexpr (LAST && PRE != 0) load_epi_operand(g, pre, m0 + wm * WM, n0 + wn * WN, g16, l16, PRE);
      const float* sa = smem + (kt & 1) * ST;
#pragma unroll
      for (int i = H; i < TM; ++i) fa[i] = TA::frag(sa, wm * WM + i * 16 + l16, 0, g16);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int i = 0; i < H; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x4(fa[i][s4], fb[j][s4], acc[i][j]);
#pragma unroll
      for (int r = 0; r < R1; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if constexpr (NMF > R1) __builtin_amdgcn_sched_group_barrier(0x008, NMF - R1, 0);
      if constexpr (!LAST) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of the next stage landed
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (MODE == 0) {  // into the stage just released
          float* na = smem + (kt & 1) * ST;
          const int k0 = kbeg + (kt + 2) * BK;
          TA::issue(g.A, g.lda, m0, k0, na, wave, lane);
          TB::issue(g.B, g.ldb, n0, k0, na + TA::ELEMS, wave, lane);
        }
        const float* xa = smem + ((kt + 1) & 1) * ST;
#pragma unroll
        for (int i = 0; i < H; ++i) fa[i] = TA::frag(xa, wm * WM + i * 16 + l16, 0, g16);
#pragma unroll
        for (int j = 0; j < TN; ++j) fbn[j] = TB::frag(xa + TA::ELEMS, wn * WN + j * 16 + l16, 0, g16);
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int i = H; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x4(fa[i][s4], fb[j][s4], acc[i][j]);
      if constexpr (!LAST) {
        constexpr int NL = MODE == 0 ? L2 : 0;
#pragma unroll
        for (int r = 0; r < NL; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
#pragma unroll
        for (int r = 0; r < R2; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if constexpr (NMF > NL + R2) __builtin_amdgcn_sched_group_barrier(0x008, NMF - NL - R2, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = fbn[j];
      }
    };
    for (int kt = 0; kt + 2 < nk; ++kt) step(kt, std::integral_constant<int, 0>{});
    if (nk > 1) step(nk - 2, std::integral_constant<int, 1>{});
    if (nk > 0) step(nk - 1, std::integral_constant<int, 2>{});
  } else {
    static_assert(BK == 32, "two 16-wide k chunks per stage");
    constexpr int NRD = TM * (AK ? 1 : 4) + TN * (BKC ? 1 : 4);  // DS reads per chunk
    constexpr int NMF = 4 * TM * TN;                              // MFMAs per chunk
    constexpr int R1 = NRD < NMF ? NRD : NMF;
    constexpr int L2 = NLD < NMF ? NLD : NMF;
    constexpr int R2 = NRD < NMF - L2 ? NRD : NMF - L2;
    floatx4 f0a[TM], f0b[TN], f1a[TM], f1b[TN];
    if (nk > 1) {
      TA::issue(g.A, g.lda, m0, kbeg + BK, smem + ST, wave, lane);
      TB::issue(g.B, g.ldb, n0, kbeg + BK, smem + ST + TA::ELEMS, wave, lane);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) f0a[i] = TA::frag(smem, wm * WM + i * 16 + l16, 0, g16);
#pragma unroll
    for (int j = 0; j < TN; ++j) f0b[j] = TB::frag(smem + TA::ELEMS, wn * WN + j * 16 + l16, 0, g16);
    auto step = [&](int kt, auto mode) {  // MODE as in the BK = 16 loop
      constexpr int MODE = decltype(mode)::value;
      constexpr bool LAST = MODE == 2;
      if constexpr (LAST && PRE != 0) load_epi_operand(g, pre, m0 + wm * WM, n0 + wn * WN, g16, l16, PRE);
      const float* sa = smem + (kt & 1) * ST;
      const float* sb = sa + TA::ELEMS;
#pragma unroll
      for (int i = 0; i < TM; ++i) f1a[i] = TA::frag(sa, wm * WM + i * 16 + l16, 1, g16);
#pragma unroll
      for (int j = 0; j < TN; ++j) f1b[j] = TB::frag(sb, wn * WN + j * 16 + l16, 1, g16);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x4(f0a[i][s4], f0b[j][s4], acc[i][j]);
#pragma unroll
      for (int r = 0; r < R1; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if constexpr (NMF > R1) __builtin_amdgcn_sched_group_barrier(0x008, NMF - R1, 0);
      if constexpr (!LAST) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of the next stage landed
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (MODE == 0) {  // into the stage just released
          float* na = smem + (kt & 1) * ST;
          const int k0 = kbeg + (kt + 2) * BK;
          TA::issue(g.A, g.lda, m0, k0, na, wave, lane);
          TB::issue(g.B, g.ldb, n0, k0, na + TA::ELEMS, wave, lane);
        }
        const float* xa = smem + ((kt + 1) & 1) * ST;
#pragma unroll
        for (int i = 0; i < TM; ++i) f0a[i] = TA::frag(xa, wm * WM + i * 16 + l16, 0, g16);
#pragma unroll
        for (int j = 0; j < TN; ++j) f0b[j] = TB::frag(xa + TA::ELEMS, wn * WN + j * 16 + l16, 0, g16);
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x4(f1a[i][s4], f1b[j][s4], acc[i][j]);
      if constexpr (!LAST) {
        constexpr int NL = MODE == 0 ? L2 : 0;
#pragma unroll
        for (int r = 0; r < NL; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
#pragma unroll
        for (int r = 0; r < R2; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if constexpr (NMF > NL + R2) __builtin_amdgcn_sched_group_barrier(0x008, NMF - NL - R2, 0);
      }
    };
    for (int kt = 0; kt + 2 < nk; ++kt) step(kt, std::integral_constant<int, 0>{});
    if (nk > 1) step(nk - 2, std::integral_constant<int, 1>{});
    if (nk > 0) step(nk - 1, std::integral_constant<int, 2>{});
  }

  if constexpr (PRE != 0) {
    if (nk == 0) load_epi_operand(g, pre, m0 + wm * WM, n0 + wn * WN, g16, l16, PRE);
    write_tile_pre<PRE>(g, acc, pre, m0 + wm * WM, n0 + wn * WN, g16, l16);
  } else {
    write_tiles(g, acc, m0 + wm * WM, n0 + wn * WN, g16, l16, /*full=*/true);
  }
}

// v(m,n) = Σ_{z=0..splits-1} P[z][m][n] summed in increasing z, then the
// fused epilogue writes C (and C2).
__global__ void __launch_bounds__(256) splitk_reduce(const float* __restrict__ P, float* __restrict__ C,
                                                      int M, int N, int ldc, int splits,
                                                      aur::Epilogue epi) {
  const size_t total = (size_t)M * N;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    float s = 0.f;  // splits == 0 (K == 0): the epilogue of an empty product
    for (int z = 0; z < splits; ++z) s += P[(size_t)z * total + i];
    const size_t row = i / N, col = i % N;
    apply_epilogue(epi, C, row * ldc + col, s);
  }
}

// splitk_reduce for N % 4 == 0: four consecutive outputs per thread (float4
// partial loads, 32-bit index math), the same increasing-z sum per element.
__global__ void __launch_bounds__(256) splitk_reduce4(const float* __restrict__ P, float* __restrict__ C,
                                                       int M, int N, int ldc, int splits,
                                                       aur::Epilogue epi) {
  const size_t plane = (size_t)M * N;
  const unsigned total4 = (unsigned)(plane / 4), un = (unsigned)N;
  for (unsigned i = blockIdx.x * blockDim.x + threadIdx.x; i < total4; i += gridDim.x * blockDim.x) {
    const unsigned e = 4 * i;
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
    for (int z = 0; z < splits; ++z) s += *reinterpret_cast<const floatx4*>(P + (size_t)z * plane + e);
    const unsigned row = e / un, col = e - row * un;
    const size_t idx = (size_t)row * ldc + col;
#pragma unroll
    for (int k = 0; k < 4; ++k) apply_epilogue(epi, C, idx + k, s[k]);
  }
}

// ------------------------------------------------------------ skinny A@Bᵀ
// Decode-shaped C[M ≤ 16·MT, N] = X[M, K]·W[N, K]ᵀ (M = sequences decoded
// together): bound by streaming W once, and too small for the tiled
// kernel's per-K-step LDS pipeline.  A block owns 16 columns of N and its
// K range; in each pass its W waves take W·U consecutive 16-wide k-chunks,
// U contiguous chunks per wave, all loads issued before the MFMAs (X, a few
// hundred KB, comes from L2).  The launcher picks U so that the decode
// shapes need exactly one pass.  Two accumulator sets halve the MFMA
// dependency chains; the per-wave tiles are summed through LDS in wave
// order (deterministic) before the epilogue.  One launch, no inter-block
// sync.  With gridDim.y > 1 the block only covers K range blockIdx.y of
// gridDim.y and stores its tile to P[blockIdx.y] with no epilogue: the
// CONSUMER of the product sums the ranges in increasing order.
//
// Loads are coalesced: lanes 4r..4r+3 read row r's 64 contiguous bytes of a
// 16-row × 16-k chunk (in the MFMA operand layout neighbouring lanes would
// read different rows, one 16-byte L1 access per lane — measured 2× slower
// at the decode shapes).  One ds_bpermute per component then moves the
// chunk into the MFMA layout (lane 16g+m holds row m, k offset 4g).
__device__ __forceinline__ floatx4 to_mfma_layout(floatx4 v, int addr) {
  floatx4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(v[e])));
  return r;
}

template <int MT, int W, int U>
__global__ void __launch_bounds__(64 * W) skinny_nt_kernel(GemmArgs g) {
  __shared__ float red[W][16 * MT][17];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g16 = lane >> 4, l16 = lane & 15;
  const int lr = lane >> 2, lk = (lane & 3) * 4;       // load mapping: row lr, k offset lk
  const int perm = 4 * (4 * l16 + g16);                // bpermute byte address of the source lane
  const int n0 = blockIdx.x * 16;
  const bool wrow_ok = n0 + lr < g.N;
  const int nchunks_all = (g.K + 15) / 16;
  const int cpb = (nchunks_all + gridDim.y - 1) / gridDim.y;  // chunks of this block's K range
  const int kb = blockIdx.y * cpb, ke = min(nchunks_all, kb + cpb);
  const float* wrow = g.B + (size_t)(wrow_ok ? n0 + lr : 0) * g.ldb;
  floatx4 acc[MT], acc2[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = acc2[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = kb + w * U; c0 < ke; c0 += W * U) {
    // Branch-free loads: an out-of-range row or k is clamped to an in-bounds
    // address and its value replaced by 0 after the scheduling barrier, so
    // every load of the pass is issued first and each MFMA waits only for
    // its own operands.  A chunk past the range is all zeros and adds
    // nothing: no branch between the loads and the math.
    floatx4 wf[U], xf[U][MT];
    bool kv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = 16 * (c0 + u) + lk;
      kv[u] = c0 + u < ke && k < g.K;  // K % 4 == 0: a float4 is all in or all out
      const int kc = kv[u] ? k : 0;
      wf[u] = *reinterpret_cast<const floatx4*>(wrow + kc);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int r = 16 * i + lr;
        xf[u][i] = *reinterpret_cast<const floatx4*>(g.A + (size_t)(r < g.M ? r : 0) * g.lda + kc);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool wv = wrow_ok && kv[u];
      const floatx4 wz = to_mfma_layout(
          floatx4{wv ? wf[u][0] : 0.f, wv ? wf[u][1] : 0.f, wv ? wf[u][2] : 0.f, wv ? wf[u][3] : 0.f}, perm);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const bool xv = kv[u] && 16 * i + lr < g.M;
        const floatx4 xz = to_mfma_layout(floatx4{xv ? xf[u][i][0] : 0.f, xv ? xf[u][i][1] : 0.f,
                                                  xv ? xf[u][i][2] : 0.f, xv ? xf[u][i][3] : 0.f},
                                          perm);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if (u & 1)
            acc2[i] = mfma16x16x4(xz[s], wz[s], acc2[i]);
          else
            acc[i] = mfma16x16x4(xz[s], wz[s], acc[i]);
        }
      }
    }
  }
  // acc + acc2 = partial C[16i + 4·g16 + e][n0 + l16] of this wave's chunks
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[w][16 * i + 4 * g16 + e][l16] = acc[i][e] + acc2[i][e];
  __syncthreads();
  for (int idx = tid; idx < 16 * MT * 16; idx += 64 * W) {
    const int row = idx >> 4, col = idx & 15;
    if (row >= g.M || n0 + col >= g.N) continue;
    float v = red[0][row][col];
#pragma unroll
    for (int ww = 1; ww < W; ++ww) v += red[ww][row][col];
    if (gridDim.y > 1)
      g.P[((size_t)blockIdx.y * g.M + row) * g.N + n0 + col] = v;
    else
      apply_epilogue(g.epi, g.C, (size_t)row * g.ldc + n0 + col, v);
  }
}

// ------------------------------------------------ decode K-range partials
// P[z][M ≤ 16·MT][N] = X[M, K_z]·W[N, K_z]ᵀ for K range z = blockIdx.y of
// length k_chunk.  A 256-thread block owns 64 columns and one K range; its X
// and W slices go through LDS 64 k at a time with coalesced float4 loads (a
// wave load instruction reads four 256-byte row pieces), the next slice
// prefetched into registers while the current one is multiplied; wave w
// multiplies columns 16w..16w+15.  Against the 16-column skinny kernel,
// every X byte staged here serves 4× more W bytes, and the K ranges keep
// about one block per CU in flight even for N = d_model.  No epilogue:
// the consumer sums the ranges in increasing order.
template <int MT>
__global__ void __launch_bounds__(256) wide_partials_kernel(GemmArgs g) {
  constexpr int SUB = 64, LD = SUB + 4, XR = 16 * MT;
  constexpr int XPT = XR * SUB / 4 / 256, WPT = 64 * SUB / 4 / 256;  // float4 per thread
  __shared__ __attribute__((aligned(16))) float xs[XR * LD];
  __shared__ __attribute__((aligned(16))) float ws[64 * LD];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g16 = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * 64;
  const int kb = blockIdx.y * g.k_chunk, ke = min(g.K, kb + g.k_chunk);
  floatx4 xr[XPT], wr[WPT];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int f = tid + 256 * i, r = f / (SUB / 4), k = k0 + (f % (SUB / 4)) * 4;
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (n0 + r < g.N && k < ke) v = *reinterpret_cast<const floatx4*>(g.B + (size_t)(n0 + r) * g.ldb + k);
      wr[i] = v;
    }
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int f = tid + 256 * i, r = f / (SUB / 4), k = k0 + (f % (SUB / 4)) * 4;
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (r < g.M && k < ke) v = *reinterpret_cast<const floatx4*>(g.A + (size_t)r * g.lda + k);
      xr[i] = v;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int f = tid + 256 * i;
      *reinterpret_cast<floatx4*>(ws + (f / (SUB / 4)) * LD + (f % (SUB / 4)) * 4) = wr[i];
    }
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int f = tid + 256 * i;
      *reinterpret_cast<floatx4*>(xs + (f / (SUB / 4)) * LD + (f % (SUB / 4)) * 4) = xr[i];
    }
  };
  floatx4 acc[MT], acc2[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = acc2[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  load(kb);
  store();
  __syncthreads();
  for (int k0 = kb; k0 < ke; k0 += SUB) {
    const bool more = k0 + SUB < ke;
    if (more) load(k0 + SUB);
#pragma unroll
    for (int u = 0; u < SUB / 16; ++u) {
      const int k = 16 * u + 4 * g16;
      const floatx4 wf = *reinterpret_cast<const floatx4*>(ws + (16 * wv + l16) * LD + k);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const floatx4 xf = *reinterpret_cast<const floatx4*>(xs + (16 * i + l16) * LD + k);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if (u & 1)
            acc2[i] = mfma16x16x4(xf[s], wf[s], acc2[i]);
          else
            acc[i] = mfma16x16x4(xf[s], wf[s], acc[i]);
        }
      }
    }
    if (more) {
      __syncthreads();  // every wave is done with the slice
      store();
      __syncthreads();
    }
  }
  const int col = n0 + 16 * wv + l16;
  if (col < g.N) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * i + 4 * g16 + e;
        if (row < g.M) g.P[((size_t)blockIdx.y * g.M + row) * g.N + col] = acc[i][e] + acc2[i][e];
      }
  }
}

// ------------------------------------ decode K-range partials, short ranges
// P[z][M ≤ 16·MT][N] for K range z of KR (64, 128 or 256) and N % 64 == 0.  A
// 256-thread block owns 64 columns (16 per wave) and one range.  Each wave
// issues every W load of its 16 rows × KR first (coalesced: lanes 4r..4r+3
// read row r's 64 contiguous bytes per 16-k chunk, moved into the MFMA
// layout with ds_bpermute), the X slice [M][KR] goes to LDS once for the
// four waves, then the MFMAs run as the W chunks land.  With these short
// ranges a CU holds three or more blocks, so the X bytes each CU reads stay
// below its W bytes — the full-K skinny kernel reads all of X per 16
// columns, twice its W bytes at K = 1024.
template <int MT, int KR>
__global__ void __launch_bounds__(256) stream_partials_kernel(GemmArgs g) {
  constexpr int XR = 16 * MT, LDX = KR + 4, NC = KR / 16;
  constexpr int XPT = XR * KR / 4 / 256;  // float4 of the X slice per thread
  static_assert(XPT >= 1 && XR * KR % 1024 == 0, "X slice/threads mismatch");
  __shared__ __attribute__((aligned(16))) float xs[XR * LDX];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g16 = lane >> 4, l16 = lane & 15;
  const int lr = lane >> 2, lk = (lane & 3) * 4;
  const int perm = 4 * (4 * l16 + g16);
  const int n0 = blockIdx.x * 64 + 16 * w;
  const int kb = blockIdx.y * KR;
  floatx4 xr[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int f = tid + 256 * i, r = f / (KR / 4), c = (f % (KR / 4)) * 4;
    // rows past M read row 0 (in bounds) and stage zeros
    const floatx4 v = *reinterpret_cast<const floatx4*>(g.A + (size_t)(r < g.M ? r : 0) * g.lda + kb + c);
    xr[i] = r < g.M ? v : floatx4{0.f, 0.f, 0.f, 0.f};
  }
  floatx4 wf[NC];
  const float* wrow = g.B + (size_t)(n0 + lr) * g.ldb + kb + lk;
#pragma unroll
  for (int c = 0; c < NC; ++c) wf[c] = *reinterpret_cast<const floatx4*>(wrow + 16 * c);
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int f = tid + 256 * i, r = f / (KR / 4), c = (f % (KR / 4)) * 4;
    *reinterpret_cast<floatx4*>(xs + r * LDX + c) = xr[i];
  }
  __syncthreads();
  floatx4 acc[MT], acc2[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = acc2[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const floatx4 wz = to_mfma_layout(wf[c], perm);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const floatx4 xf = *reinterpret_cast<const floatx4*>(xs + (16 * i + l16) * LDX + 16 * c + 4 * g16);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (c & 1)
          acc2[i] = mfma16x16x4(xf[s], wz[s], acc2[i]);
        else
          acc[i] = mfma16x16x4(xf[s], wz[s], acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 16 * i + 4 * g16 + e;
      if (row < g.M) g.P[((size_t)blockIdx.y * g.M + row) * g.N + n0 + l16] = acc[i][e] + acc2[i][e];
    }
}

struct Plan {
  int bm, bn, splits, k_chunk;
};

constexpr int kBK = 32;

// Launch plan: tile shape and split-K count, chosen by a time model.  Blocks
// are spread over the CUs, so the busiest CU runs L = ceil(blocks / CUs)
// blocks of f = 2·BM·BN·k_chunk FLOP each, at the CU's peak (256 FLOP/clk)
// times the tile's relative MFMA efficiency, and slower still when the CU
// holds a single block (one wave per SIMD leaves LDS and barrier latency
// exposed).  Split-K adds its reduction pass: the partial planes, the output
// and any epilogue operand (extra_planes) through HBM, plus one launch.
// Splits keep ≥ 512 of K per block.  The lowest modelled time wins, ties
// going to the larger tile and fewer splits.  The constants are fitted on
// MI355X to every forced configuration (6 tiles × split-K 1…16) of 50
// shapes — the config-1 and config-3 GEMMs of all three forms at M = 8192 /
// 16384 and at one GPU's 8-way data-parallel share, M = 1024 / 2048 — timed
// by `bench.py --only planner`: tile efficiency 1.00 / 0.95 / 0.90 / 0.70 /
// 0.55 (128×128 / 128×64 / 64×64 / 64×32 / 32×32), single-block factor 0.95
// / 0.95 / 0.85 / 0.7 / 0.7 (the software-pipelined main loop keeps one
// wave per SIMD nearly as busy as two), 3 TB/s for the reduction and 2 µs
// per launch; on the fitting run the pick was within 1.6 % of the measured
// best on every shape (0.15 % on average).  The two small tiles serve
// few-tile shapes (M = 1024 with N = 512: 24 → 38 % of peak).
//
// allow_wide admits the 256×128 tile (direct-load kernel only: whole tiles,
// aligned operands, A k-contiguous — with A k-strided it measured 4 % slower
// than 128×128 — and no prefetched epilogue operand): 1.03 relative
// efficiency (NT 8192×8192×512: 135.8 vs 130.7 TFLOP/s), 0.75 when alone on a CU.
Plan choose_plan(const aur_ctx* ctx, int M, int N, int K, bool allow_split, int batch = 1,
                 int extra_planes = 0, bool allow_wide = false) {
  const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  constexpr double kCuFlops = 256.0 * 2.4e9;  // FLOP/s per CU, fp32 MFMA
  constexpr double kHbm = 3.0e12, kLaunch = 2.0e-6;
  struct Cand {
    int bm, bn;
    double eff, single;
  };
  static constexpr Cand cands[] = {{256, 128, 1.03, 0.75}, {128, 128, 1.00, 0.95}, {128, 64, 0.95, 0.95},
                                   {64, 64, 0.90, 0.85},   {64, 32, 0.70, 0.7},    {32, 32, 0.55, 0.7}};
  Plan p{128, 128, 1, K};
  double best = 1e30;
  for (const Cand& c : cands) {
    if (c.bm == 256 && !allow_wide) continue;
    const long tiles = (long)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * batch;
    for (int s = 1; s <= 16; s *= 2) {
      if (s > 1 && (!allow_split || K / s < 512)) break;
      int chunk = (K + s - 1) / s;
      chunk = (chunk + kBK - 1) / kBK * kBK;
      const int splits = (K + chunk - 1) / chunk;
      const long blocks = tiles * splits;
      const long per_cu = (blocks + cus - 1) / cus;
      const double f = 2.0 * c.bm * c.bn * chunk;
      double t = per_cu * f / (kCuFlops * c.eff * (per_cu == 1 ? c.single : 1.0));
      if (splits > 1) t += (splits + 1.0 + extra_planes) * M * N * 4.0 * batch / kHbm + kLaunch;
      if (t < best * (1.0 - 1e-9)) {
        best = t;
        p = {c.bm, c.bn, splits, chunk};
      }
    }
  }
  // Tuning override: AUR_GEMM_CFG="BMxBN[:splits]".
  if (const char* env = std::getenv("AUR_GEMM_CFG")) {
    int bm = 0, bn = 0, sp = 1;
    if (std::sscanf(env, "%dx%d:%d", &bm, &bn, &sp) >= 2 &&
        ((bm == 128 && bn == 128) || (bm == 128 && bn == 64) || (bm == 64 && bn == 64) ||
         (bm == 64 && bn == 32) || (bm == 32 && bn == 32) || (bm == 256 && bn == 128 && allow_wide))) {
      p.bm = bm;
      p.bn = bn;
      if (!allow_split) sp = 1;
      sp = std::max(1, sp);
      int chunk = (K + sp - 1) / sp;
      chunk = (chunk + kBK - 1) / kBK * kBK;
      p.splits = std::max(1, (K + chunk - 1) / chunk);
      p.k_chunk = chunk;
    }
  }
  return p;
}

// cus: the device's CU count (0: unknown).  A 128×128 or 128×64 grid of at
// most one block per CU runs the 8-wave kernel (each wave 64×32 or 64×16 of
// the tile): one block then puts two waves on every SIMD, which cover each
// other's barrier and LDS waits (measured on MI355X: 8192×512×512 114.6 →
// 118.1 TFLOP/s, 8192×512×2048 130.6 → 134.8, 2048×1024×4096 with 128×64
// tiles 2-3 % faster; on grids of two or more blocks per CU the 4-wave
// kernel is 1-2 % faster).
template <int BM, int BN, bool AK, bool BKC>
void launch_tile(const GemmArgs& a, int splits, bool vec, hipStream_t st, int batch, int cus) {
  dim3 grid(a.tiles_m * a.tiles_n, batch, splits);
  if constexpr (BM == 256) {  // whole tiles only: the planner's allow_wide condition
    hipLaunchKernelGGL((gemm_f32_mfma_direct<BM, BN, AK, BKC, 0, 16>), grid, dim3(kThreads), 0, st, a);
  } else {
  const bool whole = vec && a.M % BM == 0 && a.N % BN == 0 && a.K % 32 == 0 && a.k_chunk % 32 == 0;
  if (whole && std::getenv("AUR_GEMM_STAGED") == nullptr) {
    if constexpr (BM == 128 && (BN == 128 || BN == 64)) {
      const long blocks = (long)a.tiles_m * a.tiles_n * batch * splits;
      if (cus > 0 && blocks <= cus && std::getenv("AUR_GEMM_NO_W8") == nullptr &&
          (a.split || a.epi.mode == aur::EPI_STORE || a.epi.mode == aur::EPI_ACCUM)) {
        hipLaunchKernelGGL((gemm_f32_mfma_direct<BM, BN, AK, BKC, 0, 32, 8>), grid, dim3(512), 0, st, a);
        return;
      }
    }
    if constexpr (BM == 128 && BN == 128) {
      if (!a.split && a.epi.mode == aur::EPI_RESID) {
        hipLaunchKernelGGL((gemm_f32_mfma_direct<BM, BN, AK, BKC, aur::EPI_RESID>), grid, dim3(kThreads), 0,
                           st, a);
        return;
      }
      if (!a.split && a.epi.mode == aur::EPI_GELU_BWD) {
        hipLaunchKernelGGL((gemm_f32_mfma_direct<BM, BN, AK, BKC, aur::EPI_GELU_BWD>), grid, dim3(kThreads), 0,
                           st, a);
        return;
      }
    }
    hipLaunchKernelGGL((gemm_f32_mfma_direct<BM, BN, AK, BKC>), grid, dim3(kThreads), 0, st, a);
  }
  else if (vec)
    hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, kBK, AK, BKC, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, kBK, AK, BKC, false>), grid, dim3(kThreads), 0, st, a);
  }
}

template <bool AK, bool BKC>
void launch_layout(const GemmArgs& a, const Plan& p, bool vec, hipStream_t st, int cus, int batch = 1) {
  if constexpr (AK) {
    if (p.bm == 256) return launch_tile<256, 128, AK, BKC>(a, p.splits, vec, st, batch, cus);
  }
  if (p.bm == 128 && p.bn == 128)
    launch_tile<128, 128, AK, BKC>(a, p.splits, vec, st, batch, cus);
  else if (p.bm == 128 && p.bn == 64)
    launch_tile<128, 64, AK, BKC>(a, p.splits, vec, st, batch, cus);
  else if (p.bm == 64 && p.bn == 64)
    launch_tile<64, 64, AK, BKC>(a, p.splits, vec, st, batch, cus);
  else if (p.bm == 64 && p.bn == 32)
    launch_tile<64, 32, AK, BKC>(a, p.splits, vec, st, batch, cus);
  else
    launch_tile<32, 32, AK, BKC>(a, p.splits, vec, st, batch, cus);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

// Scratch of aur_outer_accum_noalloc: the split-K partial tiles of one call,
// 2^24 floats (64 MiB) on every device the library runs on, held until the
// process ends.  Host code never uses this name as an address (on the host it
// is only a stand-in for the symbol): it takes each device's address from
// hipGetSymbolAddress once, at aur_init, and passes that to the kernels.
constexpr size_t kNoAllocScratchFloats = size_t(1) << 24;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace aur {

void noalloc_scratch_init(aur_ctx* ctx) {
  static std::mutex mu;
  static std::map<int, float*> per_device;  // device → address of its copy of `scratch`
  std::lock_guard<std::mutex> g(mu);
  auto it = per_device.find(ctx->device);
  if (it != per_device.end()) {
    ctx->noalloc_scratch = it->second;
    return;
  }
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    ctx->noalloc_err = e != hipSuccess ? (int)e : AUR_ENOMEM;
    (void)hipGetLastError();  // keep the failure from being reported by the next launch check
    return;
  }
  per_device[ctx->device] = static_cast<float*>(ptr);
  ctx->noalloc_scratch = static_cast<float*>(ptr);
}

// Split-K partial tiles: the caller's workspace (ws) or the context's
// grow-only one.
static int partials(aur_ctx* ctx, const Workspace* ws, size_t floats, float** out) {
  if (ws && ws->ptr) {
    if (ws->floats < floats)
      return set_error(ctx, AUR_ENOMEM, "gemm: workspace of %zu floats, %zu needed", ws->floats, floats);
    *out = ws->ptr;
    return 0;
  }
  // A graph captured now would keep the context workspace's address, which
  // a later growth frees: captured split-K work must bring its own.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  AUR_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return set_error(ctx, AUR_EINVAL, "gemm: split-K while the stream is captured needs a Workspace");
  int rc = ensure_workspace(ctx, floats * sizeof(float));
  if (rc) return rc;
  *out = static_cast<float*>(ctx->ws);
  return 0;
}

static void reduce_partials(aur_ctx* ctx, const float* P, float* C, int M, int N, int ldc, int splits,
                            const Epilogue& epi) {
  const size_t total = (size_t)M * N;
  if (N % 4 == 0 && total < (size_t(1) << 32) && splits > 0 && aligned16(P)) {
    const int blocks = (int)std::min<size_t>((total / 4 + 255) / 256, 4096);
    hipLaunchKernelGGL(splitk_reduce4, dim3(blocks), dim3(256), 0, ctx->stream, P, C, M, N, ldc, splits, epi);
    return;
  }
  int blocks = (int)std::min<size_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(splitk_reduce, dim3(blocks), dim3(256), 0, ctx->stream, P, C, M, N, ldc, splits, epi);
}

template <int MT, int W>
static void launch_skinny_u(dim3 grid, int u, const GemmArgs& a, hipStream_t st) {
  if (u <= 1) {
    hipLaunchKernelGGL((skinny_nt_kernel<MT, W, 1>), grid, dim3(64 * W), 0, st, a);
  } else if (u == 2) {
    hipLaunchKernelGGL((skinny_nt_kernel<MT, W, 2>), grid, dim3(64 * W), 0, st, a);
  } else if constexpr (MT == 4 || W == 16) {  // register budget: at most 4 chunks in flight
    hipLaunchKernelGGL((skinny_nt_kernel<MT, W, 4>), grid, dim3(64 * W), 0, st, a);
  } else {
    if (u <= 4)
      hipLaunchKernelGGL((skinny_nt_kernel<MT, W, 4>), grid, dim3(64 * W), 0, st, a);
    else
      hipLaunchKernelGGL((skinny_nt_kernel<MT, W, 8>), grid, dim3(64 * W), 0, st, a);
  }
}

// Decode-shaped A@Bᵀ (M ≤ 64, both operands k-contiguous, 16-byte vectors).
// splits > 1: K ranges write P[splits][M][N] instead of C (no epilogue).
// Waves per block W and chunks per wave U: the block's K range in one pass
// (W·U ≥ its 16-wide chunks) with as few chunks per wave as that allows;
// more than one block per CU's worth of columns (the tied head) prefers
// W = 8, so two blocks share a CU.  AUR_SKINNY_CFG="W:U" overrides (tuning).
static int skinny_nt(aur_ctx* ctx, const float* A, int lda, const float* B, int ldb, float* C, int ldc,
                     int M, int N, int K, const Epilogue& epi, float* P = nullptr, int splits = 1) {
  GemmArgs a{};
  a.A = A; a.B = B; a.C = C; a.M = M; a.N = N; a.K = K;
  a.lda = lda; a.ldb = ldb; a.ldc = ldc; a.epi = epi; a.P = P;
  const int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  const int blocks = (N + 15) / 16 * splits;
  const int nck = ((K + 15) / 16 + splits - 1) / splits;  // chunks per block
  int w = (mt == 4 || blocks > cus) ? 8 : 16;
  int u = 1;
  while (u < 8 && w * u < nck) u *= 2;
  if (mt == 4 && u > 4) u = 4;
  if (mt < 4 && w == 16 && u > 4) u = 4;
  if (const char* env = std::getenv("AUR_SKINNY_CFG")) {
    int ew = 0, eu = 0;
    if (std::sscanf(env, "%d:%d", &ew, &eu) == 2 && (ew == 4 || ew == 8 || ew == 16) &&
        (eu == 1 || eu == 2 || eu == 4 || eu == 8) && !(mt == 4 && (ew == 16 || eu == 8)) &&
        !(ew == 16 && eu == 8)) {
      w = ew;
      u = eu;
    }
  }
  dim3 grid((N + 15) / 16, splits);
  hipStream_t st = ctx->stream;
  if (mt == 1) {
    if (w == 16) launch_skinny_u<1, 16>(grid, u, a, st);
    else if (w == 8) launch_skinny_u<1, 8>(grid, u, a, st);
    else launch_skinny_u<1, 4>(grid, u, a, st);
  } else if (mt == 2) {
    if (w == 16) launch_skinny_u<2, 16>(grid, u, a, st);
    else if (w == 8) launch_skinny_u<2, 8>(grid, u, a, st);
    else launch_skinny_u<2, 4>(grid, u, a, st);
  } else {
    if (w == 8) launch_skinny_u<4, 8>(grid, u, a, st);
    else launch_skinny_u<4, 4>(grid, u, a, st);
  }
  AUR_LAUNCH_CHECK(ctx, "skinny_nt_kernel");
  return 0;
}

// C = epilogue(op(A)·op(B)) on ctx's stream.  See aur_gemm_ex for operand
// meaning and Epilogue (common.hpp) for the fused output forms.
int gemm(aur_ctx* ctx, bool a_kcontig, bool b_kcontig, const float* A, int lda, const float* B,
         int ldb, float* C, int ldc, int M, int N, int K, const Epilogue& epi, const Workspace* ws) {
  if (M < 0 || N < 0 || K < 0) return set_error(ctx, AUR_EINVAL, "gemm: negative dims");
  if (M == 0 || N == 0) return 0;
  if (!C || (K > 0 && (!A || !B))) return set_error(ctx, AUR_EINVAL, "gemm: null pointer");
  if ((epi.mode == EPI_RESID && !epi.R) || (epi.mode == EPI_GELU && !epi.C2) ||
      (epi.mode == EPI_GELU_BWD && !epi.X))
    return set_error(ctx, AUR_EINVAL, "gemm: epilogue operand missing");
  if (K == 0) {
    const size_t total = (size_t)M * N;
    int blocks = (int)std::min<size_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(splitk_reduce, dim3(blocks), dim3(256), 0, ctx->stream, nullptr, C, M, N, ldc,
                       0, epi);
    AUR_LAUNCH_CHECK(ctx, "splitk_reduce(K=0)");
    return 0;
  }
  // The A / B "row" extents (the contiguous index of a k-strided operand).
  const int a_rows = M, b_rows = N;
  const bool vec = aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                   (a_kcontig ? (K % 4 == 0) : (a_rows % 4 == 0)) &&
                   (b_kcontig ? (K % 4 == 0) : (b_rows % 4 == 0));
  if (vec && a_kcontig && b_kcontig && M <= 64)
    return skinny_nt(ctx, A, lda, B, ldb, C, ldc, M, N, K, epi);
  // Split-K only pays for long K with few output tiles; used for every form.
  const bool wide = vec && a_kcontig && M % 256 == 0 && N % 128 == 0 && K % 32 == 0 &&
                    epi.mode != EPI_RESID && epi.mode != EPI_GELU_BWD &&
                    std::getenv("AUR_GEMM_STAGED") == nullptr;
  Plan p = choose_plan(ctx, M, N, K, /*allow_split=*/true, 1, epi.mode == EPI_STORE ? 0 : 1, wide);
  GemmArgs a{};
  a.A = A;
  a.B = B;
  a.C = C;
  a.M = M;
  a.N = N;
  a.K = K;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.tiles_m = (M + p.bm - 1) / p.bm;
  a.tiles_n = (N + p.bn - 1) / p.bn;
  a.k_chunk = p.k_chunk;
  a.epi = epi;
  if (p.splits > 1) {
    int rc = partials(ctx, ws, (size_t)p.splits * M * N, &a.P);
    if (rc) return rc;
    a.split = 1;
  }
  if (a_kcontig && b_kcontig)
    launch_layout<true, true>(a, p, vec, ctx->stream, ctx->cu_count);
  else if (a_kcontig && !b_kcontig)
    launch_layout<true, false>(a, p, vec, ctx->stream, ctx->cu_count);
  else if (!a_kcontig && b_kcontig)
    launch_layout<false, true>(a, p, vec, ctx->stream, ctx->cu_count);
  else
    launch_layout<false, false>(a, p, vec, ctx->stream, ctx->cu_count);
  AUR_LAUNCH_CHECK(ctx, "gemm_f32_mfma");
  if (p.splits > 1) {
    reduce_partials(ctx, a.P, C, M, N, ldc, p.splits, epi);
    AUR_LAUNCH_CHECK(ctx, "splitk_reduce");
  }
  return 0;
}

int gemm(aur_ctx* ctx, bool a_kcontig, bool b_kcontig, const float* A, int lda, const float* B,
         int ldb, float* C, int ldc, int M, int N, int K, bool accumulate) {
  Epilogue e;
  e.mode = accumulate ? EPI_ACCUM : EPI_STORE;
  return gemm(ctx, a_kcontig, b_kcontig, A, lda, B, ldb, C, ldc, M, N, K, e, nullptr);
}

int gemm_batched(aur_ctx* ctx, bool a_kcontig, bool b_kcontig, const float* A, int lda, long long sA,
                 const float* B, int ldb, long long sB, float* C, int ldc, long long sC, int M, int N, int K,
                 int batch) {
  if (M < 1 || N < 1 || K < 1 || batch < 1 || batch > 65535)
    return set_error(ctx, AUR_EINVAL, "gemm_batched: bad dims (M=%d N=%d K=%d batch=%d)", M, N, K, batch);
  if (!A || !B || !C) return set_error(ctx, AUR_EINVAL, "gemm_batched: null pointer");
  if (batch == 1) return gemm(ctx, a_kcontig, b_kcontig, A, lda, B, ldb, C, ldc, M, N, K, false);
  const bool vec = aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0) && (sA % 4 == 0) &&
                   (sB % 4 == 0) && (a_kcontig ? (K % 4 == 0) : (M % 4 == 0)) &&
                   (b_kcontig ? (K % 4 == 0) : (N % 4 == 0));
  const bool wide = vec && a_kcontig && M % 256 == 0 && N % 128 == 0 && K % 32 == 0 &&
                    std::getenv("AUR_GEMM_STAGED") == nullptr;
  const Plan p = choose_plan(ctx, M, N, K, /*allow_split=*/false, batch, 0, wide);
  GemmArgs a{};
  a.A = A; a.B = B; a.C = C; a.M = M; a.N = N; a.K = K;
  a.lda = lda; a.ldb = ldb; a.ldc = ldc;
  a.tiles_m = (M + p.bm - 1) / p.bm;
  a.tiles_n = (N + p.bn - 1) / p.bn;
  a.k_chunk = p.k_chunk;
  a.sA = sA; a.sB = sB; a.sC = sC;
  if (a_kcontig && b_kcontig)
    launch_layout<true, true>(a, p, vec, ctx->stream, ctx->cu_count, batch);
  else if (a_kcontig && !b_kcontig)
    launch_layout<true, false>(a, p, vec, ctx->stream, ctx->cu_count, batch);
  else if (!a_kcontig && b_kcontig)
    launch_layout<false, true>(a, p, vec, ctx->stream, ctx->cu_count, batch);
  else
    launch_layout<false, false>(a, p, vec, ctx->stream, ctx->cu_count, batch);
  AUR_LAUNCH_CHECK(ctx, "gemm_f32_mfma (batched)");
  return 0;
}

int gemm_nt_partials_splits(int M, int N, int K) {
  (void)M;
  const int groups = (N + 63) / 64;
  int s = 1;
  while (groups * s < 256 && K / (2 * s) >= 64) s *= 2;
  // gemm_nt_partials cuts K into ranges of a multiple of 64: keep only a
  // count whose ranges are all non-empty (K = 384 fits 3 ranges of 128, not 4).
  for (; s > 1; --s) {
    const int chunk = ((K + s - 1) / s + 63) / 64 * 64;
    if ((K + chunk - 1) / chunk == s) break;
  }
  return s;
}

int gemm_nt_partials(aur_ctx* ctx, const float* A, int lda, const float* B, int ldb, float* P, int M, int N,
                     int K, int splits) {
  if (M < 1 || M > 64 || N < 1 || K < 1 || splits < 1 || (K & 3) || (lda & 3) || (ldb & 3) ||
      !aligned16(A) || !aligned16(B) || !P)
    return set_error(ctx, AUR_EINVAL, "gemm_nt_partials: unsupported shape or alignment");
  // K ranges of a multiple of 64; every one of the `splits` ranges non-empty.
  int chunk = (K + splits - 1) / splits;
  chunk = (chunk + 63) / 64 * 64;
  if ((K + chunk - 1) / chunk != splits)
    return set_error(ctx, AUR_EINVAL, "gemm_nt_partials: %d K ranges do not fit K=%d", splits, K);
  GemmArgs a{};
  a.A = A; a.B = B; a.P = P; a.M = M; a.N = N; a.K = K;
  a.lda = lda; a.ldb = ldb; a.k_chunk = chunk;
  dim3 grid((N + 63) / 64, splits);
  const bool stream = (chunk == 64 || chunk == 128 || chunk == 256) && N % 64 == 0 && K % chunk == 0;
  if (stream) {
#define AUR_STREAM_PARTIALS(MT)                                                                  \
  do {                                                                                            \
    if (chunk == 64)                                                                              \
      hipLaunchKernelGGL((stream_partials_kernel<MT, 64>), grid, dim3(256), 0, ctx->stream, a);  \
    else if (chunk == 128)                                                                        \
      hipLaunchKernelGGL((stream_partials_kernel<MT, 128>), grid, dim3(256), 0, ctx->stream, a); \
    else                                                                                          \
      hipLaunchKernelGGL((stream_partials_kernel<MT, 256>), grid, dim3(256), 0, ctx->stream, a); \
  } while (0)
    if (M <= 16)
      AUR_STREAM_PARTIALS(1);
    else if (M <= 32)
      AUR_STREAM_PARTIALS(2);
    else if (M <= 48)
      AUR_STREAM_PARTIALS(3);
    else
      AUR_STREAM_PARTIALS(4);
#undef AUR_STREAM_PARTIALS
    AUR_LAUNCH_CHECK(ctx, "stream_partials_kernel");
    return 0;
  }
  if (M <= 16)
    hipLaunchKernelGGL(wide_partials_kernel<1>, grid, dim3(256), 0, ctx->stream, a);
  else if (M <= 32)
    hipLaunchKernelGGL(wide_partials_kernel<2>, grid, dim3(256), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL(wide_partials_kernel<4>, grid, dim3(256), 0, ctx->stream, a);
  AUR_LAUNCH_CHECK(ctx, "wide_partials_kernel");
  return 0;
}

}  // namespace aur

extern "C" {

int aur_gemm_nn(aur_ctx* ctx, const float* a, const float* b, float* c, uint32_t m, uint32_t n,
                uint32_t k) {
  AUR_CHECK_CTX(ctx);
  return aur::gemm(ctx, true, false, a, (int)k, b, (int)n, c, (int)n, (int)m, (int)n, (int)k, false);
}

int aur_gemm_nt(aur_ctx* ctx, const float* a, const float* b, float* c, uint32_t m, uint32_t n,
                uint32_t k) {
  AUR_CHECK_CTX(ctx);
  return aur::gemm(ctx, true, true, a, (int)k, b, (int)k, c, (int)n, (int)m, (int)n, (int)k, false);
}

int aur_outer_accum(aur_ctx* ctx, const float* x, const float* d_y, float* dest, uint32_t d_out,
                    uint32_t d_in, uint32_t t) {
  AUR_CHECK_CTX(ctx);
  // dest(o,i) += Σ_t A(o,t)·B(t,i) with A(o,t) = d_y[t*d_out + o] (k-strided)
  // and B(t,i) = x[t*d_in + i] (k-strided).
  return aur::gemm(ctx, false, false, d_y, (int)d_out, x, (int)d_in, dest, (int)d_in, (int)d_out,
                   (int)d_in, (int)t, true);
}

int aur_outer_accum_noalloc(aur_ctx* ctx, const float* x, const float* d_y, float* dest, uint32_t d_out,
                            uint32_t d_in, uint32_t t) {
  AUR_CHECK_CTX(ctx);
  if (!ctx->noalloc_scratch)
    return aur::set_error(ctx, ctx->noalloc_err ? ctx->noalloc_err : AUR_ENOMEM,
                          "aur_outer_accum_noalloc: no scratch on device %d (hipGetSymbolAddress: %s)", ctx->device,
                          hipGetErrorString((hipError_t)ctx->noalloc_err));
  // The same launch plan and kernels as aur_outer_accum, with the split-K
  // partials in the device's scratch array instead of the context workspace.
  const aur::Workspace ws{ctx->noalloc_scratch, kNoAllocScratchFloats};
  aur::Epilogue e;
  e.mode = aur::EPI_ACCUM;
  const int rc = aur::gemm(ctx, false, false, d_y, (int)d_out, x, (int)d_in, dest, (int)d_in, (int)d_out, (int)d_in,
                           (int)t, e, &ws);
  if (rc == AUR_ENOMEM)  // the plan's partial tiles exceed the scratch: nothing was launched
    return aur::set_error(ctx, AUR_ELIMIT,
                          "aur_outer_accum_noalloc: d_out=%u d_in=%u t=%u needs more than the %zu floats of "
                          "scratch (%s)",
                          d_out, d_in, t, kNoAllocScratchFloats, ctx->last_error.c_str());
  return rc;
}

int aur_gemm_ex(aur_ctx* ctx, int a_kcontig, int b_kcontig, const float* a, uint32_t lda,
                const float* b, uint32_t ldb, float* c, uint32_t ldc, uint32_t m, uint32_t n,
                uint32_t k, int accumulate) {
  AUR_CHECK_CTX(ctx);
  // A row of each operand must fit its leading dimension (otherwise the last
  // rows read and write past the buffers), and every extent must fit an int.
  constexpr uint32_t kMax = 0x7fffffffu;
  if (m > kMax || n > kMax || k > kMax || lda > kMax || ldb > kMax || ldc > kMax)
    return aur::set_error(ctx, AUR_ELIMIT, "gemm_ex: extents above 2^31 - 1");
  if (lda < (a_kcontig ? k : m) || ldb < (b_kcontig ? k : n) || ldc < n)
    return aur::set_error(ctx, AUR_EINVAL, "gemm_ex: leading dimension below the row length (lda=%u ldb=%u ldc=%u)",
                          lda, ldb, ldc);
  return aur::gemm(ctx, a_kcontig != 0, b_kcontig != 0, a, (int)lda, b, (int)ldb, c, (int)ldc,
                   (int)m, (int)n, (int)k, accumulate != 0);
}

}  // extern "C"
