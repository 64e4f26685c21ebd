// Causal multi-head attention on gfx950 fp32 matrix cores, d_head any multiple
// of 8 up to 64 (any other d_head up to 64 through zero-padded heads).
//
// Reference semantics (src/attention.rs:396-550, src/gpu/attention.rs:21-331):
//   S = Q_h K_hᵀ / sqrt(d_head), S[i,j] = -inf for j > i, P = softmax_rows(S),
//   O_h = P V_h;  backward: dP = dO Vᵀ, rowdot_i = Σ_j P_ij dP_ij,
//   dS = P ⊙ (dP − rowdot), dQ += scale·dS K, dK += scale·dSᵀ Q, dV += Pᵀ dO.
//
// Instead of materialising P ([H,T,T] in the reference) the forward keeps
// the running row max / row sum of a flash-style tile loop and stores one
// log-sum-exp per row; the backward recomputes P tile by tile from it.
// rowdot_i equals Σ_c dO_ic O_ic, computed once per row (pass 1).  dK/dV
// come from a pass over query tiles per key tile (pass 2), which also stores
// each dS tile of the causal lower triangle to the workspace; dQ = dS·K is
// then a pass over those tiles per query tile (pass 3) that reads dS instead
// of recomputing S and dP.  Every output element has exactly one writer and
// a fixed summation order: the backward is deterministic, like the
// reference's 3-dispatch scheme (whose d_scores scratch is [H,T,T]).
//
// MFMA layout (v_mfma_f32_16x16x4_f32, see common.hpp).  A wave owns 16 rows
// (queries in the forward and dQ pass, keys in the dK/dV pass).  Scores are
// computed transposed (Sᵀ = K·Qᵀ), which leaves lane l holding column l%16
// of Sᵀ — all of them scores of ONE query row — so the softmax statistics
// are per-lane scalars and the Sᵀ accumulator registers are directly the
// B operand of the next product (Oᵀ = Vᵀ·Pᵀ).  The row max and sum are
// reduced over the four 16-lane groups with gfx950's row-swap permutes.
// The head dimension is covered in chunks of 16 (NC = ceil(DH/16)); when
// DH is not a multiple of 16 the last chunk's upper half (8 columns) is zero.
#include "common.hpp"

#include <algorithm>
#include <cstdlib>

namespace {

constexpr int TQ = 64;  // rows per tile (4 waves × 16)
constexpr float LOG2E = 1.4426950408889634f;

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* o;    // forward output (bwd pass 1)
  const float* dO;   // gradient of the output
  float* out;        // forward output
  float* lse;        // [B, H, T]
  float* D;          // [B, H, T] rowdot
  float* ds;         // [B, H, ntri] 64×64 dS tiles of the causal lower triangle (ds_slot)
  int ntri;          // nqt·(nqt+1)/2 tiles per (sequence, head)
  float* dq;
  float* dk;
  float* dv;
  int ld_qkv;        // row stride of q, k, v
  int ld_o;          // row stride of out / o / dO
  int ld_d;          // row stride of dq, dk, dv
  int T, H;
  float scale;       // 1/sqrt(d_head)
  int overwrite;     // backward: store dq/dk/dv instead of accumulating into them
};

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

// Max and sum over lanes l, l^16, l^32, l^48 (the four 16-lane rows), every
// lane getting the result.  v_permlane16_swap exchanges the odd rows of its
// first operand with the even rows of its second (v_permlane32_swap: the
// upper half with the lower half), so with both operands = v each lane ends
// up holding its own value and its partner row's: VALU only, no LDS round
// trip as with a bpermute.  Sums add (r0 + r1) + (r2 + r3) in every lane.
__device__ __forceinline__ float rows4_max(float v) {
  const unsigned u = __float_as_uint(v);
  auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
  const unsigned u2 = __float_as_uint(v);
  auto t = __builtin_amdgcn_permlane32_swap(u2, u2, false, false);
  return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float rows4_sum(float v) {
  const unsigned u = __float_as_uint(v);
  auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  const unsigned u2 = __float_as_uint(v);
  auto t = __builtin_amdgcn_permlane32_swap(u2, u2, false, false);
  return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

template <int DH>
struct Geo {
  static constexpr int NC = (DH + 15) / 16;  // 16-wide chunks of the head dim
  static constexpr int LDT = NC * 16 + 4;    // padded LDS row stride (floats)
  static constexpr int TILE = TQ * LDT;
  static constexpr int F4 = TQ * DH / 4;     // float4 per [64 × DH] tile
  static constexpr int NV = (F4 + 255) / 256;
  // Does a float4 at head-dim offset `d` hold real data?
  __device__ static __forceinline__ bool live(int d) { return DH % 16 == 0 || d < DH; }
};

// A [64 rows × DH] fp32 tile (rows r0.., zero-filled at r >= T) copied from a
// row-major source with row stride ld into registers, then into LDS.  LDS
// columns past DH (DH = 8) are zero-filled once by zero_pad_cols.
template <int DH>
struct TileRegs {
  using G = Geo<DH>;
  floatx4 v[G::NV];
  int r0 = 0, T = 0;  // of the last load: rows r0 + r ≥ T are stored as zeros
  // Branch-free, and nothing consumes the loaded values before store(): a
  // row past T is read from row T − 1 (in range) and zeroed only when stored,
  // so the loads stay in flight under whatever runs in between.
  __device__ __forceinline__ void load(const float* __restrict__ base, int ld, int r0_, int T_,
                                       int tid) {
    r0 = r0_;
    T = T_;
#pragma unroll
    for (int i = 0; i < G::NV; ++i) {
      const int f = tid + i * 256;
      const int r = f / (DH / 4), c = (f % (DH / 4)) * 4;
      if (G::F4 % 256 == 0 || f < G::F4)
        v[i] = *reinterpret_cast<const floatx4*>(base + (size_t)min(r0 + r, T - 1) * ld + c);
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ s, int tid) const {
#pragma unroll
    for (int i = 0; i < G::NV; ++i) {
      const int f = tid + i * 256;
      const int r = f / (DH / 4), c = (f % (DH / 4)) * 4;
      if (G::F4 % 256 == 0 || f < G::F4) {
        const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<floatx4*>(s + r * G::LDT + c) = r0 + r < T ? v[i] : zero;
      }
    }
  }
};

template <int DH>
__device__ __forceinline__ void zero_pad_cols(float* s, int tid) {
  using G = Geo<DH>;
  if (DH % 16 != 0) {
    for (int i = tid; i < TQ * (G::NC * 16 - DH); i += 256) {
      const int r = i / (G::NC * 16 - DH), c = DH + i % (G::NC * 16 - DH);
      s[r * G::LDT + c] = 0.f;
    }
  }
}

// This lane's operand values of a 16-row slab:
// f[c][s] = X[row][16c + 4·(lane/16) + s]  (zero past DH or at row >= T).
template <int DH>
__device__ __forceinline__ void load_rows_frag(floatx4* f, const float* __restrict__ base, int ld,
                                               int row, int T, int g) {
#pragma unroll
  for (int c = 0; c < Geo<DH>::NC; ++c) {
    floatx4 x = {0.f, 0.f, 0.f, 0.f};
    if (row < T && Geo<DH>::live(16 * c + 4 * g))
      x = *reinterpret_cast<const floatx4*>(base + (size_t)row * ld + 16 * c + 4 * g);
    f[c] = x;
  }
}

// ---------------------------------------------------------------- forward
// One 64-key tile of the online softmax for this lane's query row.  qf holds
// Q pre-multiplied by scale·log2(e), so scores are already in the log2
// domain.  Only the diagonal tile (DIAG) needs the causal mask: every key of
// an earlier tile precedes every query of this block.  On the diagonal tile
// key sub-tiles j > w lie entirely in the future and are skipped.
template <int DH, bool DIAG>
__device__ __forceinline__ void fwd_tile(const float* __restrict__ Ks, const float* __restrict__ Vs,
                                         const floatx4* qf, floatx4* acc_o, float& m, float& l,
                                         int w, int g, int l16) {
  using G = Geo<DH>;
  constexpr int NC = G::NC, LDT = G::LDT;
  const int jmax = DIAG ? w : 3;
  floatx4 st[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    st[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (j <= jmax) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const floatx4 kf = *reinterpret_cast<const floatx4*>(Ks + (16 * j + l16) * LDT + 16 * c + 4 * g);
#pragma unroll
        for (int s = 0; s < 4; ++s) st[j] = mfma16x16x4(kf[s], qf[c][s], st[j]);
      }
    }
  }
  // st[j][e] = S[qrow][k0 + 16j + 4g + e]; on the diagonal tile the key is
  // in the future when 16j + 4g + e > 16w + l16.
  if (DIAG) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (j > jmax || 16 * j + 4 * g + e > 16 * w + l16) st[j][e] = -INFINITY;
  }
  float mx = fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3]));
#pragma unroll
  for (int j = 1; j < 4; ++j) mx = fmaxf(mx, fmaxf(fmaxf(st[j][0], st[j][1]), fmaxf(st[j][2], st[j][3])));
  mx = rows4_max(mx);
  const float m_new = fmaxf(m, mx);
  const float alpha = __builtin_amdgcn_exp2f(m - m_new);
  m = m_new;
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __builtin_amdgcn_exp2f(st[j][e] - m_new);
      st[j][e] = p;
      ps += p;
    }
  l = l * alpha + ps;
#pragma unroll
  for (int d = 0; d < NC; ++d) acc_o[d] *= alpha;
  // Oᵀ[d][q] += Vᵀ[d][key] · Pᵀ[key][q]
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j <= jmax) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float* vr = Vs + (16 * j + 4 * g + s) * LDT + l16;
#pragma unroll
        for (int d = 0; d < NC; ++d) acc_o[d] = mfma16x16x4(vr[16 * d], st[j][s], acc_o[d]);
      }
    }
  }
}

// One block = 64 query rows of one (batch, head); one LDS stage for the K
// and V tiles, the next tile prefetched into registers during the MFMAs.
template <int DH>
__global__ void __launch_bounds__(256) mha_fwd_kernel(AttnArgs a) {
  using G = Geo<DH>;
  constexpr int NC = G::NC;
  __shared__ __attribute__((aligned(16))) float sm[2][G::TILE];  // [K,V]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int nqt = (a.T + TQ - 1) / TQ;
  // grid (H, B, tiles): the tile index varies slowest, so every (head,
  // sequence)'s longest query tile is dispatched before any shorter one —
  // longest-first over the whole launch, not just within a head.
  const int qt = nqt - 1 - blockIdx.z;
  const int h = blockIdx.x, b = blockIdx.y;
  const int q0 = qt * TQ;
  const size_t row_base = (size_t)b * a.T;
  const float* Qb = a.q + row_base * a.ld_qkv + h * DH;
  const float* Kb = a.k + row_base * a.ld_qkv + h * DH;
  const float* Vb = a.v + row_base * a.ld_qkv + h * DH;

  const int qrow = q0 + 16 * w + l16;  // this lane's query row (Sᵀ column)
  floatx4 qf[NC];
  load_rows_frag<DH>(qf, Qb, a.ld_qkv, qrow, a.T, g);
  const float sl2 = a.scale * LOG2E;
#pragma unroll
  for (int c = 0; c < NC; ++c) qf[c] *= sl2;

  float m = -INFINITY, l = 0.f;
  floatx4 acc_o[NC];
#pragma unroll
  for (int d = 0; d < NC; ++d) acc_o[d] = floatx4{0.f, 0.f, 0.f, 0.f};

  zero_pad_cols<DH>(sm[0], tid);
  zero_pad_cols<DH>(sm[1], tid);
  TileRegs<DH> rk, rv;
  rk.load(Kb, a.ld_qkv, 0, a.T, tid);
  rv.load(Vb, a.ld_qkv, 0, a.T, tid);
  rk.store(sm[0], tid);
  rv.store(sm[1], tid);
  __syncthreads();

  for (int kt = 0; kt < qt; ++kt) {
    rk.load(Kb, a.ld_qkv, (kt + 1) * TQ, a.T, tid);
    rv.load(Vb, a.ld_qkv, (kt + 1) * TQ, a.T, tid);
    fwd_tile<DH, false>(sm[0], sm[1], qf, acc_o, m, l, w, g, l16);
    __syncthreads();  // every wave is done with the stage
    rk.store(sm[0], tid);
    rv.store(sm[1], tid);
    __syncthreads();
  }
  fwd_tile<DH, true>(sm[0], sm[1], qf, acc_o, m, l, w, g, l16);

  l = rows4_sum(l);
  if (qrow < a.T) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    float* orow = a.out + (row_base + qrow) * a.ld_o + h * DH;
#pragma unroll
    for (int d = 0; d < NC; ++d)
      if (G::live(16 * d + 4 * g))
        *reinterpret_cast<floatx4*>(orow + 16 * d + 4 * g) = acc_o[d] * inv;
    if (g == 0) a.lse[((size_t)b * a.H + h) * a.T + qrow] = (m + __log2f(l)) * (1.f / LOG2E);
  }
}

// Direct-load forward (d_head = 64): K and V tiles go from memory straight
// into LDS with global_load_lds_dwordx4 (a wave instruction fills 1 KB = four
// 64-float rows): no staging registers and no ds_write.  One LDS stage
// (32 KB), so that as many blocks share a CU as with the register-staged
// kernel; a block's next-tile load latency is covered by the other blocks
// (loading K and V half a tile apart, each behind the other half's compute,
// measured no faster on MI355X at C2: 0.147 ms both).
// The rows are unpadded.  K fragments are b128 reads of 16 consecutive rows
// at one granule, kept conflict-free by an XOR swizzle of the 16-byte
// granules (granule q of row r at q ^ (r & 15)); V fragments are b128 reads
// in which each group of 16 lanes reads one whole row, conflict-free as laid
// out.
// Rows past T are loaded from row T − 1 (finite, and masked: a key ≥ T is
// always in the future of every query < T).
template <bool ISK>
__device__ __forceinline__ int attn_swz(int row, int q) {
  return ISK ? q ^ (row & 15) : q;
}

template <bool ISK>
__device__ __forceinline__ void issue_kv64(const float* __restrict__ base, int ld, int r0, int T, float* lds,
                                           int w, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int L0 = 4 * (4 * w + j);  // first of the four rows of this instruction
    const int row = L0 + (lane >> 4);
    const int q = attn_swz<ISK>(row, lane & 15);
    const int grow = min(r0 + row, T - 1);
    __builtin_amdgcn_global_load_lds(base + (size_t)grow * ld + 4 * q,
                                     (__attribute__((address_space(3))) void*)(lds + L0 * 64), 16, 0, 0);
  }
}

// Sᵀ of one 64-key tile against the wave's 16 queries (K from LDS).
template <bool DIAG>
__device__ __forceinline__ void fwd_scores_direct(const float* __restrict__ Ks, const floatx4* qf, floatx4* st,
                                                  int w, int g, int l16) {
  constexpr int NC = 4;
  const int jmax = DIAG ? w : 3;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    st[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (j <= jmax) {
      const int row = 16 * j + l16;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const floatx4 kf = *reinterpret_cast<const floatx4*>(Ks + row * 64 + 4 * attn_swz<true>(row, 4 * c + g));
#pragma unroll
        for (int s = 0; s < 4; ++s) st[j] = mfma16x16x4(kf[s], qf[c][s], st[j]);
      }
    }
  }
  if (DIAG) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (j > jmax || 16 * j + 4 * g + e > 16 * w + l16) st[j][e] = -INFINITY;
  }
}

// Online softmax of the tile's scores, then O += P·V (V from LDS).
template <bool DIAG>
__device__ __forceinline__ void fwd_pv_direct(const float* __restrict__ Vs, floatx4* st, floatx4* acc_o, float& m,
                                              float& l, int w, int g, int l16) {
  constexpr int NC = 4;
  const int jmax = DIAG ? w : 3;
  float mx = fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3]));
#pragma unroll
  for (int j = 1; j < 4; ++j) mx = fmaxf(mx, fmaxf(fmaxf(st[j][0], st[j][1]), fmaxf(st[j][2], st[j][3])));
  mx = rows4_max(mx);
  const float m_new = fmaxf(m, mx);
  const float alpha = __builtin_amdgcn_exp2f(m - m_new);
  m = m_new;
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __builtin_amdgcn_exp2f(st[j][e] - m_new);
      st[j][e] = p;
      ps += p;
    }
  l = l * alpha + ps;
#pragma unroll
  for (int d = 0; d < NC; ++d) acc_o[d] *= alpha;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j <= jmax) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        // Oᵀ tile d holds the columns 4·r + d (r = 0..15): one b128 read of
        // V[key][4·l16 .. 4·l16 + 3] feeds the four tiles.
        const int key = 16 * j + 4 * g + s;
        const floatx4 v = *reinterpret_cast<const floatx4*>(Vs + key * 64 + 4 * attn_swz<false>(key, l16));
#pragma unroll
        for (int d = 0; d < NC; ++d) acc_o[d] = mfma16x16x4(v[d], st[j][s], acc_o[d]);
      }
    }
  }
}

__global__ void __launch_bounds__(256, 4) mha_fwd_direct_kernel(AttnArgs a) {
  constexpr int DH = 64, NC = 4, TILE = 64 * 64;
  __shared__ __attribute__((aligned(1024))) float sm[2][TILE];  // [K, V]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int nqt = (a.T + TQ - 1) / TQ;
  const int qt = nqt - 1 - blockIdx.z;  // longest query tiles first over the whole launch
  const int h = blockIdx.x, b = blockIdx.y;
  const int q0 = qt * TQ;
  const size_t row_base = (size_t)b * a.T;
  const float* Qb = a.q + row_base * a.ld_qkv + h * DH;
  const float* Kb = a.k + row_base * a.ld_qkv + h * DH;
  const float* Vb = a.v + row_base * a.ld_qkv + h * DH;

  issue_kv64<true>(Kb, a.ld_qkv, 0, a.T, sm[0], w, lane);
  issue_kv64<false>(Vb, a.ld_qkv, 0, a.T, sm[1], w, lane);
  const int qrow = q0 + 16 * w + l16;
  floatx4 qf[NC];
  load_rows_frag<DH>(qf, Qb, a.ld_qkv, qrow, a.T, g);
  const float sl2 = a.scale * LOG2E;
#pragma unroll
  for (int c = 0; c < NC; ++c) qf[c] *= sl2;
  float m = -INFINITY, l = 0.f;
  floatx4 acc_o[NC];
#pragma unroll
  for (int d = 0; d < NC; ++d) acc_o[d] = floatx4{0.f, 0.f, 0.f, 0.f};
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  floatx4 st[4];
  for (int kt = 0; kt < qt; ++kt) {
    fwd_scores_direct<false>(sm[0], qf, st, w, g, l16);
    fwd_pv_direct<false>(sm[1], st, acc_o, m, l, w, g, l16);
    __syncthreads();  // every wave is done with the stage
    issue_kv64<true>(Kb, a.ld_qkv, (kt + 1) * TQ, a.T, sm[0], w, lane);
    issue_kv64<false>(Vb, a.ld_qkv, (kt + 1) * TQ, a.T, sm[1], w, lane);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  fwd_scores_direct<true>(sm[0], qf, st, w, g, l16);
  fwd_pv_direct<true>(sm[1], st, acc_o, m, l, w, g, l16);
  l = rows4_sum(l);
  if (qrow < a.T) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    float* orow = a.out + (row_base + qrow) * a.ld_o + h * DH;
    // acc_o[d][i] is O[qrow][16·g + 4·i + d]
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<floatx4*>(orow + 16 * g + 4 * i) =
          floatx4{acc_o[0][i], acc_o[1][i], acc_o[2][i], acc_o[3][i]} * inv;
    if (g == 0) a.lse[((size_t)b * a.H + h) * a.T + qrow] = (m + __log2f(l)) * (1.f / LOG2E);
  }
}

// Layout of one 64×64 dS tile in the workspace: four 16-key blocks of 1024
// floats (key block kb = key / 16 at kb·1024), each holding 64 query slots of
// 16 keys (64 bytes).  Query q of sub-tile q / 16 sits in slot 16·(q / 16) +
// slot_of(q % 16), slot_of(4g + e) = 2e + 8·(g / 2) + g % 2: the four rows
// 4g + e (g = 0..3) a wave's accumulator register e holds go to slots 2e,
// 2e + 1, 2e + 8, 2e + 9, so each store instruction of pass 2 writes two
// whole 128-byte lines, and a pass-3 wave's 16 query rows of one key block
// are one contiguous KB.
__device__ __forceinline__ int ds_slot(int r16) {  // r16 = q % 16
  return 2 * (r16 & 3) + 8 * (r16 >> 3) + ((r16 >> 2) & 1);
}

// ------------------------------------------------- backward pass 1: rowdot
// D[b,h,i] = Σ_c dO[i,c]·O[i,c]  (= Σ_j P_ij dP_ij of the reference's fused
// dscores pass, src/gpu/attention.rs:163-247).  One lane per float4 of the
// row, in groups of the next power of two ≥ DH/4 (the surplus lanes add 0).
constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }

template <int DH>
__global__ void __launch_bounds__(256) mha_bwd_rowdot_kernel(AttnArgs a, int B) {
  constexpr int LPR = pow2_at_least(DH / 4);  // lanes per row
  constexpr int RPB = 256 / LPR;              // rows per block
  const int gid = blockIdx.x * RPB + threadIdx.x / LPR;  // (b, t, h) flattened
  const int part = threadIdx.x % LPR;
  const int total = B * a.T * a.H;
  float s = 0.f;
  int h = 0, bt = 0;
  if (gid < total && part < DH / 4) {
    h = gid % a.H;
    bt = gid / a.H;
    const floatx4 o = *reinterpret_cast<const floatx4*>(a.o + (size_t)bt * a.ld_o + h * DH + 4 * part);
    const floatx4 d = *reinterpret_cast<const floatx4*>(a.dO + (size_t)bt * a.ld_o + h * DH + 4 * part);
    s = o[0] * d[0] + o[1] * d[1] + o[2] * d[2] + o[3] * d[3];
  }
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) s += shfl_xor(s, m);
  if (gid < total && part == 0) {
    h = gid % a.H;
    bt = gid / a.H;
    const int b = bt / a.T, t = bt % a.T;
    a.D[((size_t)b * a.H + h) * a.T + t] = s;
  }
}

// ---------------------------------------- backward pass 2: dK, dV (and dS)
// NS: LDS stages for the Q / dO tiles (staged through registers).  NS = 1 is
// compiled for three waves per SIMD and is the default (measured on MI355X at
// C2: backward 0.431 ms against 0.449 ms for the two-stage ring, which leaves
// two waves per SIMD).
template <int DH, int NS>
__global__ void __launch_bounds__(256, (NS == 1 ? 3 : 1)) mha_bwd_dkv_kernel(AttnArgs a) {
  using G = Geo<DH>;
  constexpr int NC = G::NC, LDT = G::LDT;
  __shared__ __attribute__((aligned(16))) float sm[NS][2][G::TILE];  // [stage][Q,dO]
  __shared__ __attribute__((aligned(16))) float st_lse[NS][TQ];
  __shared__ __attribute__((aligned(16))) float st_D[NS][TQ];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int nqt = (a.T + TQ - 1) / TQ;
  const int kt = blockIdx.z;  // key tile 0 has the most work: dispatched first (grid H, B, tiles)
  const int h = blockIdx.x, b = blockIdx.y;
  const int k0 = kt * TQ;
  const size_t row_base = (size_t)b * a.T;
  const float* Qb = a.q + row_base * a.ld_qkv + h * DH;
  const float* Kb = a.k + row_base * a.ld_qkv + h * DH;
  const float* Vb = a.v + row_base * a.ld_qkv + h * DH;
  const float* dOb = a.dO + row_base * a.ld_o + h * DH;
  const size_t stat = ((size_t)b * a.H + h) * a.T;

  const int krow = k0 + 16 * w + l16;  // this lane's key (column of S)
  floatx4 kf[NC], vf[NC];
  load_rows_frag<DH>(kf, Kb, a.ld_qkv, krow, a.T, g);
  load_rows_frag<DH>(vf, Vb, a.ld_qkv, krow, a.T, g);
  // K pre-multiplied by scale·log2(e): S comes out in the log2 domain.  dK
  // is accumulated from the unscaled dS and scaled once at the end.
  const float sl2 = a.scale * LOG2E;
#pragma unroll
  for (int c = 0; c < NC; ++c) kf[c] *= sl2;

  floatx4 acc_k[NC], acc_v[NC];
#pragma unroll
  for (int d = 0; d < NC; ++d) {
    acc_k[d] = floatx4{0.f, 0.f, 0.f, 0.f};
    acc_v[d] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  for (int st = 0; st < NS; ++st) {
    zero_pad_cols<DH>(sm[st][0], tid);
    zero_pad_cols<DH>(sm[st][1], tid);
  }
  TileRegs<DH> rq, rd;
  // The next tile's row statistics, raw: scaled and masked only when stored,
  // so no wait for them (and, the load counter being in order, for the
  // tile loads before them) at the top of the tile.
  float r_lse = 0.f, r_D = 0.f;
  int r_q = 0;
  auto load_stats = [&](int q0) {
    if (tid < TQ) {
      r_q = q0 + tid;
      const int qc = min(r_q, a.T - 1);
      r_lse = a.lse[stat + qc];
      r_D = a.D[stat + qc];
    }
  };
  rq.load(Qb, a.ld_qkv, k0, a.T, tid);
  rd.load(dOb, a.ld_o, k0, a.T, tid);
  load_stats(k0);
  rq.store(sm[0][0], tid);
  rd.store(sm[0][1], tid);
  if (tid < TQ) {
    st_lse[0][tid] = r_q < a.T ? r_lse * LOG2E : 0.f;
    st_D[0][tid] = r_q < a.T ? r_D : 0.f;
  }
  __syncthreads();

  for (int qt = kt; qt < nqt; ++qt) {
    const int cur = NS == 2 ? ((qt - kt) & 1) : 0;
    const bool more = qt + 1 < nqt;
    if (more) {
      rq.load(Qb, a.ld_qkv, (qt + 1) * TQ, a.T, tid);
      rd.load(dOb, a.ld_o, (qt + 1) * TQ, a.T, tid);
      load_stats((qt + 1) * TQ);
    }
    const float* Qs = sm[cur][0];
    const float* dOs = sm[cur][1];
    const int q0 = qt * TQ;
    float* ds_tile = a.ds + (((size_t)b * a.H + h) * a.ntri + qt * (qt + 1) / 2 + kt) * (TQ * TQ);
    // Query sub-tiles jq < w of the diagonal tile lie entirely before this
    // wave's keys: fully masked.
    const int jmin = (qt == kt) ? w : 0;
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      if (jq < jmin) continue;
      floatx4 s_ = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const floatx4 qv = *reinterpret_cast<const floatx4*>(Qs + (16 * jq + l16) * LDT + 16 * c + 4 * g);
        const floatx4 dv_ = *reinterpret_cast<const floatx4*>(dOs + (16 * jq + l16) * LDT + 16 * c + 4 * g);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          s_ = mfma16x16x4(qv[s], kf[c][s], s_);   // S[q][key]
          dp = mfma16x16x4(dv_[s], vf[c][s], dp);  // dP[q][key]
        }
      }
      const floatx4 lq = *reinterpret_cast<const floatx4*>(&st_lse[cur][16 * jq + 4 * g]);
      const floatx4 Dq = *reinterpret_cast<const floatx4*>(&st_D[cur][16 * jq + 4 * g]);
      floatx4 p, ds;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int q = q0 + 16 * jq + 4 * g + e;
        float pe = __builtin_amdgcn_exp2f(s_[e] - lq[e]);
        if (qt == kt && krow > q) pe = 0.f;
        p[e] = pe;
        ds[e] = pe * (dp[e] - Dq[e]);
        // dS tile (qt, kt) for the dQ pass, in the ds_slot layout (this
        // wave's key block; row 4g + e in slot ds_slot(4g + e)).  Streamed
        // (non-temporal): it is read back only after the whole pass, and
        // keeping it out of L2 leaves room for the Q / dO tiles this block
        // and its neighbours re-read.
        __builtin_nontemporal_store(
            ds[e], &ds_tile[w * (16 * TQ) + (16 * jq + 2 * e + 8 * (g >> 1) + (g & 1)) * 16 + l16]);
      }
      // dVᵀ[d][key] += dOᵀ[d][q]·P[q][key];  dKᵀ[d][key] += Qᵀ[d][q]·dS[q][key]
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float* dor = dOs + (16 * jq + 4 * g + s) * LDT + l16;
        const float* qr = Qs + (16 * jq + 4 * g + s) * LDT + l16;
#pragma unroll
        for (int d = 0; d < NC; ++d) {
          acc_v[d] = mfma16x16x4(dor[16 * d], p[s], acc_v[d]);
          acc_k[d] = mfma16x16x4(qr[16 * d], ds[s], acc_k[d]);
        }
      }
    }
    if (more) {
      if (NS == 1) __syncthreads();  // every wave is done with the only stage
      rq.store(sm[(cur + 1) % NS][0], tid);
      rd.store(sm[(cur + 1) % NS][1], tid);
      if (tid < TQ) {
        st_lse[(cur + 1) % NS][tid] = r_q < a.T ? r_lse * LOG2E : 0.f;
        st_D[(cur + 1) % NS][tid] = r_q < a.T ? r_D : 0.f;
      }
    }
    __syncthreads();
  }
  if (krow < a.T) {
    float* dkr = a.dk + (row_base + krow) * a.ld_d + h * DH;
    float* dvr = a.dv + (row_base + krow) * a.ld_d + h * DH;
#pragma unroll
    for (int d = 0; d < NC; ++d) {
      if (!G::live(16 * d + 4 * g)) continue;
      floatx4* pk = reinterpret_cast<floatx4*>(dkr + 16 * d + 4 * g);
      floatx4* pv = reinterpret_cast<floatx4*>(dvr + 16 * d + 4 * g);
      *pk = a.overwrite ? acc_k[d] * a.scale : *pk + acc_k[d] * a.scale;
      *pv = a.overwrite ? acc_v[d] : *pv + acc_v[d];
    }
  }
}

// ---------------------------------------------------- backward pass 3: dQ
// dQ[q] = scale · Σ_key dS[q][key] K[key] over the key tiles 0..qt of this
// query tile, in increasing key order, from the dS tiles pass 2 stored.  A
// wave owns 16 query rows; lane l reads dS[16w + l%16][16j + 4·(l/16) .. +3]
// (one float4 per 16-key block j, from the row's ds_slot), which is exactly the B operand of
// dQᵀ[d][q] += Kᵀ[d][key]·dSᵀ[key][q] in the Sᵀ layout of the other passes.
// K tiles go through LDS double-buffered, the next tile's dS fragments are
// loaded into registers while the current ones are multiplied.  On the
// diagonal tile only sub-tiles j ≤ w hold keys at or before this wave's
// queries (pass 2 wrote them, zero where masked); the others are skipped.
template <int DH>
__global__ void __launch_bounds__(256) mha_bwd_dq_kernel(AttnArgs a) {
  using G = Geo<DH>;
  constexpr int NC = G::NC, LDT = G::LDT;
  __shared__ __attribute__((aligned(16))) float sm[2][G::TILE];  // K tiles
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int nqt = (a.T + TQ - 1) / TQ;
  const int qt = nqt - 1 - blockIdx.z;  // longest query tiles first (grid H, B, tiles)
  const int h = blockIdx.x, b = blockIdx.y;
  const size_t row_base = (size_t)b * a.T;
  const float* Kb = a.k + row_base * a.ld_qkv + h * DH;
  // dS tile (qt, kt) at tiles + kt·TQ², this lane's row slot and keys folded in
  const float* tiles = a.ds + (((size_t)b * a.H + h) * a.ntri + qt * (qt + 1) / 2) * (TQ * TQ) +
                       (16 * w + ds_slot(l16)) * 16 + 4 * g;
  auto load_ds = [&](int kt, floatx4* f) {  // read once: streamed past L2
#pragma unroll
    for (int j = 0; j < 4; ++j)
      f[j] = __builtin_nontemporal_load(
          reinterpret_cast<const floatx4*>(tiles + (size_t)kt * (TQ * TQ) + j * (16 * TQ)));
  };

  floatx4 acc[NC];
#pragma unroll
  for (int d = 0; d < NC; ++d) acc[d] = floatx4{0.f, 0.f, 0.f, 0.f};
  zero_pad_cols<DH>(sm[0], tid);
  zero_pad_cols<DH>(sm[1], tid);
  TileRegs<DH> rk;
  floatx4 fc[4], fn[4];
  rk.load(Kb, a.ld_qkv, 0, a.T, tid);
  load_ds(0, fc);
  rk.store(sm[0], tid);
  __syncthreads();
  for (int kt = 0; kt <= qt; ++kt) {
    const bool more = kt < qt;
    if (more) {
      rk.load(Kb, a.ld_qkv, (kt + 1) * TQ, a.T, tid);
      load_ds(kt + 1, fn);
    }
    const float* Ks = sm[kt & 1];
    const int jmax = more ? 3 : w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j > jmax) continue;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float* kr = Ks + (16 * j + 4 * g + s) * LDT + l16;
#pragma unroll
        for (int d = 0; d < NC; ++d) acc[d] = mfma16x16x4(kr[16 * d], fc[j][s], acc[d]);
      }
    }
    if (more) {
      // the other buffer was last read in iteration kt-1, before the barrier
      rk.store(sm[(kt + 1) & 1], tid);
#pragma unroll
      for (int j = 0; j < 4; ++j) fc[j] = fn[j];
      __syncthreads();
    }
  }
  const int qrow = qt * TQ + 16 * w + l16;
  if (qrow < a.T) {
    float* dqr = a.dq + (row_base + qrow) * a.ld_d + h * DH;
#pragma unroll
    for (int d = 0; d < NC; ++d) {
      if (!G::live(16 * d + 4 * g)) continue;
      floatx4* p = reinterpret_cast<floatx4*>(dqr + 16 * d + 4 * g);
      *p = a.overwrite ? acc[d] * a.scale : *p + acc[d] * a.scale;
    }
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Workspace: rowdot D [B,H,T], padded to 256 bytes, then the dS tiles.
size_t ws_d_floats(size_t b, size_t t, size_t n_head) { return (b * t * n_head + 63) / 64 * 64; }

// Floats of that layout: D plus every 64×64 tile of the causal lower
// triangle, ≈ b·n_head·t²/2 for long sequences.
size_t tiled_ws_floats(size_t b, size_t t, size_t n_head) {
  const size_t nqt = (t + TQ - 1) / TQ;
  return ws_d_floats(b, t, n_head) + b * n_head * (nqt * (nqt + 1) / 2) * TQ * TQ;
}

bool dh_supported(uint32_t d) { return d >= 8 && d <= 64 && d % 8 == 0; }

int check_common(aur_ctx* ctx, uint32_t b, uint32_t t, uint32_t n_head, uint32_t d_head,
                 uint32_t ld_qkv, uint32_t ld_o) {
  if (d_head < 1 || d_head > 64)
    return aur::set_error(ctx, AUR_ELIMIT, "attention: d_head=%u, supported 1..64 (the reference's "
                          "one-thread-per-column backward, src/gpu/attention.rs:266-331)", d_head);
  if (b == 0 || t == 0 || n_head == 0) return aur::set_error(ctx, AUR_EINVAL, "attention: empty shape");
  if (ld_qkv < n_head * d_head || ld_o < n_head * d_head ||
      (dh_supported(d_head) && ((ld_qkv & 3) || (ld_o & 3))))
    return aur::set_error(ctx, AUR_EINVAL, "attention: bad row stride (%u, %u)", ld_qkv, ld_o);
  if (n_head > 65535 || b > 65535 || (t + TQ - 1) / TQ > 65535)
    return aur::set_error(ctx, AUR_ELIMIT, "attention: grid too large");
  return 0;
}

// Direct-load dQ pass (d_head = 64): K tiles go straight into a swizzled,
// double-buffered LDS ring (granule q of row r at q ^ (((r >> 2) & 3) << 2),
// conflict-free for the b32 reads of rows 4g + s × 16 columns), no staging
// registers, one barrier per tile.  K rows past T are loaded from row T − 1: every dS entry
// of a key ≥ T is zero for the queries < T (pass 2 masks them), so they add
// nothing.
__global__ void __launch_bounds__(256, 5) mha_bwd_dq_direct_kernel(AttnArgs a) {
  constexpr int DH = 64, NC = 4;
  __shared__ __attribute__((aligned(1024))) float sm[2][64 * 64];  // K tiles
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int nqt = (a.T + TQ - 1) / TQ;
  const int qt = nqt - 1 - blockIdx.z;  // longest query tiles first (grid H, B, tiles)
  const int h = blockIdx.x, b = blockIdx.y;
  const size_t row_base = (size_t)b * a.T;
  const float* Kb = a.k + row_base * a.ld_qkv + h * DH;
  const float* tiles = a.ds + (((size_t)b * a.H + h) * a.ntri + qt * (qt + 1) / 2) * (TQ * TQ) +
                       (16 * w + ds_slot(l16)) * 16 + 4 * g;
  auto load_ds = [&](int kt, floatx4* f) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // read once: streamed past L2, which keeps the K tiles
      f[j] = __builtin_nontemporal_load(
          reinterpret_cast<const floatx4*>(tiles + (size_t)kt * (TQ * TQ) + j * (16 * TQ)));
    }
  };
  auto issue_k = [&](int kt, float* lds) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int L0 = 4 * (4 * w + j);
      const int row = L0 + (lane >> 4);
      const int q = (lane & 15) ^ (((row >> 2) & 3) << 2);
      const int grow = min(kt * TQ + row, a.T - 1);
      __builtin_amdgcn_global_load_lds(Kb + (size_t)grow * a.ld_qkv + 4 * q,
                                       (__attribute__((address_space(3))) void*)(lds + L0 * 64), 16, 0, 0);
    }
  };
  floatx4 acc[NC];
#pragma unroll
  for (int d = 0; d < NC; ++d) acc[d] = floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 fc[4], fn[4];
  issue_k(0, sm[0]);
  load_ds(0, fc);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // acc += dS(tile)·K(tile) over this wave's sub-tiles j ≤ jmax
  auto tile_mfma = [&](const float* Ks, int jmax) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j > jmax) continue;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int r = 16 * j + 4 * g + s;
#pragma unroll
        for (int d = 0; d < NC; ++d) {
          const int col = 16 * d + l16;
          acc[d] = mfma16x16x4(Ks[r * 64 + 4 * ((col >> 2) ^ (((r >> 2) & 3) << 2)) + (col & 3)], fc[j][s], acc[d]);
        }
      }
    }
  };
  // Key tiles below the diagonal: a branch-free body, in which the next
  // tile's 8 loads (4 K granule rows straight into LDS, 4 dS fragments) are
  // spread among the first MFMAs and the K fragment reads (one b32 per MFMA)
  // run two ahead of their MFMAs (sched_group_barrier classes: 0x008 MFMA,
  // 0x020 VMEM read, 0x100 DS read).  Measured on MI355X at C2: backward
  // 0.406-0.408 → 0.400-0.402 ms against the compiler's own schedule.
  for (int kt = 0; kt < qt; ++kt) {
    // the other buffer was released by the previous barrier
    issue_k(kt + 1, sm[(kt + 1) & 1]);
    load_ds(kt + 1, fn);
    tile_mfma(sm[kt & 1], 3);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
#pragma unroll
    for (int r = 0; r < 24; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) fc[j] = fn[j];
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  tile_mfma(sm[qt & 1], w);  // the diagonal tile: sub-tiles j ≤ w
  const int qrow = qt * TQ + 16 * w + l16;
  if (qrow < a.T) {
    float* dqr = a.dq + (row_base + qrow) * a.ld_d + h * DH;
#pragma unroll
    for (int d = 0; d < NC; ++d) {
      floatx4* pq = reinterpret_cast<floatx4*>(dqr + 16 * d + 4 * g);
      *pq = a.overwrite ? acc[d] * a.scale : *pq + acc[d] * a.scale;
    }
  }
}

// d_head that is not a multiple of 8 (any 1..64, as the reference's
// kernels take): the heads are copied into a layout whose heads are padded
// with zero columns to the next multiple of 8 — zero columns add nothing to
// a score, an output row or a gradient — the kernels run at that width with
// the true scale 1/sqrt(d_head), and the results are copied back.
__global__ void __launch_bounds__(256) pad_heads_kernel(const float* __restrict__ src, int ld, int H, int dh,
                                                        int dhp, float* __restrict__ dst, size_t rows) {
  const size_t n = rows * H * dhp;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % dhp);
    const size_t rh = i / dhp;
    const int h = (int)(rh % H);
    const size_t r = rh / H;
    dst[i] = c < dh ? src[r * ld + (size_t)h * dh + c] : 0.f;
  }
}

__global__ void __launch_bounds__(256) unpad_heads_kernel(const float* __restrict__ src, int H, int dh, int dhp,
                                                          float* __restrict__ dst, int ld, size_t rows,
                                                          int accumulate) {
  const size_t n = rows * H * dh;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % dh);
    const size_t rh = i / dh;
    const int h = (int)(rh % H);
    const size_t r = rh / H;
    const float v = src[(r * H + h) * dhp + c];
    float* p = dst + r * ld + (size_t)h * dh + c;
    *p = accumulate ? *p + v : v;
  }
}

unsigned pad_grid(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 8192); }

template <int DH>
void launch_fwd(const AttnArgs& a, int b, hipStream_t st) {
  dim3 grid(a.H, b, (a.T + TQ - 1) / TQ);
  if constexpr (DH == 64) {
    if (std::getenv("AUR_ATTN_FWD_STAGED") == nullptr) {
      hipLaunchKernelGGL(mha_fwd_direct_kernel, grid, dim3(256), 0, st, a);
      return;
    }
  }
  hipLaunchKernelGGL((mha_fwd_kernel<DH>), grid, dim3(256), 0, st, a);
}

template <int DH>
void launch_bwd(const AttnArgs& a, int b, hipStream_t st) {
  constexpr int RPB = 256 / pow2_at_least(DH / 4);  // rows per block of mha_bwd_rowdot_kernel
  const size_t rows = (size_t)b * a.T * a.H;
  hipLaunchKernelGGL(mha_bwd_rowdot_kernel<DH>, dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256),
                     0, st, a, b);
  dim3 grid(a.H, b, (a.T + TQ - 1) / TQ);
  if (std::getenv("AUR_ATTN_DKV_NS2") == nullptr)
    hipLaunchKernelGGL((mha_bwd_dkv_kernel<DH, 1>), grid, dim3(256), 0, st, a);  // also stores dS
  else
    hipLaunchKernelGGL((mha_bwd_dkv_kernel<DH, 2>), grid, dim3(256), 0, st, a);
  if (DH == 64 && std::getenv("AUR_ATTN_DQ_STAGED") == nullptr)
    hipLaunchKernelGGL(mha_bwd_dq_direct_kernel, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((mha_bwd_dq_kernel<DH>), grid, dim3(256), 0, st, a);
}

}  // namespace

// overwrite = 0: dq/dk/dv += (the C ABI's contract); 1: dq/dk/dv = (callers
// that would otherwise zero them first).
// ws_tiled: the caller's ws holds tiled_ws_floats (the model's own arena).
// Otherwise ws holds only what aur_mha_bwd_ws_bytes promises — at most the
// reference's d_scores_scratch, n_head·t·t floats per sequence — and when the
// tiled layout needs more than that (short or ragged t) D and the tiles go
// to the context's workspace instead (refused while the stream is being
// captured, since that workspace may be reallocated).
// scale_dh: the d_head of the scale 1/sqrt(scale_dh) (the caller's, when the
// heads arrive padded); 0 = d_head.
static int mha_bwd_impl(aur_ctx* ctx, int overwrite, bool ws_tiled, const float* q, const float* k,
                        const float* v, uint32_t ld_qkv, const float* out, const float* d_out, uint32_t ld_out,
                        const float* lse, float* dq, float* dk, float* dv, uint32_t ld_dqkv, float* ws,
                        uint32_t b, uint32_t t, uint32_t n_head, uint32_t d_head, uint32_t scale_dh = 0) {
  AUR_CHECK_CTX(ctx);
  if (int rc = check_common(ctx, b, t, n_head, d_head, ld_qkv, ld_out)) return rc;
  if (ld_dqkv < n_head * d_head || (dh_supported(d_head) && (ld_dqkv & 3)))
    return aur::set_error(ctx, AUR_EINVAL, "mha_bwd: bad gradient row stride %u", ld_dqkv);
  if (!q || !k || !v || !out || !d_out || !lse || !dq || !dk || !dv || !ws)
    return aur::set_error(ctx, AUR_EINVAL, "mha_bwd: null pointer");
  if (!dh_supported(d_head)) {
    // padded heads (see pad_heads_kernel): q, k, v, o, dO and the three
    // gradients at width dhp, then the tiled workspace, in the context's
    // workspace; the kernels store the padded gradients, which are then
    // added to (or stored into) the caller's
    const uint32_t dhp = (d_head + 7) / 8 * 8;
    const size_t rows = (size_t)b * t, n = rows * n_head * dhp;
    if (int rc = aur::ensure_workspace(ctx, (8 * n + tiled_ws_floats(b, t, n_head)) * sizeof(float))) return rc;
    float* P = static_cast<float*>(ctx->ws);
    const float* srcs[5] = {q, k, v, out, d_out};
    const uint32_t lds[5] = {ld_qkv, ld_qkv, ld_qkv, ld_out, ld_out};
    for (int i = 0; i < 5; ++i)
      hipLaunchKernelGGL(pad_heads_kernel, dim3(pad_grid(n)), dim3(256), 0, ctx->stream, srcs[i], (int)lds[i],
                         (int)n_head, (int)d_head, (int)dhp, P + i * n, rows);
    AUR_LAUNCH_CHECK(ctx, "pad_heads_kernel");
    const uint32_t ldp = n_head * dhp;
    if (int rc = mha_bwd_impl(ctx, 1, true, P, P + n, P + 2 * n, ldp, P + 3 * n, P + 4 * n, ldp, lse, P + 5 * n,
                              P + 6 * n, P + 7 * n, ldp, P + 8 * n, b, t, n_head, dhp, d_head))
      return rc;
    float* dsts[3] = {dq, dk, dv};
    for (int i = 0; i < 3; ++i)
      hipLaunchKernelGGL(unpad_heads_kernel, dim3(pad_grid(rows * n_head * d_head)), dim3(256), 0, ctx->stream,
                         P + (5 + i) * n, (int)n_head, (int)d_head, (int)dhp, dsts[i], (int)ld_dqkv, rows,
                         overwrite ? 0 : 1);
    AUR_LAUNCH_CHECK(ctx, "unpad_heads_kernel");
    return 0;
  }
  if (!al16(q) || !al16(k) || !al16(v) || !al16(out) || !al16(d_out) || !al16(dq) || !al16(dk) ||
      !al16(dv) || !al16(ws))
    return aur::set_error(ctx, AUR_EINVAL, "mha_bwd: tensors must be 16-byte aligned");
  const size_t tiled = tiled_ws_floats(b, t, n_head);
  if (!ws_tiled && tiled > (size_t)b * n_head * t * t) {
    if (int rc = aur::ensure_workspace(ctx, tiled * sizeof(float))) return rc;
    ws = static_cast<float*>(ctx->ws);
  }
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = out; a.dO = d_out; a.lse = const_cast<float*>(lse);
  a.D = ws; a.dq = dq; a.dk = dk; a.dv = dv;
  a.ds = ws + ws_d_floats(b, t, n_head);
  a.overwrite = overwrite;
  a.ntri = (int)(((t + TQ - 1) / TQ) * ((t + TQ - 1) / TQ + 1) / 2);
  a.ld_qkv = (int)ld_qkv; a.ld_o = (int)ld_out; a.ld_d = (int)ld_dqkv;
  a.T = (int)t; a.H = (int)n_head;
  a.scale = 1.0f / sqrtf((float)(scale_dh ? scale_dh : d_head));
  switch (d_head) {
    case 8: launch_bwd<8>(a, (int)b, ctx->stream); break;
    case 16: launch_bwd<16>(a, (int)b, ctx->stream); break;
    case 24: launch_bwd<24>(a, (int)b, ctx->stream); break;
    case 32: launch_bwd<32>(a, (int)b, ctx->stream); break;
    case 40: launch_bwd<40>(a, (int)b, ctx->stream); break;
    case 48: launch_bwd<48>(a, (int)b, ctx->stream); break;
    case 56: launch_bwd<56>(a, (int)b, ctx->stream); break;
    default: launch_bwd<64>(a, (int)b, ctx->stream); break;
  }
  AUR_LAUNCH_CHECK(ctx, "mha_bwd kernels");
  return 0;
}


extern "C" {

int aur_mha_fwd_ex(aur_ctx* ctx, const float* q, const float* k, const float* v, uint32_t ld_qkv,
                   float* out, uint32_t ld_out, float* lse, uint32_t b, uint32_t t,
                   uint32_t n_head, uint32_t d_head) {
  AUR_CHECK_CTX(ctx);
  if (int rc = check_common(ctx, b, t, n_head, d_head, ld_qkv, ld_out)) return rc;
  if (!q || !k || !v || !out || !lse) return aur::set_error(ctx, AUR_EINVAL, "mha_fwd: null pointer");
  uint32_t scale_dh = d_head;
  float* out_p = nullptr;  // padded output to copy back
  const size_t rows = (size_t)b * t;
  const uint32_t d_user = d_head, ld_out_user = ld_out;
  float* out_user = out;
  if (!dh_supported(d_head)) {
    // padded heads (see pad_heads_kernel): q, k, v and the output at width
    // dhp in the context's workspace
    const uint32_t dhp = (d_head + 7) / 8 * 8;
    const size_t n = rows * n_head * dhp;
    if (int rc = aur::ensure_workspace(ctx, 4 * n * sizeof(float))) return rc;
    float* P = static_cast<float*>(ctx->ws);
    const float* srcs[3] = {q, k, v};
    for (int i = 0; i < 3; ++i)
      hipLaunchKernelGGL(pad_heads_kernel, dim3(pad_grid(n)), dim3(256), 0, ctx->stream, srcs[i], (int)ld_qkv,
                         (int)n_head, (int)d_head, (int)dhp, P + i * n, rows);
    AUR_LAUNCH_CHECK(ctx, "pad_heads_kernel");
    q = P; k = P + n; v = P + 2 * n; out = out_p = P + 3 * n;
    ld_qkv = ld_out = n_head * dhp;
    d_head = dhp;
  } else if (!al16(q) || !al16(k) || !al16(v) || !al16(out)) {
    return aur::set_error(ctx, AUR_EINVAL, "mha_fwd: tensors must be 16-byte aligned");
  }
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.out = out; a.lse = lse;
  a.ld_qkv = (int)ld_qkv; a.ld_o = (int)ld_out;
  a.T = (int)t; a.H = (int)n_head;
  a.scale = 1.0f / sqrtf((float)scale_dh);
  switch (d_head) {
    case 8: launch_fwd<8>(a, (int)b, ctx->stream); break;
    case 16: launch_fwd<16>(a, (int)b, ctx->stream); break;
    case 24: launch_fwd<24>(a, (int)b, ctx->stream); break;
    case 32: launch_fwd<32>(a, (int)b, ctx->stream); break;
    case 40: launch_fwd<40>(a, (int)b, ctx->stream); break;
    case 48: launch_fwd<48>(a, (int)b, ctx->stream); break;
    case 56: launch_fwd<56>(a, (int)b, ctx->stream); break;
    default: launch_fwd<64>(a, (int)b, ctx->stream); break;
  }
  AUR_LAUNCH_CHECK(ctx, "mha_fwd_kernel");
  if (out_p) {
    hipLaunchKernelGGL(unpad_heads_kernel, dim3(pad_grid(rows * n_head * d_user)), dim3(256), 0, ctx->stream,
                       out_p, (int)n_head, (int)d_user, (int)d_head, out_user, (int)ld_out_user, rows, 0);
    AUR_LAUNCH_CHECK(ctx, "unpad_heads_kernel");
  }
  return 0;
}

int aur_mha_fwd(aur_ctx* ctx, const float* q, const float* k, const float* v, float* out, float* lse,
                uint32_t b, uint32_t t, uint32_t n_head, uint32_t d_head) {
  return aur_mha_fwd_ex(ctx, q, k, v, n_head * d_head, out, n_head * d_head, lse, b, t, n_head, d_head);
}

size_t aur_mha_bwd_ws_bytes(uint32_t b, uint32_t t, uint32_t n_head) {
  return std::min(tiled_ws_floats(b, t, n_head), (size_t)b * n_head * t * t) * sizeof(float);
}

int aur_mha_bwd_ex(aur_ctx* ctx, const float* q, const float* k, const float* v, uint32_t ld_qkv,
                   const float* out, const float* d_out, uint32_t ld_out, const float* lse, float* dq,
                   float* dk, float* dv, uint32_t ld_dqkv, float* ws, uint32_t b, uint32_t t,
                   uint32_t n_head, uint32_t d_head) {
  return mha_bwd_impl(ctx, 0, false, q, k, v, ld_qkv, out, d_out, ld_out, lse, dq, dk, dv, ld_dqkv, ws, b, t,
                      n_head, d_head);
}

int aur_mha_bwd(aur_ctx* ctx, const float* q, const float* k, const float* v, const float* out,
                const float* lse, const float* d_out, float* dq, float* dk, float* dv, float* ws,
                uint32_t b, uint32_t t, uint32_t n_head, uint32_t d_head) {
  const uint32_t d = n_head * d_head;
  return aur_mha_bwd_ex(ctx, q, k, v, d, out, d_out, d, lse, dq, dk, dv, d, ws, b, t, n_head, d_head);
}

}  // extern "C"

namespace aur {

int mha_bwd_store(aur_ctx* ctx, const float* q, const float* k, const float* v, int ld_qkv, const float* out,
                  const float* d_out, int ld_out, const float* lse, float* dq, float* dk, float* dv, int ld_dqkv,
                  float* ws, int b, int t, int n_head, int d_head) {
  AUR_CHECK_CTX(ctx);
  return mha_bwd_impl(ctx, 1, true, q, k, v, (uint32_t)ld_qkv, out, d_out, (uint32_t)ld_out, lse, dq, dk, dv,
                      (uint32_t)ld_dqkv, ws, (uint32_t)b, (uint32_t)t, (uint32_t)n_head, (uint32_t)d_head);
}

size_t mha_bwd_tiled_ws_floats(int b, int t, int n_head) { return tiled_ws_floats(b, t, n_head); }

}  // namespace aur
