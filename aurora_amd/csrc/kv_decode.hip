// KV-cache decode attention: one new query per (sequence, head) against the
// cached K/V rows [0, t_total).  Reference: MhaKvCacheKernel
// (src/gpu/kv_cache.rs:247-351) and the CPU block_step attention
// (src/transformer/kv_cache.rs:181-219): s_j = q·k_j/sqrt(d_head),
// p = softmax(s), out = Σ_j p_j v_j.
//
// The work is HBM-bound (every cached K and V row is read once per step), so
// the kernel is shaped for memory-level parallelism rather than math:
//   * the key axis is split into chunks of KC keys; one 256-thread block per
//     (chunk, head, sequence) — thousands of blocks at the decode shapes;
//   * d_head/4 lanes cover one K/V row of a head with float4 loads (256
//     contiguous bytes at d_head = 64, 4 keys per wave load instruction),
//     in lane groups of the next power of two (d_head = 24, 40, 48, 56 leave
//     the surplus lanes of a group idle: they read an in-range float4 and
//     contribute zeros);
//   * each block writes its chunk's (row max, row sum, unnormalised output);
//     a second kernel merges the chunks of a (sequence, head) in increasing
//     chunk order — a fixed order, so the result is deterministic.
// When the (sequence, head) pairs alone fill the chip (B·H ≥ CUs, as in
// batched decode), one launch does it all: a block per (sequence, head),
// each wave streams every W-th group of keys with an online softmax, and
// the waves' (max, sum, output) are merged through LDS in wave order.
// That drops the second launch and the blocks for chunks past a
// sequence's end.
#include "common.hpp"
#include "step_ops.hpp"

#include <cstdlib>

namespace {

constexpr int DHMAX = 64;
constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }
constexpr int KC = 128;              // keys per chunk (block)
constexpr int KPW = KC / 4;          // keys per wave
constexpr int PART = 4 + DHMAX;      // per-chunk record: m, l, pad, pad, o[d_head]
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

// Cross-lane exchange without the LDS round trip of a bpermute: the value
// of lane (this lane ^ M), M a power of two ≤ 32.  M = 1, 2 are DPP
// quad_perm moves; M = 16, 32 the row-swap permutes (v_permlane16_swap swaps
// the odd rows of its first operand with the even rows of its second,
// v_permlane32_swap the upper half with the lower half, so with both
// operands = v one result holds this lane's value and the other its
// partner's).  For M = 4, 8 the exact exchange is a bpermute, unless
// UNIFORM: the value is the same on every lane of each aligned group of M
// lanes, and then row_half_mirror (lane ^ 7) and row_mirror (lane ^ 15)
// read a lane holding the partner's value.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int M, bool UNIFORM>
__device__ __forceinline__ float lane_xor(float v) {
  if constexpr (M == 1) {
    return dpp_mov<0xB1>(v);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (M == 2) {
    return dpp_mov<0x4E>(v);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (M == 4 && UNIFORM) {
    return dpp_mov<0x141>(v);  // row_half_mirror
  } else if constexpr (M == 8 && UNIFORM) {
    return dpp_mov<0x140>(v);  // row_mirror
  } else if constexpr (M == 16 || M == 32) {
    const unsigned u = __float_as_uint(v);
    const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float((threadIdx.x & M) ? r[0] : r[1]);
  } else {
    return shfl_xor(v, M);
  }
}
// Σ / max over each aligned group of G lanes, from groups of S lanes whose
// values are uniform (S = 1: none are), as the butterfly v ∘= v(lane ^ M)
// for M = S, 2S, … < G, every lane adding its own value first.
// Σ over lanes l, l ^ S, l ^ 2S, … (the same position in every group of S
// lanes), for values that differ between the lanes of a group.
template <int S>
__device__ __forceinline__ float group_sum_lanes(float v) {
  if constexpr (S < 64) {
    v += lane_xor<S, false>(v);
    return group_sum_lanes<2 * S>(v);
  } else {
    return v;
  }
}
template <int S, int G, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
  if constexpr (S < G) {
    const float o = lane_xor<S, true>(v);
    v = MAX ? fmaxf(v, o) : v + o;
    return group_reduce<2 * S, G, MAX>(v);
  } else {
    return v;
  }
}

struct KvArgs {
  const float* q;       // [B, ld_q] rows, head h at h*d_head
  const float* kh;      // [B, max_len, ld]
  const float* vh;
  float* out;           // [B, ld]
  float* ws;            // [B, H, nch, PART]
  const int32_t* t_dev; // per-sequence lengths (device) or null
  int t_scalar;         // length when t_dev is null
  int ld;               // row stride of the history and out (= n_head * d_head)
  int ld_q;             // row stride of q, knew, vnew (d, or 3d inside a fused qkv row)
  int max_len;
  int H;
  int nch;
  float scale;
  // Fused append (decode step): the newest key/value row (position T-1) is
  // read from knew/vnew instead of the history, and the chunk block that
  // owns it writes it into the history.  Null: the history already has it.
  const float* knew;
  const float* vnew;
  // q, knew and vnew may be K-range partial products of the QKV projection:
  // the value is the sum of nparts (≤ 8) rows pstride floats apart, in order.
  int nparts;
  size_t pstride;
  // Blocks with blockIdx.y >= nseq only prefetch (kv_seq_kernel).
  int nseq;
  aur::L2Prefetch pf;
};

// Prefetch block `slot` of XCD `xcd` loads its share of the row groups
// x ≡ xcd (mod 8) of every matrix of the plan, 16 bytes per lane, with
// ordinary (L2-allocating) loads; the values are only summed so the loads
// are kept.
__device__ void l2_prefetch(const aur::L2Prefetch& pf, int xcd, int slot) {
  float acc = 0.f;
  for (int m = 0; m < pf.nmat; ++m) {
    const int G = pf.group[m];
    const size_t gf4 = (size_t)G * pf.row_floats[m] / 4;  // float4 per row group
    const int ngroups = pf.rows[m] / G;
    const int mine = ngroups > xcd ? (ngroups - xcd + 7) / 8 : 0;  // groups of this XCD
    const size_t total = (size_t)mine * gf4;
    const size_t per = (total + pf.blocks_per_xcd - 1) / pf.blocks_per_xcd;
    const size_t b0 = (size_t)slot * per, b1 = b0 + per < total ? b0 + per : total;
    const floatx4* base = reinterpret_cast<const floatx4*>(pf.ptr[m]);
    for (size_t f = b0 + threadIdx.x; f < b1; f += blockDim.x) {
      const size_t t = f / gf4, within = f - t * gf4;
      const floatx4 v = base[(xcd + 8 * t) * gf4 + within];
      acc += v[0];
    }
  }
  if (acc == 1.2345678e-38f) *pf.sink = acc;
}

// Σ_z p[z·stride] for z < np (≤ 8), ascending; the loads are all issued
// before the adds (clamped index, branch-free).
__device__ __forceinline__ floatx4 sum_parts(const float* p, int np, size_t stride) {
  if (np <= 1) return *reinterpret_cast<const floatx4*>(p);
  floatx4 t[8];
#pragma unroll
  for (int z = 0; z < 8; ++z) t[z] = *reinterpret_cast<const floatx4*>(p + (size_t)min(z, np - 1) * stride);
  floatx4 v = t[0];
#pragma unroll
  for (int z = 1; z < 8; ++z)
    if (z < np) v += t[z];
  return v;
}

// out[b, h*DH + d] = Σ_c 2^(m_c − M) o_c[d] / Σ_c 2^(m_c − M) l_c, c ascending.
template <int DH>
__device__ __forceinline__ void merge_chunks(const KvArgs& a, int b, int h, int d) {
  const float* rec = a.ws + ((size_t)b * a.H + h) * a.nch * PART;
  float M = -INFINITY;
  for (int c = 0; c < a.nch; ++c) M = fmaxf(M, rec[c * PART]);
  float L = 0.f, o = 0.f;
  for (int c = 0; c < a.nch; ++c) {
    const float f = exp2f(rec[c * PART] - M);
    L += f * rec[c * PART + 1];
    o += f * rec[c * PART + 4 + d];
  }
  a.out[(size_t)b * a.ld + h * DH + d] = L > 0.f ? o / L : 0.f;
}

// DH/4 lanes cover one K/V row (LPK), so one wave load instruction covers
// KPS = 64/LPK keys.
template <int DH>
__global__ void __launch_bounds__(256) kv_chunk_kernel(KvArgs a) {
  constexpr int NP = DH / 4, LPK = pow2_at_least(NP), KPS = 64 / LPK;
  __shared__ float sc[KC];
  __shared__ float red[4];
  __shared__ __attribute__((aligned(16))) float obuf[4][DH];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane / LPK, part = lane % LPK;
  const bool live = part < NP;             // a lane of the group past the row is idle
  const int pa = live ? part : NP - 1;     // its loads stay in range
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int T = a.t_dev ? a.t_dev[b] : a.t_scalar;
  const int c0 = c * KC;
  float* rec = a.ws + (((size_t)b * a.H + h) * a.nch + c) * PART;
  if (c0 >= T) {  // chunk past this sequence's end: neutral record
    if (tid < PART) rec[tid] = tid == 0 ? -INFINITY : 0.f;
  } else {
    const size_t hist = (size_t)b * a.max_len;
    floatx4 qv = sum_parts(a.q + (size_t)b * a.ld_q + h * DH + 4 * pa, a.nparts, a.pstride);
    qv *= live ? a.scale * LOG2E : 0.f;

    // Every K and V row of this wave's keys is requested before any math, so
    // the block has its whole 2·KC·DH·4-byte share of HBM traffic in flight.
    floatx4 kreg[KPW / KPS], vreg[KPW / KPS];
#pragma unroll
    for (int it = 0; it < KPW / KPS; ++it) {
      const int key = c0 + w * KPW + KPS * it + g;
      floatx4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
      if (key < T) {
        if (a.knew && key == T - 1) {
          const size_t o = (size_t)b * a.ld_q + h * DH + 4 * pa;
          kv = sum_parts(a.knew + o, a.nparts, a.pstride);
          vv = sum_parts(a.vnew + o, a.nparts, a.pstride);
          if (live) {
            *reinterpret_cast<floatx4*>(const_cast<float*>(a.kh) + (hist + key) * a.ld + h * DH + 4 * pa) = kv;
            *reinterpret_cast<floatx4*>(const_cast<float*>(a.vh) + (hist + key) * a.ld + h * DH + 4 * pa) = vv;
          }
        } else {
          kv = *reinterpret_cast<const floatx4*>(a.kh + (hist + key) * a.ld + h * DH + 4 * pa);
          vv = *reinterpret_cast<const floatx4*>(a.vh + (hist + key) * a.ld + h * DH + 4 * pa);
        }
      }
      kreg[it] = kv;
      vreg[it] = vv;
    }
    // Scores of this wave's keys, KPS per step (one per LPK-lane group).
    float s_loc[KPW / KPS];
#pragma unroll
    for (int it = 0; it < KPW / KPS; ++it) {
      const floatx4 kv = kreg[it];
      s_loc[it] = qv[0] * kv[0] + qv[1] * kv[1] + qv[2] * kv[2] + qv[3] * kv[3];
    }
#pragma unroll
    for (int it = 0; it < KPW / KPS; ++it) {
      const float s = group_reduce<1, LPK, false>(s_loc[it]);  // the key's LPK lanes
      const int kl = w * KPW + KPS * it + g;
      if (part == 0) sc[kl] = (c0 + kl < T) ? s : -INFINITY;
    }
    __syncthreads();

    // Chunk max and exp-sum (log2 domain).
    float v = tid < KC ? sc[tid] : -INFINITY;
    v = group_reduce<1, 64, true>(v);
    if (lane == 0) red[w] = v;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float e = 0.f;
    if (tid < KC) {
      e = exp2f(sc[tid] - M);
      sc[tid] = e;
    }
    float sum = e;
    sum = group_reduce<1, 64, false>(sum);
    if (lane == 0) red[w] = sum;
    __syncthreads();
    const float L = (red[0] + red[1]) + (red[2] + red[3]);

    // Unnormalised Σ_j p_j v_j over this wave's keys, 4 dims per lane.
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int it = 0; it < KPW / KPS; ++it) {
      const int kl = w * KPW + KPS * it + g;
      acc += sc[kl] * vreg[it];  // sc = 0 for keys >= T (exp2(-inf))
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = group_sum_lanes<LPK>(acc[i]);
    if (g == 0 && live) *reinterpret_cast<floatx4*>(&obuf[w][4 * part]) = acc;
    __syncthreads();
    if (tid < DH) {
      rec[4 + tid] = (obuf[0][tid] + obuf[1][tid]) + (obuf[2][tid] + obuf[3][tid]);
      if (tid == 0) {
        rec[0] = M;
        rec[1] = L;
      }
    }
  }
}

// One block of SW waves per (head, sequence); NT: the history rows, read
// once per step, are loaded non-temporally (streamed past the caches).
// Round r covers keys [r·SW·U·KPS, (r+1)·SW·U·KPS); wave w loads its U key
// groups of the round (KPS keys per load instruction, LPK lanes per key) and
// folds them into its running (m, l, acc) in the log2 domain.  The loads are branch-free (a key
// past the end is clamped to the last one and masked in the math) and the
// next round is loaded before the current one is used, so each wave keeps
// two rounds of HBM reads in flight instead of one round trip per round.
template <int DH, int U, int SW, bool NT>
__global__ void __launch_bounds__(64 * SW) kv_seq_kernel(KvArgs a, int t_max) {
  constexpr int NP = DH / 4, LPK = pow2_at_least(NP), KPS = 64 / LPK;
  constexpr int ROUND = SW * U * KPS;
  __shared__ float wm[SW], wl[SW];
  __shared__ __attribute__((aligned(16))) float wo[SW][DH];
  __shared__ __attribute__((aligned(16))) float qkn[3][DH];  // q (scaled), new k, new v of this head
  if ((int)blockIdx.y >= a.nseq) {  // appended prefetch blocks (a.nseq·H is a multiple of 8)
    const int lin = blockIdx.x + gridDim.x * blockIdx.y;
    l2_prefetch(a.pf, lin % 8, (lin - a.nseq * (int)gridDim.x) / 8);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane / LPK, part = lane % LPK;
  const bool live = part < NP;          // a lane of the group past the row is idle
  const int pa = live ? part : NP - 1;  // its loads stay in range
  const int h = blockIdx.x, b = blockIdx.y;
  const int T = min(a.t_dev ? a.t_dev[b] : a.t_scalar, t_max);
  const size_t hist = (size_t)b * a.max_len;
  const size_t col = (size_t)h * DH + 4 * pa;
  const int last = max(T - 1, 0);
  // History rows only: the new row's slot may be mid-append (every value in
  // it is finite either way); key T-1 takes the shared row before use.
  auto load = [&](int base, floatx4* kr, floatx4* vr) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int key = min(base + (u * SW + w) * KPS + g, last);
      const floatx4* kp = reinterpret_cast<const floatx4*>(a.kh + (hist + key) * a.ld + col);
      const floatx4* vp = reinterpret_cast<const floatx4*>(a.vh + (hist + key) * a.ld + col);
      kr[u] = NT ? __builtin_nontemporal_load(kp) : *kp;
      vr[u] = NT ? __builtin_nontemporal_load(vp) : *vp;
    }
  };
  float m = -INFINITY, l = 0.f;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  floatx4 kc[U], vc[U];
  // The first round's history loads go out before the QKV-partial loads
  // below, so the block waits for one memory round trip, not two (the
  // append's stores would otherwise keep them behind it).
  load(0, kc, vc);
  // One lane group reads q and the new K/V row (summing the QKV partials)
  // and shares them through LDS; it also appends the new row (position
  // T-1) to the history, which nothing in this launch reads back.
  if (w == 0 && g == 0 && live) {
    const size_t o = (size_t)b * a.ld_q + col;
    const floatx4 q4 = sum_parts(a.q + o, a.nparts, a.pstride) * (a.scale * LOG2E);
    *reinterpret_cast<floatx4*>(&qkn[0][4 * part]) = q4;
    if (a.knew) {
      const floatx4 k4 = sum_parts(a.knew + o, a.nparts, a.pstride);
      const floatx4 v4 = sum_parts(a.vnew + o, a.nparts, a.pstride);
      *reinterpret_cast<floatx4*>(&qkn[1][4 * part]) = k4;
      *reinterpret_cast<floatx4*>(&qkn[2][4 * part]) = v4;
      if (T >= 1) {
        *reinterpret_cast<floatx4*>(const_cast<float*>(a.kh) + (hist + T - 1) * a.ld + col) = k4;
        *reinterpret_cast<floatx4*>(const_cast<float*>(a.vh) + (hist + T - 1) * a.ld + col) = v4;
      }
    }
  }
  __syncthreads();
  const floatx4 qv = *reinterpret_cast<const floatx4*>(&qkn[0][4 * pa]) * (live ? 1.f : 0.f);
  floatx4 knew_v = {0.f, 0.f, 0.f, 0.f}, vnew_v = {0.f, 0.f, 0.f, 0.f};
  if (a.knew) {
    knew_v = *reinterpret_cast<const floatx4*>(&qkn[1][4 * pa]);
    vnew_v = *reinterpret_cast<const floatx4*>(&qkn[2][4 * pa]);
  }
  for (int base = 0; base < T; base += ROUND) {
    floatx4 kn[U], vn[U];
    load(base + ROUND, kn, vn);  // clamped: past the end it re-reads the last row (cached)
    if (a.knew) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (base + (u * SW + w) * KPS + g == T - 1) {
          kc[u] = knew_v;
          vc[u] = vnew_v;
        }
    }
    float sc[U];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float s = qv[0] * kc[u][0] + qv[1] * kc[u][1] + qv[2] * kc[u][2] + qv[3] * kc[u][3];
      s = group_reduce<1, LPK, false>(s);  // the key's LPK lanes
      if (base + (u * SW + w) * KPS + g >= T) s = -INFINITY;
      sc[u] = s;
      mx = fmaxf(mx, s);
    }
    mx = group_reduce<LPK, 64, true>(mx);  // uniform over each key's LPK lanes
    const float m_new = fmaxf(m, mx);
    if (m_new != -INFINITY) {  // wave-uniform: some key of this wave so far
      const float alpha = exp2f(m - m_new);
      l *= alpha;
      acc *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = exp2f(sc[u] - m_new);  // 0 for keys past T
        l += p;
        acc += p * vc[u];
      }
      m = m_new;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kc[u] = kn[u];
      vc[u] = vn[u];
    }
  }
  // Sum the lane groups (each group holds its own keys' l and acc; l is
  // uniform over a group's lanes, acc is not: it holds the lane's dims).
  l = group_reduce<LPK, 64, false>(l);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = group_sum_lanes<LPK>(acc[i]);
  if (g == 0 && live) *reinterpret_cast<floatx4*>(&wo[w][4 * part]) = acc;
  if (lane == 0) {
    wm[w] = m;
    wl[w] = l;
  }
  __syncthreads();
  if (tid < DH) {
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < SW; ++i) M = fmaxf(M, wm[i]);
    float L = 0.f, o = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int i = 0; i < SW; ++i) {
        const float f = exp2f(wm[i] - M);  // 0 for a wave that saw no key
        L += f * wl[i];
        o += f * wo[i][tid];
      }
    }
    a.out[(size_t)b * a.ld + h * DH + tid] = L > 0.f ? o / L : 0.f;
  }
}

// Any d_head (the reference's kernel stride-loops over the head's columns,
// src/gpu/kv_cache.rs:339-348): one block per (head, sequence); a thread per
// key computes its score (scalar loads: d_head need not allow float4), the
// scores live in LDS (dynamic, t_max floats), the block takes their max and
// sum, and a thread per output column sums p_j·v_j over the keys.  A
// generality path, not a bandwidth-shaped one; no fused append, no
// partials.
__device__ float block_reduce(float v, float* red, bool is_max) {
  for (int m = 32; m >= 1; m >>= 1) {
    const float o = __shfl_xor(v, m, 64);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();  // red is reused
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < nw; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

__global__ void __launch_bounds__(256) kv_generic_kernel(KvArgs a, int t_max, int dh) {
  extern __shared__ float sc[];
  __shared__ float red[4];
  const int h = blockIdx.x, b = blockIdx.y;
  const int T = min(a.t_dev ? a.t_dev[b] : a.t_scalar, t_max);
  const float* q = a.q + (size_t)b * a.ld_q + (size_t)h * dh;
  const size_t hist = (size_t)b * a.max_len, col = (size_t)h * dh;
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < T; j += blockDim.x) {
    const float* k = a.kh + (hist + j) * a.ld + col;
    float s = 0.f;
    for (int c = 0; c < dh; ++c) s += q[c] * k[c];
    s *= a.scale;
    sc[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_reduce(mx, red, true);
  float sum = 0.f;
  for (int j = threadIdx.x; j < T; j += blockDim.x) {
    const float e = expf(sc[j] - mx);
    sc[j] = e;
    sum += e;
  }
  sum = block_reduce(sum, red, false);  // its barriers also publish sc
  const float inv = sum > 0.f ? 1.f / sum : 0.f;
  for (int c = threadIdx.x; c < dh; c += blockDim.x) {
    float acc = 0.f;
    for (int j = 0; j < T; ++j) acc += sc[j] * inv * a.vh[(hist + j) * a.ld + col + c];
    a.out[(size_t)b * a.ld + col + c] = acc;
  }
}

template <int DH>
__global__ void __launch_bounds__(64) kv_combine_kernel(KvArgs a) {
  merge_chunks<DH>(a, blockIdx.y, blockIdx.x, threadIdx.x);
}

// Launches ceil(t_max / KC) chunks per (head, sequence); t_max must be at
// least every sequence's length (a shorter sequence's surplus chunks write
// neutral records).  The scratch records are laid out [B][H][nch].
template <int DH>
void launch_dh(const KvArgs& a, int B, hipStream_t st) {
  dim3 g1(a.nch, a.H, B);
  hipLaunchKernelGGL(kv_chunk_kernel<DH>, g1, dim3(256), 0, st, a);
  dim3 g2(a.H, B);
  hipLaunchKernelGGL(kv_combine_kernel<DH>, g2, dim3(DH), 0, st, a);
}

template <int DH>
void launch_seq(const KvArgs& a, int B, int t_max, hipStream_t st) {
  // 4 waves per block (two blocks, eight waves per CU at B·H = 512), U = 2
  // key groups per wave per round, history rows loaded non-temporally.
  // Measured on MI355X in the config-4 decode step (0.865 ms/step with 8
  // waves, U = 4, cached loads): non-temporal loads alone 0.831, with 4
  // waves 0.827, 4 waves and U = 2 0.815; U = 1 0.859, 2 waves 0.879, the
  // best shape without non-temporal loads 0.864.  A plain 2 GiB read
  // behaves alike: fastest with two 4-wave blocks per CU and non-temporal
  // loads (6.5 TB/s; 5.0-5.9 TB/s with more waves per CU or cached loads).
  // Prefetch blocks: whole rows of H blocks, 8·blocks_per_xcd of them.
  const int extra = a.pf.nmat > 0 ? (8 * a.pf.blocks_per_xcd + a.H - 1) / a.H : 0;
  hipLaunchKernelGGL((kv_seq_kernel<DH, 2, 4, true>), dim3(a.H, B + extra), dim3(64 * 4), 0, st, a, t_max);
}

// The chunked kernels write ceil(t/KC) records of PART floats per
// (sequence, head) to the scratch, which must not need more than the
// reference's scratch [n_head, max_len] per sequence (src/gpu/transformer.rs:
// 2432).  They are used only when the records of a full-length history fit
// in max_len floats; otherwise (max_len below PART, or just above a multiple
// of KC) the scratch-free one-block-per-(sequence, head) kernel runs.
bool chunks_fit(int max_len) { return (long)((max_len + KC - 1) / KC) * PART <= max_len; }

// d_head of the bandwidth-shaped kernels; any other takes kv_generic_kernel.
bool dh_ok(uint32_t d) { return d >= 8 && d <= 64 && d % 8 == 0; }

constexpr int kGenericMaxKeys = 16384;  // LDS scores of kv_generic_kernel (64 KiB)

int launch(aur_ctx* ctx, KvArgs& a, int B, int t_max, int d_head) {
  if (!dh_ok((uint32_t)d_head)) {
    if (t_max > kGenericMaxKeys)
      return aur::set_error(ctx, AUR_ELIMIT, "mha_kv_step: d_head=%d takes the generic kernel, which holds at "
                            "most %d keys", d_head, kGenericMaxKeys);
    hipLaunchKernelGGL(kv_generic_kernel, dim3(a.H, B), dim3(256), (size_t)t_max * sizeof(float), ctx->stream, a,
                       t_max, d_head);
    AUR_LAUNCH_CHECK(ctx, "kv_generic_kernel");
    return 0;
  }
  a.nch = (t_max + KC - 1) / KC;
  const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  const bool seq = ((long)B * a.H >= cus && std::getenv("AUR_KV_CHUNKED") == nullptr) ||
                   !chunks_fit(a.max_len);
#define AUR_KV_CASE(DH) \
  case DH: seq ? launch_seq<DH>(a, B, t_max, ctx->stream) : launch_dh<DH>(a, B, ctx->stream); break
  switch (d_head) {
    AUR_KV_CASE(8);
    AUR_KV_CASE(16);
    AUR_KV_CASE(24);
    AUR_KV_CASE(32);
    AUR_KV_CASE(40);
    AUR_KV_CASE(48);
    AUR_KV_CASE(56);
    default: seq ? launch_seq<64>(a, B, t_max, ctx->stream) : launch_dh<64>(a, B, ctx->stream); break;
  }
#undef AUR_KV_CASE
  AUR_LAUNCH_CHECK(ctx, "kv decode kernels");
  return 0;
}

bool aligned16_kv(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" {

size_t aur_mha_kv_ws_bytes(uint32_t b, uint32_t n_head, uint32_t max_len) {
  const size_t nch = (max_len + KC - 1) / KC;
  return chunks_fit((int)max_len) ? (size_t)b * n_head * nch * PART * sizeof(float) : 0;
}

int aur_mha_kv_step(aur_ctx* ctx, const float* q_new, const float* k_history, const float* v_history,
                    float* out, float* scratch, uint32_t t_total, uint32_t n_head, uint32_t d_head,
                    uint32_t max_len) {
  AUR_CHECK_CTX(ctx);
  if (d_head == 0) return aur::set_error(ctx, AUR_EINVAL, "mha_kv_step: d_head=0");
  if (t_total == 0 || t_total > max_len || n_head == 0)
    return aur::set_error(ctx, AUR_EINVAL, "mha_kv_step: t_total=%u max_len=%u", t_total, max_len);
  if (!q_new || !k_history || !v_history || !out || !scratch)
    return aur::set_error(ctx, AUR_EINVAL, "mha_kv_step: null pointer");
  KvArgs a{};
  a.q = q_new; a.kh = k_history; a.vh = v_history; a.out = out; a.ws = scratch;
  a.t_dev = nullptr; a.t_scalar = (int)t_total;
  a.nseq = 1;
  a.ld = (int)(n_head * d_head); a.ld_q = a.ld; a.max_len = (int)max_len; a.H = (int)n_head;
  a.scale = 1.0f / sqrtf((float)d_head);
  return launch(ctx, a, 1, (int)t_total, (int)d_head);
}

int aur_mha_kv_step_batched(aur_ctx* ctx, const float* q_new, const float* k_history,
                            const float* v_history, float* out, float* scratch, const int32_t* t_total,
                            uint32_t t_max, uint32_t b, uint32_t n_head, uint32_t d_head,
                            uint32_t max_len) {
  AUR_CHECK_CTX(ctx);
  return aur::mha_kv_batched(ctx, q_new, (int)(n_head * d_head), k_history, v_history, out, scratch,
                             t_total, (int)t_max, (int)b, (int)n_head, (int)d_head, (int)max_len);
}

}  // extern "C"

namespace aur {

int mha_kv_batched(aur_ctx* ctx, const float* q, int ld_q, const float* k_history,
                   const float* v_history, float* out, float* scratch, const int32_t* t_total, int t_max,
                   int b, int n_head, int d_head, int max_len, const float* k_new, const float* v_new,
                   int nparts, size_t part_stride, const L2Prefetch* prefetch) {
  if (d_head <= 0) return set_error(ctx, AUR_EINVAL, "mha_kv_step_batched: d_head=%d", d_head);
  if (!dh_ok((uint32_t)d_head) && (k_new || v_new || nparts > 1))
    return set_error(ctx, AUR_ELIMIT, "mha_kv_step_batched: the fused append and QKV partials need d_head a "
                     "multiple of 8 up to 64 (d_head=%d)", d_head);
  if (b <= 0 || n_head <= 0 || t_max <= 0 || t_max > max_len || ld_q < n_head * d_head ||
      (dh_ok((uint32_t)d_head) && (ld_q & 3)))
    return set_error(ctx, AUR_EINVAL, "mha_kv_step_batched: b=%d t_max=%d max_len=%d ld_q=%d", b, t_max,
                     max_len, ld_q);
  if (!q || !k_history || !v_history || !out || !scratch || !t_total || (!k_new != !v_new))
    return set_error(ctx, AUR_EINVAL, "mha_kv_step_batched: null pointer");
  if (nparts < 1 || nparts > 8 || (nparts > 1 && (part_stride < (size_t)b * ld_q || (part_stride & 3))))
    return set_error(ctx, AUR_EINVAL, "mha_kv_step_batched: nparts=%d part_stride=%zu", nparts, part_stride);
  KvArgs a{};
  a.q = q; a.kh = k_history; a.vh = v_history; a.out = out; a.ws = scratch;
  a.t_dev = t_total; a.t_scalar = 0;
  a.ld = n_head * d_head; a.ld_q = ld_q; a.max_len = max_len; a.H = n_head;
  a.scale = 1.0f / sqrtf((float)d_head);
  a.knew = k_new; a.vnew = v_new;
  a.nparts = nparts; a.pstride = part_stride;
  a.nseq = b;
  if (prefetch && prefetch->nmat > 0) {
    // Only the one-block-per-(sequence, head) kernel carries prefetch blocks
    // (the chunked kernels ignore the plan), and their slot arithmetic needs
    // the attention blocks to fill whole rounds of the 8 XCDs.
    if ((b * n_head) % 8 == 0 && prefetch->blocks_per_xcd > 0 && prefetch->nmat <= 3 && prefetch->sink) {
      bool ok = true;
      for (int m = 0; m < prefetch->nmat; ++m)
        ok = ok && prefetch->ptr[m] && prefetch->group[m] > 0 && prefetch->rows[m] % prefetch->group[m] == 0 &&
             prefetch->row_floats[m] % 4 == 0 && aligned16_kv(prefetch->ptr[m]);
      if (ok) a.pf = *prefetch;
    }
  }
  return launch(ctx, a, b, t_max, d_head);
}

}  // namespace aur
