// Step-support kernels around the GEMM / attention hot path: everything one
// training step (embed → blocks → LN → tied head → CE → backward → clip →
// AdamW) and one KV-cache decode step need besides the matrix products.
// All reductions have a fixed order (no atomics), so a step is bitwise
// reproducible run to run.  These are bandwidth-bound elementwise / row
// kernels: one wave per row, float4 traffic where the row allows it.
//
// Reference semantics: LN src/attention.rs:84-157 (eps 1e-5, biased
// variance), softmax-CE src/transformer/model.rs:820-858, embedding
// src/transformer/embedding.rs:95-142, clip model.rs:1011-1017 with the
// L2 norm of model.rs:442-500, AdamW src/optimizer.rs:58-90.
#include "common.hpp"
#include "step_ops.hpp"

namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Block-wide sum for 256 threads; every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ---------------------------------------------------------------- embedding
// out[r, :] = w_tok[tok[r], :] + w_pos[pos(r), :],  pos(r) = pos_dev ? pos_dev[r] : r % T.
__global__ void __launch_bounds__(256) embed_fwd_kernel(const float* __restrict__ w_tok,
                                                        const float* __restrict__ w_pos,
                                                        const uint32_t* __restrict__ tok,
                                                        const int32_t* __restrict__ pos_dev, int T,
                                                        float* __restrict__ out, int rows, int d,
                                                        int32_t* __restrict__ lens) {
  const int r = blockIdx.x;
  if (r >= rows) return;
  const int p = pos_dev ? pos_dev[r] : r % T;
  if (lens && threadIdx.x == 0) lens[r] = p + 1;  // decode: attention length incl. this token
  const float* a = w_tok + (size_t)tok[r] * d;
  const float* b = w_pos + (size_t)p * d;
  float* o = out + (size_t)r * d;
  for (int c = threadIdx.x; c < d; c += blockDim.x) o[c] = a[c] + b[c];
}

// g_w_tok[v, :] += Σ_{r ∈ rows(v)} dy[r, :] with rows(v) ascending (CSR built
// on the host from the token ids: tok_ids[u], row_off[u]..row_off[u+1]).
__global__ void __launch_bounds__(256) embed_tok_bwd_kernel(const float* __restrict__ dy,
                                                            const uint32_t* __restrict__ tok_ids,
                                                            const int32_t* __restrict__ row_off,
                                                            const int32_t* __restrict__ row_idx,
                                                            float* __restrict__ g_w_tok, int d) {
  const int u = blockIdx.x;
  const int beg = row_off[u], end = row_off[u + 1];
  float* g = g_w_tok + (size_t)tok_ids[u] * d;
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    float s = 0.f;
    for (int i = beg; i < end; ++i) s += dy[(size_t)row_idx[i] * d + c];
    g[c] += s;
  }
}

// g_w_pos[t, :] += Σ_b dy[b*T + t, :], b ascending.
__global__ void __launch_bounds__(256) embed_pos_bwd_kernel(const float* __restrict__ dy, int B, int T,
                                                            float* __restrict__ g_w_pos, int d) {
  const int t = blockIdx.x;
  float* g = g_w_pos + (size_t)t * d;
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    float s = 0.f;
    for (int b = 0; b < B; ++b) s += dy[((size_t)b * T + t) * d + c];
    g[c] += s;
  }
}

// ---------------------------------------------------------------- layer norm
// One wave per row: mu = Σx/d, var = Σ(x−mu)²/d, s = 1/sqrt(var + eps),
// y = (x − mu)·s·γ + β.  Saves mean and s for the backward.
__global__ void __launch_bounds__(256) ln_fwd_kernel(const float* __restrict__ x,
                                                     const float* __restrict__ gamma,
                                                     const float* __restrict__ beta,
                                                     float* __restrict__ y, float* __restrict__ mean,
                                                     float* __restrict__ rstd, int rows, int d,
                                                     float eps) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float* xr = x + (size_t)r * d;
  float s = 0.f;
  for (int c = lane; c < d; c += 64) s += xr[c];
  const float mu = wave_sum(s) / (float)d;
  float v = 0.f;
  for (int c = lane; c < d; c += 64) {
    const float t = xr[c] - mu;
    v += t * t;
  }
  const float var = wave_sum(v) / (float)d;
  const float is = 1.0f / sqrtf(var + eps);
  float* yr = y + (size_t)r * d;
  for (int c = lane; c < d; c += 64) yr[c] = (xr[c] - mu) * is * gamma[c] + beta[c];
  if (lane == 0) {
    if (mean) mean[r] = mu;
    if (rstd) rstd[r] = is;
  }
}

// Row-resident forms for d = 256·NV (the model widths): one wave per row,
// float4 traffic, the row read once into registers and reused for the
// statistics and the output.
template <int NV>
__global__ void __launch_bounds__(256) ln_fwd_vec_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta,
                                                         float* __restrict__ y, float* __restrict__ mean,
                                                         float* __restrict__ rstd, int rows, float eps) {
  constexpr int D = 256 * NV;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const floatx4* xr = reinterpret_cast<const floatx4*>(x + (size_t)r * D);
  floatx4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = xr[lane + 64 * i];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
  const float mu = wave_sum(s) / (float)D;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) q += (v[i][e] - mu) * (v[i][e] - mu);
  const float is = 1.0f / sqrtf(wave_sum(q) / (float)D + eps);
  const floatx4* g4 = reinterpret_cast<const floatx4*>(gamma);
  const floatx4* b4 = reinterpret_cast<const floatx4*>(beta);
  floatx4* yr = reinterpret_cast<floatx4*>(y + (size_t)r * D);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const floatx4 gg = g4[lane + 64 * i], bb = b4[lane + 64 * i];
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (v[i][e] - mu) * is * gg[e] + bb[e];
    yr[lane + 64 * i] = o;
  }
  if (lane == 0) {
    if (mean) mean[r] = mu;
    if (rstd) rstd[r] = is;
  }
}

// The same for few rows (decode: one row per sequence): one 256-thread block
// per row, float4 traffic, so a launch over 32 rows is not latency-bound.
// Requires d % 4 == 0 and 16-byte aligned rows.
__global__ void __launch_bounds__(256) ln_fwd_rowblock_kernel(const float* __restrict__ x,
                                                              const float* __restrict__ gamma,
                                                              const float* __restrict__ beta,
                                                              float* __restrict__ y,
                                                              float* __restrict__ mean,
                                                              float* __restrict__ rstd, int d,
                                                              float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const float* xr = x + (size_t)r * d;
  float s = 0.f;
  for (int c = threadIdx.x * 4; c < d; c += 1024) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(xr + c);
    s += (v[0] + v[1]) + (v[2] + v[3]);
  }
  const float mu = block_sum(s, red) / (float)d;
  float q = 0.f;
  for (int c = threadIdx.x * 4; c < d; c += 1024) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(xr + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) q += (v[e] - mu) * (v[e] - mu);
  }
  const float is = 1.0f / sqrtf(block_sum(q, red) / (float)d + eps);
  float* yr = y + (size_t)r * d;
  for (int c = threadIdx.x * 4; c < d; c += 1024) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(xr + c);
    const floatx4 gg = *reinterpret_cast<const floatx4*>(gamma + c);
    const floatx4 bb = *reinterpret_cast<const floatx4*>(beta + c);
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (v[e] - mu) * is * gg[e] + bb[e];
    *reinterpret_cast<floatx4*>(yr + c) = o;
  }
  if (threadIdx.x == 0) {
    if (mean) mean[r] = mu;
    if (rstd) rstd[r] = is;
  }
}

// Decode-step LayerNorm that first completes the residual add of a split-K
// projection: x = R + (P[0] + P[1] + … + P[np−1]) (ranges in order, the
// product summed before the residual is added, as an unsplit GEMM's
// epilogue would), writes x (the residual stream) and y = LN(x).  One block
// per row; each thread keeps its ≤ 4 float4 of the row in registers.
__global__ void __launch_bounds__(256) ln_fwd_sum_kernel(const float* __restrict__ R,
                                                         const float* __restrict__ P, int np,
                                                         size_t pstride, float* __restrict__ xo,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta,
                                                         float* __restrict__ y, int d, float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  // γ and β are requested with the row, not after the two reductions: one
  // memory round trip fewer per launch.
  floatx4 gg[4], bb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (threadIdx.x + 256 * i) * 4;
    if (c < d) {
      gg[i] = *reinterpret_cast<const floatx4*>(gamma + c);
      bb[i] = *reinterpret_cast<const floatx4*>(beta + c);
    }
  }
  floatx4 xv[4];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (threadIdx.x + 256 * i) * 4;
    floatx4 v = {0.f, 0.f, 0.f, 0.f};
    if (c < d) {
      // Partials summed in z order.  16 at a time, branch-free (an index
      // past np re-reads the last partial and adds 0), so all of a batch's
      // loads are in flight together — one memory round trip for np ≤ 16.
      const float* pc = P + (size_t)r * d + c;
      const floatx4 rv = *reinterpret_cast<const floatx4*>(R + (size_t)r * d + c);
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int z0 = 0; z0 < np; z0 += 16) {
        floatx4 t[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
          t[j] = *reinterpret_cast<const floatx4*>(pc + (size_t)min(z0 + j, np - 1) * pstride);
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (z0 + j < np) acc += t[j];
      }
      v = rv + acc;
      *reinterpret_cast<floatx4*>(xo + (size_t)r * d + c) = v;
      s += (v[0] + v[1]) + (v[2] + v[3]);
    }
    xv[i] = v;
  }
  const float mu = block_sum(s, red) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (threadIdx.x + 256 * i) * 4;
    if (c < d)
#pragma unroll
      for (int e = 0; e < 4; ++e) q += (xv[i][e] - mu) * (xv[i][e] - mu);
  }
  const float is = 1.0f / sqrtf(block_sum(q, red) / (float)d + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (threadIdx.x + 256 * i) * 4;
    if (c < d) {
      floatx4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (xv[i][e] - mu) * is * gg[i][e] + bb[i][e];
      *reinterpret_cast<floatx4*>(y + (size_t)r * d + c) = o;
    }
  }
}

// dx = s·(g − (Σg + x̂·Σ(g·x̂))/d) [+ dres],  g = dy·γ,  x̂ = (x − mu)·s.
__global__ void __launch_bounds__(256) ln_bwd_kernel(const float* __restrict__ x,
                                                     const float* __restrict__ mean,
                                                     const float* __restrict__ rstd,
                                                     const float* __restrict__ gamma,
                                                     const float* __restrict__ dy,
                                                     const float* __restrict__ dres,
                                                     float* __restrict__ dx, int rows, int d) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float mu = mean[r], s = rstd[r];
  const float* xr = x + (size_t)r * d;
  const float* dyr = dy + (size_t)r * d;
  float sg = 0.f, sgx = 0.f;
  for (int c = lane; c < d; c += 64) {
    const float g = dyr[c] * gamma[c];
    sg += g;
    sgx += g * ((xr[c] - mu) * s);
  }
  sg = wave_sum(sg);
  sgx = wave_sum(sgx);
  const float inv_d = 1.0f / (float)d;
  float* dxr = dx + (size_t)r * d;
  const float* dr = dres ? dres + (size_t)r * d : nullptr;
  for (int c = lane; c < d; c += 64) {
    const float g = dyr[c] * gamma[c];
    const float xh = (xr[c] - mu) * s;
    float v = s * (g - inv_d * (sg + xh * sgx));
    if (dr) v += dr[c];
    dxr[c] = v;
  }
}

// ln_bwd_kernel for d = 256·NV: x, dy, γ (and dres) read once as float4.
template <int NV>
__global__ void __launch_bounds__(256) ln_bwd_vec_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ mean,
                                                         const float* __restrict__ rstd,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ dy,
                                                         const float* __restrict__ dres,
                                                         float* __restrict__ dx, int rows) {
  constexpr int D = 256 * NV;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float mu = mean[r], s = rstd[r];
  const floatx4* xr = reinterpret_cast<const floatx4*>(x + (size_t)r * D);
  const floatx4* dyr = reinterpret_cast<const floatx4*>(dy + (size_t)r * D);
  const floatx4* g4 = reinterpret_cast<const floatx4*>(gamma);
  floatx4 g[NV], xh[NV];
  float sg = 0.f, sgx = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const floatx4 xv = xr[lane + 64 * i], dv = dyr[lane + 64 * i], gv = g4[lane + 64 * i];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      g[i][e] = dv[e] * gv[e];
      xh[i][e] = (xv[e] - mu) * s;
      sg += g[i][e];
      sgx += g[i][e] * xh[i][e];
    }
  }
  sg = wave_sum(sg);
  sgx = wave_sum(sgx);
  const float inv_d = 1.0f / (float)D;
  floatx4* dxr = reinterpret_cast<floatx4*>(dx + (size_t)r * D);
  const floatx4* dr = dres ? reinterpret_cast<const floatx4*>(dres + (size_t)r * D) : nullptr;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = s * (g[i][e] - inv_d * (sg + xh[i][e] * sgx));
    if (dr) o += dr[lane + 64 * i];
    dxr[lane + 64 * i] = o;
  }
}

// Partial column sums over a chunk of rows: pg[chunk][c] = Σ dy·x̂, pb = Σ dy.
constexpr int LN_CHUNK = 64;
__global__ void __launch_bounds__(256) ln_param_partial_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ mean,
                                                               const float* __restrict__ rstd,
                                                               const float* __restrict__ dy,
                                                               float* __restrict__ pg,
                                                               float* __restrict__ pb, int rows,
                                                               int d) {
  const int chunk = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= d) return;
  const int r0 = chunk * LN_CHUNK, r1 = min(rows, r0 + LN_CHUNK);
  float sgm = 0.f, sb = 0.f;
  // Unrolled so that several rows' loads are in flight; the sums still run
  // in increasing r.
#pragma unroll 16
  for (int r = r0; r < r1; ++r) {
    const float g = dy[(size_t)r * d + c];
    sgm += g * ((x[(size_t)r * d + c] - mean[r]) * rstd[r]);
    sb += g;
  }
  pg[(size_t)chunk * d + c] = sgm;
  pb[(size_t)chunk * d + c] = sb;
}

// ln_bwd_vec_kernel fused with the γ/β partial sums, so that x and dy are read
// once for dx, dγ and dβ.  A block owns LN_FCHUNK consecutive rows, eight per
// wave; each lane keeps Σ dy·x̂ and Σ dy for its columns over its wave's rows
// (ascending r), the four waves' sums are added in wave order through LDS, and
// wave 0 writes the chunk's partial row of pg / pb.  For NV ≤ 4 the loads of
// two rows are issued before either is reduced, to keep more bytes in flight.
constexpr int LN_FCHUNK = 32;
template <int NV>
__global__ void __launch_bounds__(256) ln_bwd_fused_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ rstd,
                                                           const float* __restrict__ gamma,
                                                           const float* __restrict__ dy,
                                                           const float* __restrict__ dres,
                                                           float* __restrict__ dx, float* __restrict__ pg,
                                                           float* __restrict__ pb, int rows) {
  constexpr int D = 256 * NV;
  constexpr int RPW = LN_FCHUNK / 4;
  constexpr int RB = NV <= 4 ? 2 : 1;
  __shared__ floatx4 red[2][3][64 * NV];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rbase = blockIdx.x * LN_FCHUNK + w * RPW;
  const floatx4* g4 = reinterpret_cast<const floatx4*>(gamma);
  floatx4 gam[NV], accg[NV], accb[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    gam[i] = g4[lane + 64 * i];
    accg[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    accb[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  const float inv_d = 1.0f / (float)D;
  for (int j = 0; j < RPW; j += RB) {
    floatx4 xv[RB][NV], dv[RB][NV], rv[RB][NV];
    float mu[RB], s[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      // A row past the end is clamped to the last row: its loads stay in
      // bounds and its results are never used.
      const int rr = min(rbase + j + b, rows - 1);
      mu[b] = mean[rr];
      s[b] = rstd[rr];
      const floatx4* xr = reinterpret_cast<const floatx4*>(x + (size_t)rr * D);
      const floatx4* dyr = reinterpret_cast<const floatx4*>(dy + (size_t)rr * D);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        xv[b][i] = xr[lane + 64 * i];
        dv[b][i] = dyr[lane + 64 * i];
      }
      // The residual gradient is loaded with x and dy, not after the row's
      // reductions, so its latency overlaps theirs.
      if (dres) {
        const floatx4* drr = reinterpret_cast<const floatx4*>(dres + (size_t)rr * D);
#pragma unroll
        for (int i = 0; i < NV; ++i) rv[b][i] = drr[lane + 64 * i];
      } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) rv[b][i] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const int r = rbase + j + b;
      if (r >= rows) break;  // r depends only on the wave: uniform
      floatx4 g[NV], xh[NV];
      float sg = 0.f, sgx = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g[i][e] = dv[b][i][e] * gam[i][e];
          xh[i][e] = (xv[b][i][e] - mu[b]) * s[b];
          sg += g[i][e];
          sgx += g[i][e] * xh[i][e];
          accg[i][e] += dv[b][i][e] * xh[i][e];
          accb[i][e] += dv[b][i][e];
        }
      }
      sg = wave_sum(sg);
      sgx = wave_sum(sgx);
      floatx4* dxr = reinterpret_cast<floatx4*>(dx + (size_t)r * D);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        floatx4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = s[b] * (g[i][e] - inv_d * (sg + xh[i][e] * sgx));
        if (dres) o += rv[b][i];
        dxr[lane + 64 * i] = o;
      }
    }
  }
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      red[0][w - 1][lane + 64 * i] = accg[i];
      red[1][w - 1][lane + 64 * i] = accb[i];
    }
  }
  __syncthreads();
  if (w == 0) {
    floatx4* pgr = reinterpret_cast<floatx4*>(pg + (size_t)blockIdx.x * D);
    floatx4* pbr = reinterpret_cast<floatx4*>(pb + (size_t)blockIdx.x * D);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      floatx4 sgv = accg[i], sbv = accb[i];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        sgv += red[0][k][lane + 64 * i];
        sbv += red[1][k][lane + 64 * i];
      }
      pgr[lane + 64 * i] = sgv;
      pbr[lane + 64 * i] = sbv;
    }
  }
}

// dγ[c] += Σ_chunk pg[chunk][c], dβ[c] += Σ_chunk pb[chunk][c].  A block owns
// 4 columns; its 256 threads are 4 columns × 64 chunk classes (thread
// q·4 + col takes chunks ≡ q mod 64, summed ascending).  A wave's 16 class
// sums per column are combined by a fixed xor butterfly and the four waves'
// sums are added in wave order through LDS — a fixed order, so the result is
// deterministic — with d / 4 blocks to spread the partial rows' reads.
__global__ void __launch_bounds__(256) ln_param_final_kernel(const float* __restrict__ pg,
                                                             const float* __restrict__ pb,
                                                             int nchunks, float* __restrict__ dgamma,
                                                             float* __restrict__ dbeta, int d) {
  __shared__ float sg_[4][4], sb_[4][4];
  const int col = threadIdx.x & 3, q = threadIdx.x >> 2, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 4 + col;
  float sg = 0.f, sb = 0.f;
  if (c < d)
    for (int k = q; k < nchunks; k += 64) {
      sg += pg[(size_t)k * d + c];
      sb += pb[(size_t)k * d + c];
    }
#pragma unroll
  for (int m = 4; m < 64; m <<= 1) {
    sg += __shfl_xor(sg, m, 64);
    sb += __shfl_xor(sb, m, 64);
  }
  if ((threadIdx.x & 63) < 4) {
    sg_[w][col] = sg;
    sb_[w][col] = sb;
  }
  __syncthreads();
  if (threadIdx.x < 4 && c < d) {
    dgamma[c] += ((sg_[0][col] + sg_[1][col]) + sg_[2][col]) + sg_[3][col];
    dbeta[c] += ((sb_[0][col] + sb_[1][col]) + sb_[2][col]) + sb_[3][col];
  }
}

// ---------------------------------------------------------------- softmax-CE
// In place: logits row → (softmax − onehot(target))·scale, and
// nll[r] = −ln(max(p_target, 1e-12)).
__global__ void __launch_bounds__(256) softmax_ce_kernel(float* __restrict__ logits,
                                                         const uint32_t* __restrict__ targets,
                                                         float* __restrict__ nll, int V,
                                                         float scale) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  float* row = logits + (size_t)r * V;
  float mx = -INFINITY;
  for (int c = threadIdx.x; c < V; c += 256) mx = fmaxf(mx, row[c]);
  mx = block_max(mx, red);
  float s = 0.f;
  for (int c = threadIdx.x; c < V; c += 256) {
    const float e = expf(row[c] - mx);
    row[c] = e;
    s += e;
  }
  s = block_sum(s, red);
  const float inv = 1.0f / s;
  const uint32_t tgt = targets[r];
  __syncthreads();
  if (threadIdx.x == 0) nll[r] = -logf(fmaxf(row[tgt] * inv, 1e-12f));
  __syncthreads();
  for (int c = threadIdx.x; c < V; c += 256) {
    float g = row[c] * inv;
    if ((uint32_t)c == tgt) g -= 1.0f;
    row[c] = g * scale;
  }
}

// Row-resident variant for V = 1024·NV: each thread keeps its NV float4 of
// the row in registers, so the logits are read once and the gradient written
// once (the loop form above re-reads the row for every pass: ~2.5× the HBM
// traffic).  Same arithmetic per element (expf, one reciprocal of the sum).
template <int NV>
__global__ void __launch_bounds__(256) softmax_ce_vec_kernel(float* __restrict__ logits,
                                                             const uint32_t* __restrict__ targets,
                                                             float* __restrict__ nll, float scale) {
  constexpr int V = 1024 * NV;
  __shared__ float red[4];
  __shared__ float tgt_p;
  const int r = blockIdx.x;
  float* row = logits + (size_t)r * V;
  floatx4 x[NV];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    x[i] = *reinterpret_cast<const floatx4*>(row + 4 * (threadIdx.x + 256 * i));
    mx = fmaxf(mx, fmaxf(fmaxf(x[i][0], x[i][1]), fmaxf(x[i][2], x[i][3])));
  }
  mx = block_max(mx, red);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[i][e] = expf(x[i][e] - mx);
      s += x[i][e];
    }
  s = block_sum(s, red);
  const float inv = 1.0f / s;
  const uint32_t tgt = targets[r];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t c0 = 4u * (threadIdx.x + 256u * i);
    if (tgt >= c0 && tgt < c0 + 4u) tgt_p = x[i][tgt - c0];
  }
  __syncthreads();
  if (threadIdx.x == 0) nll[r] = -logf(fmaxf(tgt_p * inv, 1e-12f));
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t c0 = 4u * (threadIdx.x + 256u * i);
    floatx4 g = x[i] * inv;
    if (tgt >= c0 && tgt < c0 + 4u) g[tgt - c0] -= 1.0f;
    *reinterpret_cast<floatx4*>(row + c0) = g * scale;
  }
}

// ---------------------------------------------------------- grad norm / clip
// Deterministic two-stage Σ g²: fixed-size blocks, then one block in order.
__global__ void __launch_bounds__(256) sumsq_partial_kernel(const float* __restrict__ g, size_t n,
                                                            float* __restrict__ part) {
  __shared__ float red[4];
  const size_t per = (n + gridDim.x - 1) / gridDim.x;
  const size_t beg = (size_t)blockIdx.x * per, end = min(n, beg + per);
  float s = 0.f;
  for (size_t i = beg + threadIdx.x; i < end; i += 256) s += g[i] * g[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

// stats[0] = ‖g‖₂ and stats[1] = the clip factor (max_norm/‖g‖ if
// ‖g‖ > max_norm > 0, else 1) — or, with frob_inv, 1/(‖g‖ + 1e-7): Muon's
// Frobenius bound before Newton–Schulz (src/gpu/muon.rs:112-156).
__global__ void __launch_bounds__(256) norm_final_kernel(const float* __restrict__ part, int nparts,
                                                         float max_norm, float* __restrict__ stats,
                                                         int frob_inv) {
  __shared__ float red[4];
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += 256) s += part[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) {
    const float nrm = sqrtf(s);
    stats[0] = nrm;
    if (frob_inv)
      stats[1] = 1.0f / (nrm + 1e-7f);
    else
      stats[1] = (max_norm > 0.f && nrm > max_norm && nrm > 0.f) ? max_norm / nrm : 1.0f;
  }
}

// ---------------------------------------------------------------- AdamW
// Elements [0, n_decay) get decoupled weight decay, [n_decay, n) do not.
// The gradient is multiplied by *clip (the clip factor) on the fly, which
// equals the reference's in-place grads.scale(max/‖g‖) before the update.
__global__ void __launch_bounds__(256) adamw_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                    float* __restrict__ m1, float* __restrict__ m2,
                                                    size_t n, size_t n_decay,
                                                    const float* __restrict__ clip, float lr,
                                                    float b1, float b2, float eps, float wd, float bc1,
                                                    float bc2) {
  const float cf = clip ? *clip : 1.0f;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gi = cf == 1.0f ? g[i] : g[i] * cf;
    const float a = b1 * m1[i] + (1.0f - b1) * gi;
    const float b = b2 * m2[i] + (1.0f - b2) * gi * gi;
    m1[i] = a;
    m2[i] = b;
    const float mh = a / bc1, vh = b / bc2;
    float step = lr * mh / (sqrtf(vh) + eps);
    if (i < n_decay) step += lr * wd * p[i];
    p[i] -= step;
  }
}

__global__ void __launch_bounds__(256) scale_kernel(float* __restrict__ x, size_t n,
                                                    const float* __restrict__ f) {
  const float cf = *f;
  if (cf == 1.0f) return;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) x[i] *= cf;
}

// ---------------------------------------------------------------- Muon
// m = β·m + g; update = nesterov ? g + β·m : m   (src/optimizer.rs:273-285,
// src/gpu/muon.rs:18-37).
__global__ void __launch_bounds__(256) muon_momentum_kernel(const float* __restrict__ g, float* __restrict__ m,
                                                            float* __restrict__ upd, size_t n, float beta,
                                                            int nesterov) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gi = g[i];
    const float mn = beta * m[i] + gi;
    m[i] = mn;
    upd[i] = nesterov ? gi + beta * mn : mn;
  }
}

// Newton–Schulz coefficient matrix of nb stacked m × m matrices:
// out = a·I + b·A + c·A², so that one product out·X gives a·X + (b·A + c·A²)·X
// (the reference combines B = b·A + c·A² and X' = a·X + B·X in two passes,
// src/gpu/muon.rs:421-515).
__global__ void __launch_bounds__(256) ns_combine_kernel(float* __restrict__ out, const float* __restrict__ A,
                                                         const float* __restrict__ A2, float a, float b,
                                                         float c, size_t m, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const size_t e = i % (m * m);
    out[i] = b * A[i] + c * A2[i] + (e / m == e % m ? a : 0.f);
  }
}

// dst[c][r] = src[r][c] for src [rows × cols], through 32×33 LDS tiles so
// both sides are coalesced (src/gpu/muon.rs:204-271 load/store).
__global__ void __launch_bounds__(256) transpose_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                        int rows, int cols) {
  __shared__ float t[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 8 rows per pass
  for (int i = ty; i < 32; i += 8) {
    const int r = r0 + i, c = c0 + tx;
    if (r < rows && c < cols) t[i][tx] = src[(size_t)r * cols + c];
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int c = c0 + i, r = r0 + tx;
    if (r < rows && c < cols) dst[(size_t)c * rows + r] = t[tx][i];
  }
}

// params -= lr·scale·update + lr·wd·params   (src/optimizer.rs:292-304,
// src/gpu/muon.rs:517-560; decoupled decay applies to every Muon matrix).
__global__ void __launch_bounds__(256) muon_apply_kernel(float* __restrict__ p, const float* __restrict__ upd,
                                                         size_t n, float lr_scale, float lr_wd) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float step = lr_scale * upd[i];
    if (lr_wd != 0.f) step += lr_wd * p[i];
    p[i] -= step;
  }
}

// ------------------------------------------------------------------ KV cache
// Copies the k and v parts of qkv rows into the per-sequence history:
//   hist[b, pos, :] = qkv[row, d:2d] / qkv[row, 2d:3d]
// decode: row = b, pos = pos_dev[b];  prefill: row = b*T + t, pos = t.
__global__ void __launch_bounds__(256) kv_store_kernel(const float* __restrict__ qkv, int d,
                                                       float* __restrict__ kh, float* __restrict__ vh,
                                                       int max_len, const int32_t* __restrict__ pos_dev,
                                                       int T) {
  const int row = blockIdx.x;
  int b, pos;
  if (pos_dev) {
    b = row;
    pos = pos_dev[row];
  } else {
    b = row / T;
    pos = row % T;
  }
  const float* src = qkv + (size_t)row * 3 * d;
  float* kd = kh + ((size_t)b * max_len + pos) * d;
  float* vd = vh + ((size_t)b * max_len + pos) * d;
  for (int c = threadIdx.x; c < d; c += 256) {
    kd[c] = src[d + c];
    vd[c] = src[2 * d + c];
  }
}

// First index of the row maximum (src/transformer/loss.rs argmax: strict >).
// pos (optional): the row's sequence position is advanced by one — the end
// of a decode step.
__global__ void __launch_bounds__(256) argmax_kernel(const float* __restrict__ logits, int V,
                                                     uint32_t* __restrict__ out, int32_t* __restrict__ pos) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int r = blockIdx.x;
  const float* row = logits + (size_t)r * V;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int c = threadIdx.x; c < V; c += 256) {
    const float v = row[c];
    if (v > best) {
      best = v;
      bi = c;
    }
  }
  sv[threadIdx.x] = best;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = 128; s >= 1; s >>= 1) {
    if (threadIdx.x < s) {
      const float ov = sv[threadIdx.x + s];
      const int oi = si[threadIdx.x + s];
      if (ov > sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < si[threadIdx.x])) {
        sv[threadIdx.x] = ov;
        si[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[r] = (uint32_t)(si[0] == 0x7fffffff ? 0 : si[0]);
    if (pos) pos[r] += 1;
  }
}

// The same for V % 4 == 0 with 16-byte aligned rows; the kernel can also
// complete a split-K product first: logits = P[0] + … + P[np−1] (summed in
// range order, written to `logits` when P is not that buffer).  Each thread
// holds 8 float4 columns per pass, all loads of a pass issued together; the
// (value, index) pairs reduce across the block, ties to the lower index.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__global__ void __launch_bounds__(256) argmax_sum_kernel(const float* __restrict__ P, int np, size_t pstride,
                                                         float* __restrict__ logits, int V,
                                                         uint32_t* __restrict__ out, int32_t* __restrict__ pos) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const float* pr = P + (size_t)r * V;
  float* lr = logits + (size_t)r * V;
  const bool store = P != logits;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int c0 = 0; c0 < V; c0 += 8 * 1024) {
    floatx4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = c0 + 1024 * j + 4 * tid;
      floatx4 a = {0.f, 0.f, 0.f, 0.f};
      if (c < V) {
        a = *reinterpret_cast<const floatx4*>(pr + c);
        for (int z = 1; z < np; ++z) a += *reinterpret_cast<const floatx4*>(pr + z * pstride + c);
        if (store) *reinterpret_cast<floatx4*>(lr + c) = a;
      }
      v[j] = a;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = c0 + 1024 * j + 4 * tid;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c + e < V && v[j][e] > best) {  // ascending columns: strict > keeps the first
          best = v[j][e];
          bi = c + e;
        }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    argmax_merge(best, bi, ov, oi);
  }
  if ((tid & 63) == 0) {
    sv[tid >> 6] = best;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) argmax_merge(best, bi, sv[w], si[w]);
    out[r] = (uint32_t)(bi == 0x7fffffff ? 0 : bi);
    if (pos) pos[r] += 1;
  }
}

// Decode step input: x = w_tok[tok] + w_pos[pos] (kv_cache.rs:103-115), lens =
// pos + 1, and y = LN(x) with the first block's γ/β — the embedding and the
// first LayerNorm in one launch.  One block per row, d % 4 == 0, d <= 4096.
__global__ void __launch_bounds__(256) embed_ln_kernel(const float* __restrict__ w_tok,
                                                       const float* __restrict__ w_pos,
                                                       const uint32_t* __restrict__ tok,
                                                       const int32_t* __restrict__ pos_dev,
                                                       float* __restrict__ xo, const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, float* __restrict__ y,
                                                       int32_t* __restrict__ lens, int d, float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  floatx4 gg[4], bb[4];  // requested before the dependent row loads
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (threadIdx.x + 256 * i) * 4;
    if (c < d) {
      gg[i] = *reinterpret_cast<const floatx4*>(gamma + c);
      bb[i] = *reinterpret_cast<const floatx4*>(beta + c);
    }
  }
  const int p = pos_dev[r];
  if (lens && threadIdx.x == 0) lens[r] = p + 1;
  const float* a = w_tok + (size_t)tok[r] * d;
  const float* b = w_pos + (size_t)p * d;
  floatx4 xv[4];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (threadIdx.x + 256 * i) * 4;
    floatx4 v = {0.f, 0.f, 0.f, 0.f};
    if (c < d) {
      v = *reinterpret_cast<const floatx4*>(a + c) + *reinterpret_cast<const floatx4*>(b + c);
      *reinterpret_cast<floatx4*>(xo + (size_t)r * d + c) = v;
      s += (v[0] + v[1]) + (v[2] + v[3]);
    }
    xv[i] = v;
  }
  const float mu = block_sum(s, red) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (threadIdx.x + 256 * i) * 4;
    if (c < d)
#pragma unroll
      for (int e = 0; e < 4; ++e) q += (xv[i][e] - mu) * (xv[i][e] - mu);
  }
  const float is = 1.0f / sqrtf(block_sum(q, red) / (float)d + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (threadIdx.x + 256 * i) * 4;
    if (c < d) {
      floatx4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (xv[i][e] - mu) * is * gg[i][e] + bb[i][e];
      *reinterpret_cast<floatx4*>(y + (size_t)r * d + c) = o;
    }
  }
}

__global__ void gather_rows_kernel(const float* __restrict__ src, int ld_src, int row_step,
                                   int row_off, float* __restrict__ dst, int rows, int d) {
  const int r = blockIdx.x;
  if (r >= rows) return;
  const float* s = src + ((size_t)r * row_step + row_off) * ld_src;
  float* o = dst + (size_t)r * d;
  for (int c = threadIdx.x; c < d; c += 256) o[c] = s[c];
}

unsigned grid_1d(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 16384); }

}  // namespace

namespace aur {

#define LAUNCH_OK(ctx, name) AUR_LAUNCH_CHECK(ctx, name); return 0

int embed_forward(aur_ctx* ctx, const float* w_tok, const float* w_pos, const uint32_t* tok,
                  const int32_t* pos_dev, int T, float* out, int rows, int d, int32_t* lens) {
  hipLaunchKernelGGL(embed_fwd_kernel, dim3(rows), dim3(256), 0, ctx->stream, w_tok, w_pos, tok, pos_dev,
                     T, out, rows, d, lens);
  LAUNCH_OK(ctx, "embed_fwd_kernel");
}

int embed_backward(aur_ctx* ctx, const float* dy, int B, int T, int d, const uint32_t* tok_ids,
                   const int32_t* row_off, const int32_t* row_idx, int n_unique, float* g_w_tok,
                   float* g_w_pos) {
  if (n_unique > 0)
    hipLaunchKernelGGL(embed_tok_bwd_kernel, dim3(n_unique), dim3(256), 0, ctx->stream, dy, tok_ids,
                       row_off, row_idx, g_w_tok, d);
  hipLaunchKernelGGL(embed_pos_bwd_kernel, dim3(T), dim3(256), 0, ctx->stream, dy, B, T, g_w_pos, d);
  LAUNCH_OK(ctx, "embed_bwd kernels");
}

int layer_norm_forward(aur_ctx* ctx, const float* x, const float* gamma, const float* beta, float* y,
                       float* mean, float* rstd, int rows, int d, float eps) {
  const bool vec = d % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                                   reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta)) &
                                  15) == 0;
  const dim3 g4((rows + 3) / 4);
  if (rows < 1024 && vec)
    hipLaunchKernelGGL(ln_fwd_rowblock_kernel, dim3(rows), dim3(256), 0, ctx->stream, x, gamma, beta, y, mean,
                       rstd, d, eps);
  else if (vec && d == 256)
    hipLaunchKernelGGL(ln_fwd_vec_kernel<1>, g4, dim3(256), 0, ctx->stream, x, gamma, beta, y, mean, rstd, rows, eps);
  else if (vec && d == 512)
    hipLaunchKernelGGL(ln_fwd_vec_kernel<2>, g4, dim3(256), 0, ctx->stream, x, gamma, beta, y, mean, rstd, rows, eps);
  else if (vec && d == 1024)
    hipLaunchKernelGGL(ln_fwd_vec_kernel<4>, g4, dim3(256), 0, ctx->stream, x, gamma, beta, y, mean, rstd, rows, eps);
  else if (vec && d == 2048)
    hipLaunchKernelGGL(ln_fwd_vec_kernel<8>, g4, dim3(256), 0, ctx->stream, x, gamma, beta, y, mean, rstd, rows, eps);
  else
    hipLaunchKernelGGL(ln_fwd_kernel, g4, dim3(256), 0, ctx->stream, x, gamma, beta, y, mean, rstd, rows, d, eps);
  LAUNCH_OK(ctx, "ln_fwd_kernel");
}

int layer_norm_forward_sum(aur_ctx* ctx, const float* R, const float* P, int np, float* x_out,
                           const float* gamma, const float* beta, float* y, int rows, int d, float eps) {
  if (d % 4 != 0 || d > 4096 || np < 1)
    return set_error(ctx, AUR_EINVAL, "layer_norm_forward_sum: d=%d np=%d unsupported", d, np);
  hipLaunchKernelGGL(ln_fwd_sum_kernel, dim3(rows), dim3(256), 0, ctx->stream, R, P, np, (size_t)rows * d,
                     x_out, gamma, beta, y, d, eps);
  LAUNCH_OK(ctx, "ln_fwd_sum_kernel");
}

size_t layer_norm_backward_ws_floats(int rows, int d) {
  static_assert(LN_FCHUNK <= LN_CHUNK, "the fused kernel's chunks are the finer ones");
  return 2 * (size_t)((rows + LN_FCHUNK - 1) / LN_FCHUNK) * d;
}

int layer_norm_backward(aur_ctx* ctx, const float* x, const float* mean, const float* rstd,
                        const float* gamma, const float* dy, const float* dres, float* dx,
                        float* dgamma, float* dbeta, float* ws, int rows, int d) {
  const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma) |
                     reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(dres) |
                     reinterpret_cast<uintptr_t>(dx)) & 15) == 0;
  const bool fused = vec && (reinterpret_cast<uintptr_t>(ws) & 15) == 0 && rows > 0 &&
                     (d == 256 || d == 512 || d == 1024 || d == 2048) && getenv("AUR_LN_UNFUSED") == nullptr;
  if (fused) {
    const int nch = (rows + LN_FCHUNK - 1) / LN_FCHUNK;
    float* pg = ws;
    float* pb = ws + (size_t)nch * d;
    const dim3 gc(nch);
    if (d == 256)
      hipLaunchKernelGGL(ln_bwd_fused_kernel<1>, gc, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, pg, pb, rows);
    else if (d == 512)
      hipLaunchKernelGGL(ln_bwd_fused_kernel<2>, gc, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, pg, pb, rows);
    else if (d == 1024)
      hipLaunchKernelGGL(ln_bwd_fused_kernel<4>, gc, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, pg, pb, rows);
    else
      hipLaunchKernelGGL(ln_bwd_fused_kernel<8>, gc, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, pg, pb, rows);
    hipLaunchKernelGGL(ln_param_final_kernel, dim3((d + 3) / 4), dim3(256), 0, ctx->stream, pg, pb, nch,
                       dgamma, dbeta, d);
    LAUNCH_OK(ctx, "ln_bwd_fused kernels");
  }
  const dim3 g4((rows + 3) / 4);
  if (vec && d == 256)
    hipLaunchKernelGGL(ln_bwd_vec_kernel<1>, g4, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, rows);
  else if (vec && d == 512)
    hipLaunchKernelGGL(ln_bwd_vec_kernel<2>, g4, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, rows);
  else if (vec && d == 1024)
    hipLaunchKernelGGL(ln_bwd_vec_kernel<4>, g4, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, rows);
  else if (vec && d == 2048)
    hipLaunchKernelGGL(ln_bwd_vec_kernel<8>, g4, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, rows);
  else
    hipLaunchKernelGGL(ln_bwd_kernel, g4, dim3(256), 0, ctx->stream, x, mean, rstd, gamma, dy, dres, dx, rows, d);
  const int nch = (rows + LN_CHUNK - 1) / LN_CHUNK;
  float* pg = ws;
  float* pb = ws + (size_t)nch * d;
  hipLaunchKernelGGL(ln_param_partial_kernel, dim3((d + 255) / 256, nch), dim3(256), 0, ctx->stream, x,
                     mean, rstd, dy, pg, pb, rows, d);
  hipLaunchKernelGGL(ln_param_final_kernel, dim3((d + 3) / 4), dim3(256), 0, ctx->stream, pg, pb, nch,
                     dgamma, dbeta, d);
  LAUNCH_OK(ctx, "ln_bwd kernels");
}

int softmax_ce(aur_ctx* ctx, float* logits, const uint32_t* targets, float* nll, int rows, int V,
               float scale) {
  const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && V % 1024 == 0;
  switch (vec ? V / 1024 : 0) {
    case 1: hipLaunchKernelGGL(softmax_ce_vec_kernel<1>, dim3(rows), dim3(256), 0, ctx->stream, logits, targets, nll, scale); break;
    case 2: hipLaunchKernelGGL(softmax_ce_vec_kernel<2>, dim3(rows), dim3(256), 0, ctx->stream, logits, targets, nll, scale); break;
    case 4: hipLaunchKernelGGL(softmax_ce_vec_kernel<4>, dim3(rows), dim3(256), 0, ctx->stream, logits, targets, nll, scale); break;
    case 8: hipLaunchKernelGGL(softmax_ce_vec_kernel<8>, dim3(rows), dim3(256), 0, ctx->stream, logits, targets, nll, scale); break;
    case 16: hipLaunchKernelGGL(softmax_ce_vec_kernel<16>, dim3(rows), dim3(256), 0, ctx->stream, logits, targets, nll, scale); break;
    default:
      hipLaunchKernelGGL(softmax_ce_kernel, dim3(rows), dim3(256), 0, ctx->stream, logits, targets, nll, V,
                         scale);
  }
  LAUNCH_OK(ctx, "softmax_ce_kernel");
}

constexpr int kNormParts = 1024;

int grad_norm(aur_ctx* ctx, const float* g, size_t n, float max_norm, float* part, float* stats) {
  hipLaunchKernelGGL(sumsq_partial_kernel, dim3(kNormParts), dim3(256), 0, ctx->stream, g, n, part);
  hipLaunchKernelGGL(norm_final_kernel, dim3(1), dim3(256), 0, ctx->stream, part, kNormParts, max_norm,
                     stats, 0);
  LAUNCH_OK(ctx, "grad norm kernels");
}

int grad_norm2(aur_ctx* ctx, const float* g1, size_t n1, const float* g2, size_t n2, float max_norm,
               float* part, float* stats) {
  hipLaunchKernelGGL(sumsq_partial_kernel, dim3(kNormParts / 2), dim3(256), 0, ctx->stream, g1, n1, part);
  hipLaunchKernelGGL(sumsq_partial_kernel, dim3(kNormParts / 2), dim3(256), 0, ctx->stream, g2, n2,
                     part + kNormParts / 2);
  hipLaunchKernelGGL(norm_final_kernel, dim3(1), dim3(256), 0, ctx->stream, part, kNormParts, max_norm,
                     stats, 0);
  LAUNCH_OK(ctx, "grad norm kernels");
}

int frob_inv(aur_ctx* ctx, const float* x, size_t n, float* part, float* stats) {
  hipLaunchKernelGGL(sumsq_partial_kernel, dim3(kNormParts), dim3(256), 0, ctx->stream, x, n, part);
  hipLaunchKernelGGL(norm_final_kernel, dim3(1), dim3(256), 0, ctx->stream, part, kNormParts, 0.f, stats,
                     1);
  LAUNCH_OK(ctx, "frobenius kernels");
}

size_t grad_norm_ws_floats() { return kNormParts; }

int muon_momentum(aur_ctx* ctx, const float* g, float* m, float* upd, size_t n, float beta, bool nesterov) {
  hipLaunchKernelGGL(muon_momentum_kernel, dim3(grid_1d(n)), dim3(256), 0, ctx->stream, g, m, upd, n, beta,
                     nesterov ? 1 : 0);
  LAUNCH_OK(ctx, "muon_momentum_kernel");
}

int ns_combine(aur_ctx* ctx, float* out, const float* A, const float* A2, float a, float b, float c, int m,
               int nb) {
  const size_t n = (size_t)nb * m * m;
  hipLaunchKernelGGL(ns_combine_kernel, dim3(grid_1d(n)), dim3(256), 0, ctx->stream, out, A, A2, a, b, c,
                     (size_t)m, n);
  LAUNCH_OK(ctx, "ns_combine_kernel");
}

int transpose(aur_ctx* ctx, const float* src, float* dst, int rows, int cols) {
  hipLaunchKernelGGL(transpose_kernel, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(256), 0, ctx->stream,
                     src, dst, rows, cols);
  LAUNCH_OK(ctx, "transpose_kernel");
}

int muon_apply(aur_ctx* ctx, float* p, const float* upd, size_t n, float lr_scale, float lr_wd) {
  hipLaunchKernelGGL(muon_apply_kernel, dim3(grid_1d(n)), dim3(256), 0, ctx->stream, p, upd, n, lr_scale,
                     lr_wd);
  LAUNCH_OK(ctx, "muon_apply_kernel");
}

int scale_by(aur_ctx* ctx, float* x, size_t n, const float* factor) {
  hipLaunchKernelGGL(scale_kernel, dim3(grid_1d(n)), dim3(256), 0, ctx->stream, x, n, factor);
  LAUNCH_OK(ctx, "scale_kernel");
}

int adamw(aur_ctx* ctx, float* p, const float* g, float* m1, float* m2, size_t n, size_t n_decay,
          const float* clip, float lr, float b1, float b2, float eps, float wd, float bc1, float bc2) {
  hipLaunchKernelGGL(adamw_kernel, dim3(grid_1d(n)), dim3(256), 0, ctx->stream, p, g, m1, m2, n, n_decay,
                     clip, lr, b1, b2, eps, wd, bc1, bc2);
  LAUNCH_OK(ctx, "adamw_kernel");
}

int kv_store(aur_ctx* ctx, const float* qkv, int d, float* kh, float* vh, int max_len,
             const int32_t* pos_dev, int rows, int T) {
  hipLaunchKernelGGL(kv_store_kernel, dim3(rows), dim3(256), 0, ctx->stream, qkv, d, kh, vh, max_len,
                     pos_dev, T);
  LAUNCH_OK(ctx, "kv_store_kernel");
}

int argmax_rows(aur_ctx* ctx, const float* logits, int rows, int V, uint32_t* out, int32_t* pos) {
  if (V % 4 == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0) {
    hipLaunchKernelGGL(argmax_sum_kernel, dim3(rows), dim3(256), 0, ctx->stream, logits, 1, (size_t)0,
                       const_cast<float*>(logits), V, out, pos);
    LAUNCH_OK(ctx, "argmax_sum_kernel");
  }
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, ctx->stream, logits, V, out, pos);
  LAUNCH_OK(ctx, "argmax_kernel");
}

int embed_layer_norm(aur_ctx* ctx, const float* w_tok, const float* w_pos, const uint32_t* tok,
                     const int32_t* pos_dev, float* x_out, const float* gamma, const float* beta, float* y,
                     int32_t* lens, int rows, int d, float eps) {
  if (d % 4 != 0 || d > 4096 || !pos_dev)
    return set_error(ctx, AUR_EINVAL, "embed_layer_norm: d=%d unsupported", d);
  hipLaunchKernelGGL(embed_ln_kernel, dim3(rows), dim3(256), 0, ctx->stream, w_tok, w_pos, tok, pos_dev, x_out,
                     gamma, beta, y, lens, d, eps);
  LAUNCH_OK(ctx, "embed_ln_kernel");
}

int gather_rows(aur_ctx* ctx, const float* src, int ld_src, int row_step, int row_off, float* dst,
                int rows, int d) {
  hipLaunchKernelGGL(gather_rows_kernel, dim3(rows), dim3(256), 0, ctx->stream, src, ld_src, row_step,
                     row_off, dst, rows, d);
  LAUNCH_OK(ctx, "gather_rows_kernel");
}

}  // namespace aur
