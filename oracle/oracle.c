/*
 * oracle.c — CPU restatement of the reference's CPU path for the GEMM /
 * causal-attention hot path.  TEST INFRASTRUCTURE ONLY: it is the checker
 * that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * compare libaurora_hip.so against.  Nothing in the product links it.
 *
 * The reference (danielkrul97/aurora) is Rust; no Rust toolchain exists in
 * this environment, so each function below restates one reference function
 * in C with the same loop order and fp32 summation structure, citing the
 * file:line it follows.  Compiled with -O3 -ffp-contract=off so a*b+c stays
 * two roundings where the Rust code writes `+=` (Rust does not contract),
 * and fmaf() is used exactly where the Rust code calls mul_add.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define LINEAR_BLOCK_T 8 /* src/attention.rs:214 */
#define HEAD_BLOCK_T 8   /* src/transformer/embedding.rs:148 */
#define NEG_INF_MASK (-1.0e30f) /* src/attention.rs:26 */

/* linalg::dot — src/linalg.rs:49-67: 8 fused accumulators, pairwise tree,
 * sequential remainder. */
float ora_dot(const float* a, const float* b, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t full = n / 8 * 8;
  for (size_t i = 0; i < full; i += 8)
    for (int j = 0; j < 8; ++j) acc[j] = fmaf(a[i + j], b[i + j], acc[j]);
  float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  for (size_t i = full; i < n; ++i) s += a[i] * b[i];
  return s;
}

/* cpu_gemm — src/gpu/matmul.rs:413-425: C[m,n] = A[m,k]·B[k,n], sequential k. */
void ora_cpu_gemm(const float* a, const float* b, float* c, size_t m, size_t k, size_t n) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (size_t kk = 0; kk < k; ++kk) acc += a[i * k + kk] * b[kk * n + j];
      c[i * n + j] = acc;
    }
}

/* cpu_gemm_transpose_b — src/gpu/matmul.rs:429-441: C = A[m,k]·B[n,k]ᵀ. */
void ora_cpu_gemm_transpose_b(const float* a, const float* b, float* c, size_t m, size_t k,
                              size_t n) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (size_t kk = 0; kk < k; ++kk) acc += a[i * k + kk] * b[j * k + kk];
      c[i * n + j] = acc;
    }
}

/* linear_forward — src/attention.rs:219-238: y[t,o] = dot(W[o,:], x[t,:]),
 * positions in blocks of LINEAR_BLOCK_T, weight row outer. Rows [r0, r1). */
void ora_linear_forward_rows(const float* w, const float* x, float* y, size_t r0, size_t r1,
                             size_t d_in, size_t d_out) {
  size_t t0 = r0;
  while (t0 < r1) {
    size_t tb = (r1 - t0) < LINEAR_BLOCK_T ? (r1 - t0) : LINEAR_BLOCK_T;
    for (size_t o = 0; o < d_out; ++o) {
      const float* row = w + o * d_in;
      for (size_t tt = 0; tt < tb; ++tt) {
        size_t i = t0 + tt;
        y[i * d_out + o] = ora_dot(row, x + i * d_in, d_in);
      }
    }
    t0 += tb;
  }
}

void ora_linear_forward(const float* w, const float* x, float* y, size_t t, size_t d_in,
                        size_t d_out) {
  ora_linear_forward_rows(w, x, y, 0, t, d_in, d_out);
}

/* linear_backward — src/attention.rs:241-274: dx = dy·W (dx zeroed here, as
 * the Rust returns a fresh vec), d_w += dyᵀ·x, one pass, same loop order. */
void ora_linear_backward(const float* w, const float* x, const float* dy, float* dx, float* d_w,
                         size_t t, size_t d_in, size_t d_out) {
  memset(dx, 0, sizeof(float) * t * d_in);
  size_t t0 = 0;
  while (t0 < t) {
    size_t tb = (t - t0) < LINEAR_BLOCK_T ? (t - t0) : LINEAR_BLOCK_T;
    for (size_t o = 0; o < d_out; ++o) {
      const float* row = w + o * d_in;
      float* drow = d_w + o * d_in;
      for (size_t tt = 0; tt < tb; ++tt) {
        size_t i = t0 + tt;
        float g = dy[i * d_out + o];
        const float* xr = x + i * d_in;
        float* dxr = dx + i * d_in;
        for (size_t kk = 0; kk < d_in; ++kk) {
          drow[kk] += g * xr[kk];
          dxr[kk] += g * row[kk];
        }
      }
    }
    t0 += tb;
  }
}

/* OUTER_ACCUM_WGSL — src/gpu/reduce.rs:15-115: acc = Σ_t dY[t,o]·X[t,i]
 * accumulated in t order from zero, then one read-modify-write dest += acc. */
void ora_outer_accum(const float* x, const float* d_y, float* dest, size_t d_out, size_t d_in,
                     size_t t) {
  for (size_t o = 0; o < d_out; ++o)
    for (size_t i = 0; i < d_in; ++i) {
      float acc = 0.0f;
      for (size_t tt = 0; tt < t; ++tt) acc += d_y[tt * d_out + o] * x[tt * d_in + i];
      dest[o * d_in + i] = dest[o * d_in + i] + acc;
    }
}

/* tied_lm_head_forward — src/transformer/embedding.rs:152-169. */
void ora_tied_head_forward(const float* h, const float* w_tok, float* logits, size_t t,
                           size_t vocab, size_t d) {
  size_t t0 = 0;
  while (t0 < t) {
    size_t tb = (t - t0) < HEAD_BLOCK_T ? (t - t0) : HEAD_BLOCK_T;
    for (size_t v = 0; v < vocab; ++v) {
      const float* wr = w_tok + v * d;
      for (size_t tt = 0; tt < tb; ++tt) {
        size_t ti = t0 + tt;
        logits[ti * vocab + v] = ora_dot(h + ti * d, wr, d);
      }
    }
    t0 += tb;
  }
}

/* lm_head_backward — src/transformer/embedding.rs:175-206: d_h returned
 * fresh (zeroed here), d_w accumulated. */
void ora_lm_head_backward(const float* h, const float* w, const float* d_logits, float* d_h,
                          float* d_w, size_t t, size_t vocab, size_t d) {
  memset(d_h, 0, sizeof(float) * t * d);
  size_t t0 = 0;
  while (t0 < t) {
    size_t tb = (t - t0) < HEAD_BLOCK_T ? (t - t0) : HEAD_BLOCK_T;
    for (size_t v = 0; v < vocab; ++v) {
      const float* wr = w + v * d;
      float* dwr = d_w + v * d;
      for (size_t tt = 0; tt < tb; ++tt) {
        size_t ti = t0 + tt;
        float g = d_logits[ti * vocab + v];
        const float* hr = h + ti * d;
        float* dhr = d_h + ti * d;
        for (size_t c = 0; c < d; ++c) {
          dwr[c] += g * hr[c];
          dhr[c] += g * wr[c];
        }
      }
    }
    t0 += tb;
  }
}

/* scaled_dot_product_attention — src/attention.rs:396-467 (single head).
 * probs [t_q, t_k] is written (the cache the backward consumes). */
void ora_sdpa_forward(const float* q, const float* k, const float* v, float* out, float* probs,
                      size_t t_q, size_t t_k, size_t d_k, size_t d_v, int causal) {
  float scale = 1.0f / sqrtf((float)d_k);
  for (size_t i = 0; i < t_q; ++i) {
    const float* qr = q + i * d_k;
    float row_max = -INFINITY;
    for (size_t j = 0; j < t_k; ++j) {
      const float* kr = k + j * d_k;
      float s = 0.0f;
      for (size_t c = 0; c < d_k; ++c) s += qr[c] * kr[c];
      s *= scale;
      if (causal && j > i) s = NEG_INF_MASK;
      probs[i * t_k + j] = s;
      if (s > row_max) row_max = s;
    }
    float sum = 0.0f;
    for (size_t j = 0; j < t_k; ++j) {
      float e = expf(probs[i * t_k + j] - row_max);
      probs[i * t_k + j] = e;
      sum += e;
    }
    float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (size_t j = 0; j < t_k; ++j) probs[i * t_k + j] *= inv;
  }
  memset(out, 0, sizeof(float) * t_q * d_v);
  for (size_t i = 0; i < t_q; ++i) {
    const float* pr = probs + i * t_k;
    float* orow = out + i * d_v;
    for (size_t j = 0; j < t_k; ++j) {
      float p = pr[j];
      if (p == 0.0f) continue;
      const float* vr = v + j * d_v;
      for (size_t c = 0; c < d_v; ++c) orow[c] += p * vr[c];
    }
  }
}

/* scaled_dot_product_attention_backward — src/attention.rs:474-550.
 * dq, dk, dv are written (fresh), d_probs/d_scores use caller scratch of
 * t_q*t_k floats each. */
void ora_sdpa_backward(const float* q, const float* k, const float* v, const float* probs,
                       const float* d_out, float* dq, float* dk, float* dv, float* d_probs,
                       float* d_scores, size_t t_q, size_t t_k, size_t d_k, size_t d_v) {
  float scale = 1.0f / sqrtf((float)d_k);
  memset(dv, 0, sizeof(float) * t_k * d_v);
  for (size_t i = 0; i < t_q; ++i) {
    const float* pr = probs + i * t_k;
    const float* dor = d_out + i * d_v;
    for (size_t j = 0; j < t_k; ++j) {
      float p = pr[j];
      if (p == 0.0f) continue;
      float* dvr = dv + j * d_v;
      for (size_t c = 0; c < d_v; ++c) dvr[c] += p * dor[c];
    }
  }
  for (size_t i = 0; i < t_q; ++i) {
    const float* dor = d_out + i * d_v;
    for (size_t j = 0; j < t_k; ++j) {
      const float* vr = v + j * d_v;
      float s = 0.0f;
      for (size_t c = 0; c < d_v; ++c) s += dor[c] * vr[c];
      d_probs[i * t_k + j] = s;
    }
  }
  for (size_t i = 0; i < t_q; ++i) {
    const float* pr = probs + i * t_k;
    const float* dpr = d_probs + i * t_k;
    float row_dot = 0.0f;
    for (size_t j = 0; j < t_k; ++j) row_dot += pr[j] * dpr[j];
    for (size_t j = 0; j < t_k; ++j) d_scores[i * t_k + j] = pr[j] * (dpr[j] - row_dot);
  }
  memset(dq, 0, sizeof(float) * t_q * d_k);
  memset(dk, 0, sizeof(float) * t_k * d_k);
  for (size_t i = 0; i < t_q; ++i) {
    const float* qr = q + i * d_k;
    float* dqr = dq + i * d_k;
    const float* dsr = d_scores + i * t_k;
    for (size_t j = 0; j < t_k; ++j) {
      float g = dsr[j] * scale;
      if (g == 0.0f) continue;
      const float* kr = k + j * d_k;
      float* dkr = dk + j * d_k;
      for (size_t c = 0; c < d_k; ++c) {
        dqr[c] += g * kr[c];
        dkr[c] += g * qr[c];
      }
    }
  }
}

/* causal_mha_forward's per-head part — src/transformer/attention.rs:142-190
 * (non-diff branch): gather head h of q/k/v [t, H·dh], SDPA, scatter into
 * heads_out.  probs [H, t, t]; scratch of 3·t·dh + t·dh floats. */
void ora_mha_heads_forward(const float* q, const float* k, const float* v, float* heads_out,
                           float* probs, float* scratch, size_t t, size_t n_head, size_t d_head) {
  size_t d = n_head * d_head;
  float* q_h = scratch;
  float* k_h = q_h + t * d_head;
  float* v_h = k_h + t * d_head;
  float* o_h = v_h + t * d_head;
  for (size_t h = 0; h < n_head; ++h) {
    for (size_t ti = 0; ti < t; ++ti) {
      memcpy(q_h + ti * d_head, q + ti * d + h * d_head, sizeof(float) * d_head);
      memcpy(k_h + ti * d_head, k + ti * d + h * d_head, sizeof(float) * d_head);
      memcpy(v_h + ti * d_head, v + ti * d + h * d_head, sizeof(float) * d_head);
    }
    ora_sdpa_forward(q_h, k_h, v_h, o_h, probs + h * t * t, t, t, d_head, d_head, 1);
    for (size_t ti = 0; ti < t; ++ti)
      memcpy(heads_out + ti * d + h * d_head, o_h + ti * d_head, sizeof(float) * d_head);
  }
}

/* causal_mha_backward's per-head part — src/transformer/attention.rs:235-300
 * (non-diff branch).  Writes dq/dk/dv [t, H·dh]; scratch of
 * 7·t·dh + 2·t·t floats. */
void ora_mha_heads_backward(const float* q, const float* k, const float* v, const float* probs,
                            const float* d_heads_out, float* dq, float* dk, float* dv,
                            float* scratch, size_t t, size_t n_head, size_t d_head) {
  size_t d = n_head * d_head;
  float* q_h = scratch;
  float* k_h = q_h + t * d_head;
  float* v_h = k_h + t * d_head;
  float* do_h = v_h + t * d_head;
  float* dq_h = do_h + t * d_head;
  float* dk_h = dq_h + t * d_head;
  float* dv_h = dk_h + t * d_head;
  float* d_probs = dv_h + t * d_head;
  float* d_scores = d_probs + t * t;
  for (size_t h = 0; h < n_head; ++h) {
    for (size_t ti = 0; ti < t; ++ti) {
      size_t src = ti * d + h * d_head, dst = ti * d_head;
      memcpy(q_h + dst, q + src, sizeof(float) * d_head);
      memcpy(k_h + dst, k + src, sizeof(float) * d_head);
      memcpy(v_h + dst, v + src, sizeof(float) * d_head);
      memcpy(do_h + dst, d_heads_out + src, sizeof(float) * d_head);
    }
    ora_sdpa_backward(q_h, k_h, v_h, probs + h * t * t, do_h, dq_h, dk_h, dv_h, d_probs, d_scores,
                      t, t, d_head, d_head);
    for (size_t ti = 0; ti < t; ++ti) {
      size_t dst = ti * d + h * d_head, src = ti * d_head;
      memcpy(dq + dst, dq_h + src, sizeof(float) * d_head);
      memcpy(dk + dst, dk_h + src, sizeof(float) * d_head);
      memcpy(dv + dst, dv_h + src, sizeof(float) * d_head);
    }
  }
}

/* layer_norm_forward — src/attention.rs:84-114 (LayerNorm mode, not RMS). */
void ora_layer_norm_forward(const float* gamma, const float* beta, float eps, const float* x,
                            float* y, float* mean, float* inv_std, float* x_hat, size_t t,
                            size_t d) {
  float inv_d = 1.0f / (float)d;
  for (size_t i = 0; i < t; ++i) {
    const float* row = x + i * d;
    float sum = 0.0f;
    for (size_t j = 0; j < d; ++j) sum += row[j];
    float mu = sum * inv_d;
    float var = 0.0f;
    for (size_t j = 0; j < d; ++j) {
      float dv = row[j] - mu;
      var += dv * dv;
    }
    var *= inv_d;
    float s = 1.0f / sqrtf(var + eps);
    mean[i] = mu;
    inv_std[i] = s;
    for (size_t j = 0; j < d; ++j) {
      float hh = (row[j] - mu) * s;
      x_hat[i * d + j] = hh;
      y[i * d + j] = hh * gamma[j] + beta[j];
    }
  }
}

/* layer_norm_backward — src/attention.rs:117-157 (LayerNorm mode): dx
 * written, d_gamma/d_beta accumulated. */
void ora_layer_norm_backward(const float* gamma, const float* inv_std, const float* x_hat,
                             const float* dy, float* dx, float* d_gamma, float* d_beta, size_t t,
                             size_t d) {
  float inv_d = 1.0f / (float)d;
  for (size_t i = 0; i < t; ++i) {
    size_t off = i * d;
    float s = inv_std[i];
    const float* xh = x_hat + off;
    const float* dyr = dy + off;
    float sum_dy_xh_gamma = 0.0f, sum_dy_gamma = 0.0f;
    for (size_t j = 0; j < d; ++j) {
      d_gamma[j] += dyr[j] * xh[j];
      d_beta[j] += dyr[j];
      float g = dyr[j] * gamma[j];
      sum_dy_gamma += g;
      sum_dy_xh_gamma += g * xh[j];
    }
    for (size_t j = 0; j < d; ++j) {
      float g = dyr[j] * gamma[j];
      dx[off + j] = s * (g - inv_d * (sum_dy_gamma + xh[j] * sum_dy_xh_gamma));
    }
  }
}

/* gelu / gelu_backward — src/linalg.rs:72-87 (tanh form), elementwise. */
void ora_gelu(const float* x, float* y, size_t n) {
  const float k = sqrtf(2.0f / 3.14159265358979323846f);
  for (size_t i = 0; i < n; ++i) {
    float xv = x[i];
    float inner = k * (xv + 0.044715f * xv * xv * xv);
    y[i] = 0.5f * xv * (1.0f + tanhf(inner));
  }
}

void ora_gelu_backward(const float* x, float* dydx, size_t n) {
  const float k = sqrtf(2.0f / 3.14159265358979323846f);
  for (size_t i = 0; i < n; ++i) {
    float xv = x[i];
    float inner = k * (xv + 0.044715f * xv * xv * xv);
    float th = tanhf(inner);
    float sech2 = 1.0f - th * th;
    float d_inner = k * (1.0f + 3.0f * 0.044715f * xv * xv);
    dydx[i] = 0.5f * (1.0f + th) + 0.5f * xv * sech2 * d_inner;
  }
}

/* Softmax-CE with the 1/T scale fused — src/transformer/model.rs:820-858
 * (softcap = 0, z_loss = 0).  Writes d_logits, returns Σ_t NLL (the caller
 * divides by t, model.rs:911). */
float ora_softmax_ce(const float* logits, const uint32_t* targets, float* d_logits, size_t t,
                     size_t v) {
  float total = 0.0f;
  float inv_t = 1.0f / (float)t;
  for (size_t ti = 0; ti < t; ++ti) {
    const float* row = logits + ti * v;
    float* drow = d_logits + ti * v;
    float mx = -INFINITY;
    for (size_t c = 0; c < v; ++c) mx = fmaxf(mx, row[c]);
    float sum = 0.0f;
    for (size_t c = 0; c < v; ++c) {
      float e = expf(row[c] - mx);
      drow[c] = e;
      sum += e;
    }
    float inv_sum = 1.0f / sum;
    size_t tgt = targets[ti];
    float pt = drow[tgt] * inv_sum;
    if (pt < 1e-12f) pt = 1e-12f;
    total += -logf(pt);
    for (size_t c = 0; c < v; ++c) {
      float g = drow[c] * inv_sum;
      if (c == tgt) g -= 1.0f;
      drow[c] = g * inv_t;
    }
  }
  return total;
}

/* Per-token NLL in nats without a gradient: the loss_seq row the GPU
 * softmax-CE writes, -ln(max(p_target, 1e-12)) (src/gpu/softmax_ce.rs:101-102;
 * the CPU eval's logsumexp form, examples/aurora_train.rs:1713-1719, is the
 * same quantity with the clamp at ln 1e-12 = -27.631021). */
void ora_token_nll(const float* logits, const uint32_t* targets, float* nll, size_t t, size_t v) {
  for (size_t ti = 0; ti < t; ++ti) {
    const float* row = logits + ti * v;
    float mx = -INFINITY;
    for (size_t c = 0; c < v; ++c) mx = fmaxf(mx, row[c]);
    float sum = 0.0f;
    for (size_t c = 0; c < v; ++c) sum += expf(row[c] - mx);
    float pt = expf(row[targets[ti]] - mx) / sum;
    if (pt < 1e-12f) pt = 1e-12f;
    nll[ti] = -logf(pt);
  }
}

/* embed_forward / embed_backward — src/transformer/embedding.rs:95-142. */
void ora_embed_forward(const float* w_tok, const float* w_pos, const uint32_t* tokens, float* out,
                       size_t t, size_t d) {
  for (size_t ti = 0; ti < t; ++ti) {
    const float* tr = w_tok + (size_t)tokens[ti] * d;
    const float* pr = w_pos + ti * d;
    for (size_t c = 0; c < d; ++c) out[ti * d + c] = tr[c] + pr[c];
  }
}

void ora_embed_backward(const uint32_t* tokens, const float* dy, float* d_w_tok, float* d_w_pos,
                        size_t t, size_t d) {
  for (size_t ti = 0; ti < t; ++ti) {
    float* tr = d_w_tok + (size_t)tokens[ti] * d;
    float* pr = d_w_pos + ti * d;
    const float* dr = dy + ti * d;
    for (size_t c = 0; c < d; ++c) tr[c] += dr[c];
    for (size_t c = 0; c < d; ++c) pr[c] += dr[c];
  }
}

/* adamw_apply — src/optimizer.rs:58-83; bias_correction :86-90 (powi). */
void ora_adamw_apply(float* params, const float* grads, float* m1, float* m2, size_t n, float lr,
                     float beta1, float beta2, float eps, float weight_decay, float bc1, float bc2,
                     int apply_wd) {
  float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2;
  for (size_t i = 0; i < n; ++i) {
    float g = grads[i];
    m1[i] = beta1 * m1[i] + omb1 * g;
    m2[i] = beta2 * m2[i] + omb2 * g * g;
    float m1h = m1[i] / bc1;
    float m2h = m2[i] / bc2;
    float step = lr * m1h / (sqrtf(m2h) + eps);
    if (apply_wd) step += lr * weight_decay * params[i];
    params[i] -= step;
  }
}

static float powi_f(float b, int e) {
  float r = 1.0f;
  for (int i = 0; i < e; ++i) r *= b;
  return r;
}

void ora_bias_correction(int t, float beta1, float beta2, float* bc1, float* bc2) {
  *bc1 = 1.0f - powi_f(beta1, t);
  *bc2 = 1.0f - powi_f(beta2, t);
}

/* newton_schulz5 — src/optimizer.rs:147-252: Frobenius bound (skip when
 * ‖g‖² <= 1e-30), wide orientation [m × n] (physical transpose when
 * rows > cols), n_iter quintic steps A = X·Xᵀ (upper triangle, mirrored),
 * B = c·A·A + b·A, X' = a·X + B·X, each sum sequential in k; then back.
 * scratch: 2·m·m + 2·m·n floats. */
void ora_newton_schulz5(float* g, size_t rows, size_t cols, float* scratch, int n_iter) {
  size_t m = rows < cols ? rows : cols, n = rows < cols ? cols : rows;
  float frob_sq = 0.0f;
  for (size_t i = 0; i < rows * cols; ++i) frob_sq += g[i] * g[i];
  if (frob_sq <= 1e-30f) return;
  float inv_scale = 1.0f / (sqrtf(frob_sq) + 1e-7f);
  for (size_t i = 0; i < rows * cols; ++i) g[i] *= inv_scale;
  float* a_buf = scratch;
  float* b_buf = a_buf + m * m;
  float* buf_x = b_buf + m * m;
  float* buf_y = buf_x + m * n;
  int transposed = rows > cols;
  if (transposed) {
    for (size_t r = 0; r < rows; ++r)
      for (size_t c = 0; c < cols; ++c) buf_x[c * rows + r] = g[r * cols + c];
  } else {
    memcpy(buf_x, g, sizeof(float) * m * n);
  }
  const float a_coef = 3.4445f, b_coef = -4.7750f, c_coef = 2.0315f;
  float* cur = buf_x;
  float* nxt = buf_y;
  for (int it = 0; it < n_iter; ++it) {
    for (size_t i = 0; i < m; ++i)
      for (size_t j = i; j < m; ++j) {
        float s = 0.0f;
        for (size_t k = 0; k < n; ++k) s += cur[i * n + k] * cur[j * n + k];
        a_buf[i * m + j] = s;
        if (i != j) a_buf[j * m + i] = s;
      }
    for (size_t i = 0; i < m; ++i)
      for (size_t j = 0; j < m; ++j) {
        float s = 0.0f;
        for (size_t k = 0; k < m; ++k) s += a_buf[i * m + k] * a_buf[k * m + j];
        b_buf[i * m + j] = c_coef * s + b_coef * a_buf[i * m + j];
      }
    for (size_t i = 0; i < m; ++i)
      for (size_t j = 0; j < n; ++j) {
        float s = 0.0f;
        for (size_t k = 0; k < m; ++k) s += b_buf[i * m + k] * cur[k * n + j];
        nxt[i * n + j] = a_coef * cur[i * n + j] + s;
      }
    float* t = cur;
    cur = nxt;
    nxt = t;
  }
  if (transposed) {
    for (size_t r = 0; r < rows; ++r)
      for (size_t c = 0; c < cols; ++c) g[r * cols + c] = cur[c * rows + r];
  } else {
    memcpy(g, cur, sizeof(float) * m * n);
  }
}

/* muon_apply — src/optimizer.rs:259-305: momentum (Nesterov lookahead),
 * newton_schulz5, spectral scale √(max/min), decoupled decay.
 * scratch: rows·cols + 2·m·m + 2·m·n floats. */
void ora_muon_apply(float* params, const float* grads, float* mom, size_t rows, size_t cols, float lr,
                    float momentum, int nesterov, float weight_decay, int ns_steps, float* scratch) {
  size_t n_el = rows * cols;
  float* update = scratch;
  for (size_t i = 0; i < n_el; ++i) {
    mom[i] = momentum * mom[i] + grads[i];
    update[i] = nesterov ? grads[i] + momentum * mom[i] : mom[i];
  }
  ora_newton_schulz5(update, rows, cols, scratch + n_el, ns_steps);
  size_t m = rows < cols ? rows : cols, n = rows < cols ? cols : rows;
  float scale = sqrtf((float)n / (float)m);
  for (size_t i = 0; i < n_el; ++i) {
    float step = lr * scale * update[i];
    if (weight_decay > 0.0f) step += lr * weight_decay * params[i];
    params[i] -= step;
  }
}

/* ModelGrads::l2_norm's per-tensor term — src/transformer/model.rs:442-500:
 * one fp32 accumulator s += v·v carried across tensors in a fixed order. */
float ora_sumsq_acc(const float* x, size_t n, float s) {
  for (size_t i = 0; i < n; ++i) s += x[i] * x[i];
  return s;
}

void ora_scale(float* x, size_t n, float f) {
  for (size_t i = 0; i < n; ++i) x[i] *= f;
}

void ora_add_assign(float* dst, const float* src, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] += src[i];
}

/* block_step's attention — src/transformer/kv_cache.rs:181-219: one query
 * (q_new [H·dh]) against history rows [0, t_total) of k/v [*, d]. */
void ora_kv_attend(const float* q_new, const float* k_hist, const float* v_hist, float* heads_out,
                   float* scores, size_t t_total, size_t n_head, size_t d_head) {
  size_t d = n_head * d_head;
  float scale = 1.0f / sqrtf((float)d_head);
  memset(heads_out, 0, sizeof(float) * d);
  for (size_t h = 0; h < n_head; ++h) {
    size_t off = h * d_head;
    const float* qh = q_new + off;
    float row_max = -INFINITY;
    for (size_t j = 0; j < t_total; ++j) {
      const float* kr = k_hist + j * d + off;
      float s = 0.0f;
      for (size_t c = 0; c < d_head; ++c) s += qh[c] * kr[c];
      s *= scale;
      scores[j] = s;
      if (s > row_max) row_max = s;
    }
    float sum = 0.0f;
    for (size_t j = 0; j < t_total; ++j) {
      scores[j] = expf(scores[j] - row_max);
      sum += scores[j];
    }
    float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (size_t j = 0; j < t_total; ++j) scores[j] *= inv;
    for (size_t j = 0; j < t_total; ++j) {
      float p = scores[j];
      if (p == 0.0f) continue;
      const float* vr = v_hist + j * d + off;
      for (size_t c = 0; c < d_head; ++c) heads_out[off + c] += p * vr[c];
    }
  }
}

/* The reference's CPU training path runs linear_forward once per sequence,
 * sequences spread over a rayon pool (examples/aurora_train.rs:828-838).
 * This runs the same per-sequence linear_forward over `rows/rows_per_seq`
 * sequences on `nthreads` OpenMP threads (the CPU-baseline timing leg). */
#include <omp.h>
void ora_linear_forward_seqs(const float* w, const float* x, float* y, size_t rows,
                             size_t rows_per_seq, size_t d_in, size_t d_out, int nthreads) {
  long nseq = (long)((rows + rows_per_seq - 1) / rows_per_seq);
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (long s = 0; s < nseq; ++s) {
    size_t r0 = (size_t)s * rows_per_seq;
    size_t r1 = r0 + rows_per_seq < rows ? r0 + rows_per_seq : rows;
    ora_linear_forward_rows(w, x, y, r0, r1, d_in, d_out);
  }
}
