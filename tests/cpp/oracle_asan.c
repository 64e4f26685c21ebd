/* Memory-safety driver for the CPU oracle (oracle/oracle.c), built with
 * AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_oracle_sanitized.py.
 * Every buffer is its own exact-size allocation, so a read or write past the
 * size a function's contract gives (the sizes oracle/__init__.py allocates)
 * is reported.  Shapes are small and ragged on purpose: t not a multiple of
 * the 8-row blocks, d not a multiple of the 8-lane dot, one-row and one-head
 * cases, causal and non-causal attention. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

float ora_dot(const float* a, const float* b, size_t n);
void ora_cpu_gemm(const float* a, const float* b, float* c, size_t m, size_t k, size_t n);
void ora_cpu_gemm_transpose_b(const float* a, const float* b, float* c, size_t m, size_t k, size_t n);
void ora_linear_forward_rows(const float* w, const float* x, float* y, size_t r0, size_t r1, size_t d_in,
                             size_t d_out);
void ora_linear_forward(const float* w, const float* x, float* y, size_t t, size_t d_in, size_t d_out);
void ora_linear_backward(const float* w, const float* x, const float* dy, float* dx, float* d_w, size_t t,
                         size_t d_in, size_t d_out);
void ora_outer_accum(const float* x, const float* d_y, float* dest, size_t d_out, size_t d_in, size_t t);
void ora_tied_head_forward(const float* h, const float* w_tok, float* logits, size_t t, size_t vocab, size_t d);
void ora_lm_head_backward(const float* h, const float* w, const float* d_logits, float* d_h, float* d_w,
                          size_t t, size_t vocab, size_t d);
void ora_sdpa_forward(const float* q, const float* k, const float* v, float* out, float* probs, size_t t_q,
                      size_t t_k, size_t d_k, size_t d_v, int causal);
void ora_sdpa_backward(const float* q, const float* k, const float* v, const float* probs, const float* d_out,
                       float* dq, float* dk, float* dv, float* d_probs, float* d_scores, size_t t_q, size_t t_k,
                       size_t d_k, size_t d_v);
void ora_mha_heads_forward(const float* q, const float* k, const float* v, float* heads_out, float* probs,
                           float* scratch, size_t t, size_t n_head, size_t d_head);
void ora_mha_heads_backward(const float* q, const float* k, const float* v, const float* probs,
                            const float* d_heads_out, float* dq, float* dk, float* dv, float* scratch, size_t t,
                            size_t n_head, size_t d_head);
void ora_layer_norm_forward(const float* gamma, const float* beta, float eps, const float* x, float* y,
                            float* mean, float* inv_std, float* x_hat, size_t t, size_t d);
void ora_layer_norm_backward(const float* gamma, const float* inv_std, const float* x_hat, const float* dy,
                             float* dx, float* d_gamma, float* d_beta, size_t t, size_t d);
void ora_gelu(const float* x, float* y, size_t n);
void ora_gelu_backward(const float* x, float* dydx, size_t n);
float ora_softmax_ce(const float* logits, const uint32_t* targets, float* d_logits, size_t t, size_t v);
void ora_token_nll(const float* logits, const uint32_t* targets, float* nll, size_t t, size_t v);
void ora_embed_forward(const float* w_tok, const float* w_pos, const uint32_t* tokens, float* out, size_t t,
                       size_t d);
void ora_embed_backward(const uint32_t* tokens, const float* dy, float* d_w_tok, float* d_w_pos, size_t t,
                        size_t d);
void ora_adamw_apply(float* params, const float* grads, float* m1, float* m2, size_t n, float lr, float beta1,
                     float beta2, float eps, float weight_decay, float bc1, float bc2, int apply_wd);
void ora_bias_correction(int t, float beta1, float beta2, float* bc1, float* bc2);
void ora_newton_schulz5(float* g, size_t rows, size_t cols, float* scratch, int n_iter);
void ora_muon_apply(float* params, const float* grads, float* mom, size_t rows, size_t cols, float lr,
                    float momentum, int nesterov, float weight_decay, int ns_steps, float* scratch);
float ora_sumsq_acc(const float* x, size_t n, float s);
void ora_scale(float* x, size_t n, float f);
void ora_add_assign(float* dst, const float* src, size_t n);
void ora_kv_attend(const float* q_new, const float* k_hist, const float* v_hist, float* heads_out, float* scores,
                   size_t t_total, size_t n_head, size_t d_head);
void ora_linear_forward_seqs(const float* w, const float* x, float* y, size_t rows, size_t rows_per_seq,
                             size_t d_in, size_t d_out, int nthreads);

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static float urand(void) { /* SplitMix64 → U(-1, 1) */
  uint64_t z = (rng_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  z ^= z >> 31;
  return (float)((z >> 40) * (1.0 / 16777216.0)) * 2.f - 1.f;
}
static float* fbuf(size_t n) {
  float* p = malloc((n ? n : 1) * sizeof(float));
  for (size_t i = 0; i < n; ++i) p[i] = urand();
  return p;
}
static uint32_t* ubuf(size_t n, uint32_t bound) {
  uint32_t* p = malloc((n ? n : 1) * sizeof(uint32_t));
  for (size_t i = 0; i < n; ++i) p[i] = (uint32_t)((urand() + 1.f) * 0.5f * bound) % bound;
  return p;
}
static int failures = 0;
static void expect(int ok, const char* what) {
  if (!ok) {
    printf("FAIL %s\n", what);
    ++failures;
  }
}

static void gemms(size_t m, size_t k, size_t n) {
  float *a = fbuf(m * k), *b = fbuf(k * n), *bt = fbuf(n * k), *c = fbuf(m * n);
  ora_cpu_gemm(a, b, c, m, k, n);
  ora_cpu_gemm_transpose_b(a, bt, c, m, k, n);
  expect(isfinite(ora_dot(a, a, m * k)), "dot");
  free(a); free(b); free(bt); free(c);
}

static void linears(size_t t, size_t d_in, size_t d_out) {
  float *w = fbuf(d_out * d_in), *x = fbuf(t * d_in), *y = fbuf(t * d_out), *dy = fbuf(t * d_out);
  float *dx = fbuf(t * d_in), *dw = fbuf(d_out * d_in), *dest = fbuf(d_out * d_in);
  ora_linear_forward(w, x, y, t, d_in, d_out);
  ora_linear_forward_rows(w, x, y, t / 2, t, d_in, d_out);
  ora_linear_backward(w, x, dy, dx, dw, t, d_in, d_out);
  ora_outer_accum(x, dy, dest, d_out, d_in, t);
  ora_linear_forward_seqs(w, x, y, t, 3, d_in, d_out, 2);
  free(w); free(x); free(y); free(dy); free(dx); free(dw); free(dest);
}

static void heads(size_t t, size_t vocab, size_t d) {
  float *h = fbuf(t * d), *w = fbuf(vocab * d), *lg = fbuf(t * vocab), *dh = fbuf(t * d), *dw = fbuf(vocab * d);
  float *dl = fbuf(t * vocab), *nll = fbuf(t);
  uint32_t* tg = ubuf(t, (uint32_t)vocab);
  ora_tied_head_forward(h, w, lg, t, vocab, d);
  const float loss = ora_softmax_ce(lg, tg, dl, t, vocab);
  expect(isfinite(loss) && loss > 0.f, "softmax_ce loss");
  for (size_t r = 0; r < t; ++r) { /* each row of the CE gradient sums to 0 */
    double s = 0.0;
    for (size_t j = 0; j < vocab; ++j) s += dl[r * vocab + j];
    expect(fabs(s) < 1e-4, "softmax_ce gradient row sum");
  }
  ora_token_nll(lg, tg, nll, t, vocab);
  ora_lm_head_backward(h, w, dl, dh, dw, t, vocab, d);
  free(h); free(w); free(lg); free(dh); free(dw); free(dl); free(nll); free(tg);
}

static void sdpa(size_t t_q, size_t t_k, size_t d_k, size_t d_v, int causal) {
  float *q = fbuf(t_q * d_k), *k = fbuf(t_k * d_k), *v = fbuf(t_k * d_v), *out = fbuf(t_q * d_v);
  float *probs = fbuf(t_q * t_k), *dout = fbuf(t_q * d_v), *dq = fbuf(t_q * d_k), *dk = fbuf(t_k * d_k);
  float *dv = fbuf(t_k * d_v), *s1 = fbuf(t_q * t_k), *s2 = fbuf(t_q * t_k);
  ora_sdpa_forward(q, k, v, out, probs, t_q, t_k, d_k, d_v, causal);
  for (size_t i = 0; i < t_q; ++i) { /* probability rows sum to one */
    double s = 0.0;
    for (size_t j = 0; j < t_k; ++j) s += probs[i * t_k + j];
    expect(fabs(s - 1.0) < 1e-5, "sdpa probability row sum");
  }
  ora_sdpa_backward(q, k, v, probs, dout, dq, dk, dv, s1, s2, t_q, t_k, d_k, d_v);
  free(q); free(k); free(v); free(out); free(probs); free(dout); free(dq); free(dk); free(dv); free(s1);
  free(s2);
}

static void mha(size_t t, size_t n_head, size_t d_head) {
  const size_t d = n_head * d_head;
  float *q = fbuf(t * d), *k = fbuf(t * d), *v = fbuf(t * d), *out = fbuf(t * d);
  float *probs = fbuf(n_head * t * t), *sc = fbuf(4 * t * d_head), *dout = fbuf(t * d);
  float *dq = fbuf(t * d), *dk = fbuf(t * d), *dv = fbuf(t * d), *sc2 = fbuf(7 * t * d_head + 2 * t * t);
  float *qn = fbuf(d), *ho = fbuf(d), *scores = fbuf(t);
  ora_mha_heads_forward(q, k, v, out, probs, sc, t, n_head, d_head);
  ora_mha_heads_backward(q, k, v, probs, dout, dq, dk, dv, sc2, t, n_head, d_head);
  ora_kv_attend(qn, k, v, ho, scores, t, n_head, d_head);
  free(q); free(k); free(v); free(out); free(probs); free(sc); free(dout); free(dq); free(dk); free(dv);
  free(sc2); free(qn); free(ho); free(scores);
}

static void norms(size_t t, size_t d) {
  float *g = fbuf(d), *b = fbuf(d), *x = fbuf(t * d), *y = fbuf(t * d), *mean = fbuf(t), *istd = fbuf(t);
  float *xh = fbuf(t * d), *dy = fbuf(t * d), *dx = fbuf(t * d), *dg = fbuf(d), *db = fbuf(d);
  ora_layer_norm_forward(g, b, 1e-5f, x, y, mean, istd, xh, t, d);
  ora_layer_norm_backward(g, istd, xh, dy, dx, dg, db, t, d);
  ora_gelu(x, y, t * d);
  ora_gelu_backward(x, dx, t * d);
  free(g); free(b); free(x); free(y); free(mean); free(istd); free(xh); free(dy); free(dx); free(dg); free(db);
}

static void embeds(size_t t, size_t vocab, size_t t_max, size_t d) {
  float *wt = fbuf(vocab * d), *wp = fbuf(t_max * d), *out = fbuf(t * d), *dy = fbuf(t * d);
  float *dwt = fbuf(vocab * d), *dwp = fbuf(t_max * d);
  uint32_t* tok = ubuf(t, (uint32_t)vocab);
  ora_embed_forward(wt, wp, tok, out, t, d);
  ora_embed_backward(tok, dy, dwt, dwp, t, d);
  free(wt); free(wp); free(out); free(dy); free(dwt); free(dwp); free(tok);
}

static void optim(size_t rows, size_t cols) {
  const size_t n = rows * cols, m = rows < cols ? rows : cols, mx = rows < cols ? cols : rows;
  float *p = fbuf(n), *g = fbuf(n), *m1 = fbuf(n), *m2 = fbuf(n), *mom = fbuf(n);
  for (size_t i = 0; i < n; ++i) m2[i] = fabsf(m2[i]);
  float bc1 = 0.f, bc2 = 0.f;
  ora_bias_correction(3, 0.9f, 0.95f, &bc1, &bc2);
  ora_adamw_apply(p, g, m1, m2, n, 1e-3f, 0.9f, 0.95f, 1e-8f, 0.1f, bc1, bc2, 1);
  float *gg = fbuf(n), *s1 = fbuf(2 * m * m + 2 * m * mx), *s2 = fbuf(n + 2 * m * m + 2 * m * mx);
  ora_newton_schulz5(gg, rows, cols, s1, 5);
  ora_muon_apply(p, g, mom, rows, cols, 0.02f, 0.95f, 1, 0.1f, 5, s2);
  expect(isfinite(ora_sumsq_acc(p, n, 0.f)), "sumsq");
  ora_scale(p, n, 0.5f);
  ora_add_assign(p, g, n);
  free(p); free(g); free(m1); free(m2); free(mom); free(gg); free(s1); free(s2);
}

int main(void) {
  gemms(1, 1, 1);
  gemms(5, 7, 3);
  gemms(17, 13, 9);
  linears(1, 4, 3);
  linears(11, 13, 9);
  linears(16, 8, 24);
  heads(1, 5, 4);
  heads(9, 37, 12);
  sdpa(1, 1, 4, 4, 1);
  sdpa(7, 7, 5, 3, 1);
  sdpa(5, 9, 4, 6, 0);
  mha(1, 1, 8);
  mha(13, 3, 8);
  mha(70, 2, 16);
  norms(1, 4);
  norms(9, 20);
  embeds(1, 3, 1, 4);
  embeds(12, 7, 12, 8);
  optim(1, 1);
  optim(6, 10);
  optim(10, 6);
  if (failures) {
    printf("%d checks failed\n", failures);
    return 1;
  }
  printf("OK oracle under ASan/UBSan\n");
  return 0;
}
